// Batch-1 decode GEMV for Q6_K x Q8_K: production_mul_mat_q6_k_decode /
// production_mul_mat_q6_k at M = 1 (examples/kernels/mul_mat/q6_k_decode.py,
// q6_k.py:9-37), rows of up to 4096 values.
//
// Semantics (ggml_vec_dot_q6_K_q8_K_generic, ggml-cpu/quants.c:800-853):
//   y = sum_b (dw_b dx_b) * sum_{j<16} sc_j * sum_{16} (q6 - 32) * x      (exact int32)
// computed as sum_j sc_j * (P_j - 32 X_j), P_j = sum q6 x with q6 in [0, 63]
// (an exact int8 operand) and X_j the 16 activation values' sum.
//
// gfx950 mapping, as the Q4_K / Q5_K batch-1 kernels: lane l of a row owns
// superblock l / 4 and its 64-element chunk g = l % 4 (half h = g / 2 of the
// record; the low nibbles of ql[64h .. 64h + 63] for even g, the high ones
// for odd g; qh[32h .. 32h + 31]; scales 4g .. 4g + 3).  A 210-byte record
// is 2-byte aligned for odd superblocks, so the lane's bytes come into VGPRs
// from the dword below them (16-byte loads at 4-byte aligned addresses) and
// are aligned with v_alignbyte.  The 64 activation values and their four
// 16-sums are held in VGPRs; values are formed four at a time and meet the
// activation in v_dot4_i32_i8.  One fp32 term per superblock and lane, a
// DPP wave sum per row, one row of lookahead.  The activation is quantized in
// every workgroup (bit-exact with quantize_row_q8_K_ref); workgroup 0 writes Xq.
#include <algorithm>

#include "activation.h"
#include "kernels.h"
#include "runtime.h"
#include "weft_common.h"
#include "weft_hip.h"

namespace weft {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;

struct Q6Args {
  const uint8_t* W;
  const float* X;
  uint8_t* xq_out;
  float* Y;
  int N, K;
  int rows_per_wg;
  size_t ldw;
};

__global__ void __launch_bounds__(kThreads) q6k_gemv_m1_kernel(Q6Args a) {
  extern __shared__ __align__(16) char lds[];  // Q8_K activation row
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int K = a.K;
  const int nsb = K >> 8;  // <= 16
  const bool live = lane < 4 * nsb;
  const int sb = min(lane >> 2, nsb - 1), g = lane & 3, h = g >> 1;
  const uint32_t rec = (uint32_t)(kQ6_KBytes * sb);
  const uint32_t sh = rec & 3u;   // 0 or 2
  const uint32_t base = rec - sh;  // dword holding the record's first byte
  // the lane's regions, relative to base: ql [sh + 64h, +64), qh
  // [sh + 128 + 32h, +32), scales [sh + 192 + 4g, +4), d [sh + 208, +2)
  const uint32_t o_ql = base + 64 * h, o_qh = base + 128 + 32 * h, o_sc = base + 192 + 4 * g;
  const uint32_t o_d = base + 208;
  const size_t rb = a.ldw;
  const int row_first = blockIdx.x * a.rows_per_wg + wave;
  const int row_end = min(a.N, blockIdx.x * a.rows_per_wg + a.rows_per_wg);
  const int nrows = row_first < row_end ? (row_end - row_first + kWaves - 1) / kWaves : 0;

  Q8KStager16<1> stager;
  stager.prefetch(a.X, (size_t)K, K, 0, 1);
  __builtin_amdgcn_sched_barrier(0);

  // 17 dwords of ql, 9 of qh, 2 of scales, 1 holding d.  A 17th / 9th /
  // 2nd dword only carries data at sh = 2; at sh = 0 the last dword before it
  // is read again (the region may end at the row's end).
  struct RowBuf {
    uint32_t ql[17], qh[9], sc[2], d;
  };
  auto issue = [&](RowBuf& buf, int k) {
    const int row = min(row_first + k * kWaves, a.N - 1);  // clamped: always a valid row
    const uint8_t* rp = a.W + (size_t)row * rb;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 v = *reinterpret_cast<const uint4*>(rp + o_ql + 16 * i);
      buf.ql[4 * i] = v.x, buf.ql[4 * i + 1] = v.y, buf.ql[4 * i + 2] = v.z, buf.ql[4 * i + 3] = v.w;
    }
    buf.ql[16] = *reinterpret_cast<const uint32_t*>(rp + o_ql + (sh ? 64 : 60));
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint4 v = *reinterpret_cast<const uint4*>(rp + o_qh + 16 * i);
      buf.qh[4 * i] = v.x, buf.qh[4 * i + 1] = v.y, buf.qh[4 * i + 2] = v.z, buf.qh[4 * i + 3] = v.w;
    }
    buf.qh[8] = *reinterpret_cast<const uint32_t*>(rp + o_qh + (sh ? 32 : 28));
    buf.sc[0] = *reinterpret_cast<const uint32_t*>(rp + o_sc);
    buf.sc[1] = *reinterpret_cast<const uint32_t*>(rp + o_sc + (sh ? 4 : 0));
    buf.d = *reinterpret_cast<const uint32_t*>(rp + o_d);
  };
  RowBuf bufA, bufB;
  issue(bufA, 0);
  __builtin_amdgcn_sched_barrier(0);

  stager.finish(a.X, (size_t)K, blockIdx.x == 0 ? a.xq_out : nullptr, K, 0, 1, lds);
  __syncthreads();

  // this lane's 64 activation values (part a: elements 0-31 of the chunk,
  // part b: 32-63) and the sums of its four 16-value groups
  int xa[8], xb[8];
  int xs[4];
  float dx;
  {
    const Q8KView v = q8k_view(lds, K, 0);
    const int8_t* x = v.qs + 256 * sb + 64 * g;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int4 p = *reinterpret_cast<const int4*>(x + 16 * i);
      const int4 q = *reinterpret_cast<const int4*>(x + 32 + 16 * i);
      xa[4 * i] = p.x, xa[4 * i + 1] = p.y, xa[4 * i + 2] = p.z, xa[4 * i + 3] = p.w;
      xb[4 * i] = q.x, xb[4 * i + 1] = q.y, xb[4 * i + 2] = q.z, xb[4 * i + 3] = q.w;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int* src = j < 2 ? xa + 4 * j : xb + 4 * (j - 2);
      int s = dot4(0x01010101, src[0], 0);
      s = dot4(0x01010101, src[1], s);
      s = dot4(0x01010101, src[2], s);
      xs[j] = dot4(0x01010101, src[3], s);
    }
    dx = v.d[sb];
  }
  const uint32_t nsh = 4 * (g & 1);        // nibble: low for even g, high for odd
  const uint32_t hsh = 4 * (g & 1);        // qh bit pairs 2s: s = 2 (g & 1) and 2 (g & 1) + 1

  auto compute = [&](const RowBuf& buf, int k) {
    uint32_t ql[16], qh[8];
#pragma unroll
    for (int i = 0; i < 16; ++i) ql[i] = __builtin_amdgcn_alignbyte(buf.ql[i + 1], buf.ql[i], sh);  // sh 0 or 2
#pragma unroll
    for (int i = 0; i < 8; ++i) qh[i] = __builtin_amdgcn_alignbyte(buf.qh[i + 1], buf.qh[i], sh);
    const uint32_t sc4 = __builtin_amdgcn_alignbyte(buf.sc[1], buf.sc[0], sh);
    const float dw = fp16_to_fp32((buf.d >> (8 * sh)) & 0xffffu);
    // part a: ql[0 .. 31] with qh bits hsh .. hsh + 1; part b: ql[32 .. 63]
    // with bits hsh + 2 .. hsh + 3 (element l of both parts reads qh[l])
    int P[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t hb = qh[i] >> hsh;
      const uint32_t va = ((ql[i] >> nsh) & 0x0f0f0f0fu) | ((hb & 0x03030303u) << 4);
      const uint32_t vb = ((ql[8 + i] >> nsh) & 0x0f0f0f0fu) | ((hb & 0x0c0c0c0cu) << 2);
      P[i >> 2] = dot4((int)va, xa[i], P[i >> 2]);
      P[2 + (i >> 2)] = dot4((int)vb, xb[i], P[2 + (i >> 2)]);
    }
    int tot = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int scj = (int)(int8_t)((sc4 >> (8 * j)) & 0xffu);
      tot += scj * (P[j] - 32 * xs[j]);  // |P - 32 X| <= 16 * 32 * 128: exact
    }
    const int bsum = sum4(live ? tot : 0);  // the superblock's four lanes
    const float t = (lane & 3) == 0 && live ? (dw * dx) * (float)bsum : 0.f;
    const float y = wave_sum_f(t);
    if (lane == 0) a.Y[row_first + k * kWaves] = y;
  };

  int k = 0;
  for (; k + 2 < nrows; k += 2) {
    issue(bufB, k + 1);
    compute(bufA, k);
    issue(bufA, k + 2);
    compute(bufB, k + 1);
  }
  if (nrows - k == 2) {
    issue(bufB, k + 1);
    compute(bufA, k);
    compute(bufB, k + 1);
  } else if (nrows - k == 1) {
    compute(bufA, k);
  }
}

}  // namespace

// Launches the kernel above when the call suits it: one activation row of
// K <= 4096 with an even superblock count (4-byte aligned rows), 16-byte
// aligned X, W 4-byte aligned with rows a multiple of 4 bytes apart, Xq
// 4-byte aligned.
bool decode_q6k_m1(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                   const RowStrides& st) {
  const size_t rb = K / 256 * kQ6_KBytes;
  const size_t ldw = N > 1 ? st.ldw : rb;
  if (N == 0 || K == 0 || K > 4096 || K % 512 != 0 || X == nullptr || Xq == nullptr || W == nullptr ||
      Y == nullptr || !aligned(X, 16) || !aligned(W, 4) || ldw % 4 != 0 || !aligned(Y, 4) ||
      !aligned(Xq, 4) || N > (size_t)INT32_MAX || (N > 1 && ldw < rb) || ldw >= ((size_t)1 << 40))
    return false;
  const int cus = cu_count();
  const size_t wgs = std::max<size_t>(1, std::min<size_t>((size_t)cus, (N + kWaves - 1) / kWaves));
  Q6Args a;
  a.W = W;
  a.X = X;
  a.xq_out = Xq;
  a.Y = Y;
  a.N = (int)N;
  a.K = (int)K;
  // a CompileOptions NC binding sets the weight rows per workgroup
  const int nc = tile_bindings().nc;
  a.rows_per_wg = nc > 0 ? (int)std::min<size_t>(N, (size_t)nc) : (int)((N + wgs - 1) / wgs);
  a.ldw = ldw;
  const int grid = (int)((N + a.rows_per_wg - 1) / a.rows_per_wg);
  q6k_gemv_m1_kernel<<<grid, kThreads, q8k_lds_row_bytes((int)K), current_stream()>>>(a);
  check_launch("q6k_gemv_m1_kernel");
  return true;
}

}  // namespace weft
