// Batch-1 decode GEMV for Q5_K x Q8_K: production_mul_mat_q5_k_decode /
// production_mul_mat_q5_k at M = 1 (examples/kernels/mul_mat/q5_k_decode.py,
// q5_k.py:9-37), rows of up to 4096 values.
//
// Semantics (ggml_vec_dot_q5_K_q8_K_generic, ggml-cpu/quants.c:720-798):
//   y = sum_b dx_b * (dw_b * S_b - dmin_b * Mn_b)
//   S  = sum_s sc_s * sum_{32} q5 * x,   q5 = nibble | qh bit << 4 in [0, 31]    (exact)
//   Mn = sum_s m_s * (bsum_{2s} + bsum_{2s+1})                                  (exact)
//
// gfx950 mapping, as the Q4_K batch-1 kernel: lane l of a row owns
// superblock l / 4 and its 64-element chunk g = l % 4 (sub-blocks 2g, 2g+1):
// the 16-byte header, the superblock's 32 qh bytes and the chunk's 32 qs
// bytes come straight into VGPRs as five 16-byte loads (a 176-byte record is
// 16-byte aligned when the matrix is), the 64 activation values and their
// two pair sums are read from LDS into VGPRs once.  Values are formed four
// at a time (nibble | qh bit << 4) and meet the activation in
// v_dot4_i32_i8; 6-bit scales and mins multiply exact 24-bit integers; one
// fp32 term per superblock and lane, a DPP wave sum per row.  A wave walks
// its rows with one row of lookahead.  The activation is quantized in every
// workgroup (bit-exact with quantize_row_q8_K_ref); workgroup 0 writes Xq.
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

struct Q5Args {
  const uint8_t* W;
  const float* X;
  uint8_t* xq_out;
  float* Y;
  int N, K;
  int rows_per_wg;
  size_t ldw;
};

__global__ void __launch_bounds__(kThreads) q5k_gemv_m1_kernel(Q5Args a) {
  extern __shared__ __align__(16) char lds[];  // Q8_K activation row
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int K = a.K;
  const int nsb = K >> 8;  // <= 16
  const bool live = lane < 4 * nsb;
  const int sb = min(lane >> 2, nsb - 1), g = lane & 3;
  const uint32_t off = (uint32_t)(kQ5_KBytes * sb);  // 16-byte aligned
  const size_t rb = a.ldw;
  const int row_first = blockIdx.x * a.rows_per_wg + wave;
  const int row_end = min(a.N, blockIdx.x * a.rows_per_wg + a.rows_per_wg);
  const int nrows = row_first < row_end ? (row_end - row_first + kWaves - 1) / kWaves : 0;

  // activation loads first: waiting for them does not wait for the weights
  Q8KStager16<1> stager;
  stager.prefetch(a.X, (size_t)K, K, 0, 1);
  __builtin_amdgcn_sched_barrier(0);

  struct RowBuf {
    uint4 h, qh0, qh1, q0, q1;
  };
  auto issue = [&](RowBuf& buf, int k) {
    const int row = min(row_first + k * kWaves, a.N - 1);  // clamped: always a valid row
    const uint8_t* rec = a.W + (size_t)row * rb + off;
    buf.h = *reinterpret_cast<const uint4*>(rec);
    buf.qh0 = *reinterpret_cast<const uint4*>(rec + 16);
    buf.qh1 = *reinterpret_cast<const uint4*>(rec + 32);
    buf.q0 = *reinterpret_cast<const uint4*>(rec + 48 + 32 * g);
    buf.q1 = *reinterpret_cast<const uint4*>(rec + 64 + 32 * g);
  };
  RowBuf bufA, bufB;
  issue(bufA, 0);
  __builtin_amdgcn_sched_barrier(0);

  stager.finish(a.X, (size_t)K, blockIdx.x == 0 ? a.xq_out : nullptr, K, 0, 1, lds);
  __syncthreads();

  // this lane's activation: sub-block 2g (xl0, xl1) and 2g + 1 (xh0, xh1)
  int4 xl0, xl1, xh0, xh1;
  float dx;
  int bp0, bp1;
  {
    const Q8KView v = q8k_view(lds, K, 0);
    const int8_t* xb = v.qs + 256 * sb + 64 * g;
    xl0 = *reinterpret_cast<const int4*>(xb);
    xl1 = *reinterpret_cast<const int4*>(xb + 16);
    xh0 = *reinterpret_cast<const int4*>(xb + 32);
    xh1 = *reinterpret_cast<const int4*>(xb + 48);
    dx = v.d[sb];
    const int2 bp = *reinterpret_cast<const int2*>(v.bp + 8 * sb + 2 * g);
    bp0 = bp.x;
    bp1 = bp.y;
  }
  const int xlo[8] = {xl0.x, xl0.y, xl0.z, xl0.w, xl1.x, xl1.y, xl1.z, xl1.w};
  const int xhi[8] = {xh0.x, xh0.y, xh0.z, xh0.w, xh1.x, xh1.y, xh1.z, xh1.w};

  auto compute = [&](const RowBuf& buf, int k) {
    const uint4 h = buf.h;
    int sc_lo, m_lo, sc_hi, m_hi;
    q4k_scale_min(2 * g, h.y, h.z, h.w, sc_lo, m_lo);
    q4k_scale_min(2 * g + 1, h.y, h.z, h.w, sc_hi, m_hi);
    const uint32_t qs[8] = {buf.q0.x, buf.q0.y, buf.q0.z, buf.q0.w, buf.q1.x, buf.q1.y, buf.q1.z, buf.q1.w};
    const uint32_t qh[8] = {buf.qh0.x, buf.qh0.y, buf.qh0.z, buf.qh0.w,
                            buf.qh1.x, buf.qh1.y, buf.qh1.z, buf.qh1.w};
    int pl = 0, ph = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t hb = qh[i] >> (2 * g);  // bit 2g: sub-block 2g, bit 2g + 1: 2g + 1
      const uint32_t lo = (qs[i] & 0x0f0f0f0fu) | ((hb & 0x01010101u) << 4);
      const uint32_t hi = ((qs[i] >> 4) & 0x0f0f0f0fu) | ((hb & 0x02020202u) << 3);
      pl = dot4((int)lo, xlo[i], pl);
      ph = dot4((int)hi, xhi[i], ph);
    }
    // |pl|, |ph| <= 32 * 31 * 128 and scales <= 63: 24-bit multiplies are exact
    const int S = __mul24(sc_lo, pl) + __mul24(sc_hi, ph);
    const int Mn = __mul24(m_lo, bp0) + __mul24(m_hi, bp1);
    const float dw = fp16_to_fp32(h.x & 0xffffu), dmin = fp16_to_fp32(h.x >> 16);
    const float t = dx * (dw * (float)S - dmin * (float)Mn);
    // lanes past the row's last superblock duplicate it: they add exactly 0
    const float tot = wave_sum_f(live ? t : 0.f);
    if (lane == 0) a.Y[row_first + k * kWaves] = tot;
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
// K <= 4096, 16-byte aligned X and W with rows a multiple of 16 bytes apart,
// Xq 4-byte aligned.
bool decode_q5k_m1(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                   const RowStrides& st) {
  const size_t rb = K / 256 * kQ5_KBytes;
  const size_t ldw = N > 1 ? st.ldw : rb;
  if (N == 0 || K == 0 || K > 4096 || K % 256 != 0 || X == nullptr || Xq == nullptr || W == nullptr ||
      Y == nullptr || !aligned(X, 16) || !aligned(W, 16) || ldw % 16 != 0 || !aligned(Y, 4) ||
      !aligned(Xq, 4) || N > (size_t)INT32_MAX || (N > 1 && ldw < rb) || ldw >= ((size_t)1 << 40))
    return false;
  // one workgroup per CU (79 VGPRs: a second one would not be resident;
  // measured 8.7 us for two per CU against 7.95 us at 11008 x 4096)
  const int cus = cu_count();
  const size_t wgs = std::max<size_t>(1, std::min<size_t>((size_t)cus, (N + kWaves - 1) / kWaves));
  Q5Args a;
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
  q5k_gemv_m1_kernel<<<grid, kThreads, q8k_lds_row_bytes((int)K), current_stream()>>>(a);
  check_launch("q5k_gemv_m1_kernel");
  return true;
}

}  // namespace weft
