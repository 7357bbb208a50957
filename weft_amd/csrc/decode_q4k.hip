// Q4_K x Q8_K decode GEMV (production_mul_mat_q4_k_decode) and
// quantized_vec_dot_q4_k_q8_k.
//
// Semantics (examples/kernels/mul_mat/q4_k_decode.py:10-20,
// examples/kernels/vec_dot/q4_k_q8_k.py:8-36, GGML
// ggml_vec_dot_q4_K_q8_K_generic ggml-cpu/quants.c:645-718):
//   Y[m, n] = sum_b dx_b * (dw_b * S_b - dmin_b * Mn_b)
//   S_b  = sum_s sc_s * sum_{32 lanes of sub-block s} q4 * q8   (exact int32)
//   Mn_b = sum_s m_s * (bsum_{2s} + bsum_{2s+1})                 (exact int32)
//
// gfx950 mapping.  The kernel is HBM-bound: every weight byte is read once.
// A wave walks one weight row at a time.  Lane t of a 64-item step owns
// (superblock s = t/8, 16-byte qs chunk j = t%8): it issues one 16-byte load
// of its qs chunk and one 16-byte load of the superblock's header (d, dmin,
// 12 scale bytes; the 8 lanes of a superblock hit the same line), so each
// step reads 8 whole consecutive superblocks (1152 B) with 16-byte loads.
// The 32 nibbles of a chunk are two 16-element halves of sub-blocks 2g and
// 2g+1 (g = j/2); each half is dotted against the Q8_K activation held in
// LDS with four v_dot4_i32_i8, scaled by its 6-bit sub-block scale (unpacked
// in VGPRs), and converted to fp32 once per lane.  A row's lanes are summed
// with a wave reduction.
//
// The activation is quantized inside every workgroup (one wave per Q8_K
// superblock, bit-exact with quantize_row_q8_K_ref) so the whole mul_mat is
// one launch; workgroup 0 also stores the records into Xq.  The grid has
// about one workgroup per CU so that quantization is paid once per CU.
#include <algorithm>

#include "activation.h"
#include "kernels.h"
#include "runtime.h"
#include "weft_hip.h"

namespace weft {
namespace {

constexpr int kThreads = 1024;
constexpr int kMaxRowsPerPass = 4;  // activation rows staged per launch
constexpr int kChunk = 4;           // 64-item steps loaded before computing

struct Q4KArgs {
  const uint8_t* W;
  const float* X;        // fp32 activation (quantize path) or null
  const uint8_t* xq_in;  // quantized activation (vec_dot path) or null
  uint8_t* xq_out;       // Xq written by workgroup 0, or null
  float* Y;
  int N, K;
  int m0, mb;            // activation rows of this launch
  int rows_per_wg;
  long long y_stride;    // elements between output rows
};

template <bool A16>
__device__ __forceinline__ uint4 load16(const uint8_t* p) {
  if constexpr (A16) {
    return *reinterpret_cast<const uint4*>(p);
  } else {
    const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
    uint4 r;
    r.x = q[0] | ((uint32_t)q[1] << 16);
    r.y = q[2] | ((uint32_t)q[3] << 16);
    r.z = q[4] | ((uint32_t)q[5] << 16);
    r.w = q[6] | ((uint32_t)q[7] << 16);
    return r;
  }
}

template <bool A16>
__global__ void __launch_bounds__(kThreads) q4k_gemv_kernel(Q4KArgs a) {
  extern __shared__ __align__(16) char lds[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nwaves = blockDim.x / kWave;
  const int K = a.K;

  if (a.X != nullptr)
    stage_q8k_quantize(a.X, blockIdx.x == 0 ? a.xq_out : nullptr, K, a.m0, a.mb, lds);
  else
    stage_q8k_load(a.xq_in, K, a.m0, a.mb, lds);
  __syncthreads();

  const int nsb = K >> 8;
  const int items = nsb * 8;
  const size_t rb = (size_t)nsb * kQ4_KBytes;
  const int row0 = blockIdx.x * a.rows_per_wg;
  const int row1 = min(a.N, row0 + a.rows_per_wg);

  for (int row = row0 + wave; row < row1; row += nwaves) {
    const uint8_t* wr = a.W + (size_t)row * rb;
    float acc[kMaxRowsPerPass];
#pragma unroll
    for (int m = 0; m < kMaxRowsPerPass; ++m) acc[m] = 0.f;

    for (int t0 = 0; t0 < items; t0 += kWave * kChunk) {
      uint4 hdr[kChunk], qs[kChunk];
#pragma unroll
      for (int c = 0; c < kChunk; ++c) {
        const int t = t0 + kWave * c + lane;
        if (t < items) {
          const uint8_t* sb = wr + (size_t)(t >> 3) * kQ4_KBytes;
          hdr[c] = load16<A16>(sb);
          qs[c] = load16<A16>(sb + 16 + 16 * (t & 7));
        }
      }
#pragma unroll
      for (int c = 0; c < kChunk; ++c) {
        const int t = t0 + kWave * c + lane;
        if (t >= items) continue;
        const int s = t >> 3, j = t & 7, g = j >> 1, half = j & 1;
        int sc_lo, m_lo, sc_hi, m_hi;
        q4k_scale_min(2 * g, hdr[c].y, hdr[c].z, hdr[c].w, sc_lo, m_lo);
        q4k_scale_min(2 * g + 1, hdr[c].y, hdr[c].z, hdr[c].w, sc_hi, m_hi);
        const float dw = fp16_to_fp32(hdr[c].x & 0xffffu);
        const float dmin = fp16_to_fp32(hdr[c].x >> 16);
        const uint32_t q0 = qs[c].x, q1 = qs[c].y, q2 = qs[c].z, q3 = qs[c].w;
        const uint32_t l0 = q0 & 0x0f0f0f0fu, l1 = q1 & 0x0f0f0f0fu;
        const uint32_t l2 = q2 & 0x0f0f0f0fu, l3 = q3 & 0x0f0f0f0fu;
        const uint32_t h0 = (q0 >> 4) & 0x0f0f0f0fu, h1 = (q1 >> 4) & 0x0f0f0f0fu;
        const uint32_t h2 = (q2 >> 4) & 0x0f0f0f0fu, h3 = (q3 >> 4) & 0x0f0f0f0fu;
#pragma unroll
        for (int m = 0; m < kMaxRowsPerPass; ++m) {
          if (m >= a.mb) break;
          const Q8KView v = q8k_view(lds, K, m);
          const int8_t* xb = v.qs + 256 * s + 64 * g + 16 * half;
          const int4 xl = *reinterpret_cast<const int4*>(xb);
          const int4 xh = *reinterpret_cast<const int4*>(xb + 32);
          int pl = dot4((int)l0, xl.x, 0);
          pl = dot4((int)l1, xl.y, pl);
          pl = dot4((int)l2, xl.z, pl);
          pl = dot4((int)l3, xl.w, pl);
          int ph = dot4((int)h0, xh.x, 0);
          ph = dot4((int)h1, xh.y, ph);
          ph = dot4((int)h2, xh.z, ph);
          ph = dot4((int)h3, xh.w, ph);
          const int S = sc_lo * pl + sc_hi * ph;
          const int2 bp = *reinterpret_cast<const int2*>(v.bp + 8 * s + 2 * g);
          const int Mn = half ? 0 : m_lo * bp.x + m_hi * bp.y;
          const float dx = v.d[s];
          acc[m] += (dw * dx) * (float)S - (dmin * dx) * (float)Mn;
        }
      }
    }
#pragma unroll
    for (int m = 0; m < kMaxRowsPerPass; ++m) {
      if (m >= a.mb) break;
      const float tot = wave_sum(acc[m]);
      if (lane == 0) a.Y[(size_t)(a.m0 + m) * a.y_stride + row] = tot;
    }
  }
}

// Shared launcher: X != null -> quantize (and write Xq), else read xq_in.
void launch_q4k(const uint8_t* W, const float* X, const uint8_t* xq_in, uint8_t* xq_out, float* Y,
                size_t N, size_t K, size_t M) {
  if (N == 0 || M == 0 || K == 0) return;
  if (K % 256 != 0 || W == nullptr || Y == nullptr || (X == nullptr && xq_in == nullptr) ||
      N > (size_t)INT32_MAX || K > (size_t)INT32_MAX || M > (size_t)INT32_MAX ||
      !aligned(W, 2) || !aligned(Y, 4) || (xq_in && !aligned(xq_in, 4)) ||
      (xq_out && !aligned(xq_out, 4)) || (X && !aligned(X, 4))) {
    set_error(hipErrorInvalidValue);
    return;
  }
  const size_t row_lds = q8k_lds_row_bytes((int)K);
  const size_t lds_cap = max_lds_per_block();
  if (row_lds > lds_cap) {
    set_error(hipErrorInvalidValue);  // activation row does not fit in LDS
    return;
  }
  const int mb_max = (int)std::min<size_t>(kMaxRowsPerPass, lds_cap / row_lds);
  const int cus = cu_count();
  const int rows_per_wg = (int)((N + cus - 1) / cus);
  const int grid = (int)((N + rows_per_wg - 1) / rows_per_wg);
  const bool a16 = aligned(W, 16);
  for (size_t m0 = 0; m0 < M; m0 += mb_max) {
    Q4KArgs a;
    a.W = W;
    a.X = X;
    a.xq_in = xq_in;
    a.xq_out = xq_out;
    a.Y = Y;
    a.N = (int)N;
    a.K = (int)K;
    a.m0 = (int)m0;
    a.mb = (int)std::min<size_t>(mb_max, M - m0);
    a.rows_per_wg = rows_per_wg;
    a.y_stride = (long long)N;
    const size_t lds = row_lds * a.mb;
    if (a16)
      q4k_gemv_kernel<true><<<grid, kThreads, lds, current_stream()>>>(a);
    else
      q4k_gemv_kernel<false><<<grid, kThreads, lds, current_stream()>>>(a);
    check_launch();
  }
}

}  // namespace

void decode_q4k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                size_t M) {
  launch_q4k(W, X, nullptr, Xq, Y, N, K, M);
}

}  // namespace weft

extern "C" {

void production_mul_mat_q4_k_decode(const uint8_t* W, const float* X, uint8_t* Xq, float* Y,
                                    size_t N, size_t K, size_t M) {
  if (X == nullptr || Xq == nullptr) {
    weft::set_error(hipErrorInvalidValue);
    return;
  }
  weft::launch_q4k(W, X, nullptr, Xq, Y, N, K, M);
}

void quantized_vec_dot_q4_k_q8_k(const uint8_t* W, const uint8_t* X, float* Y, size_t K) {
  if (X == nullptr) {
    weft::set_error(hipErrorInvalidValue);
    return;
  }
  weft::launch_q4k(W, nullptr, X, nullptr, Y, 1, K, 1);
}

}  // extern "C"
