// Q4_K x Q8_K prefill GEMM on int8 MFMA (production_mul_mat_q4_k_staged,
// production_mul_mat_q4_k; examples/kernels/mul_mat/q4_k_staged.py:9-37).
//
//   Y[m, n] = sum_b dx[m,b] * (dw[n,b] * S[m,n,b] - dmin[n,b] * Mn[m,n,b])
//   S  = sum_s sc[n,b,s] * sum_{k in s} q8[m,k] * q4[n,k]     (exact int32)
//   Mn = sum_s m[n,b,s]  * sum_{k in s} q8[m,k]                (exact int32)
//
// The 6-bit sub-block scale sc does not fit an int8 operand once multiplied
// by a nibble (sc*q <= 945), and applying it per sub-block on VALU costs one
// instruction per output per 32 products -- twice the MFMA time.  So the
// scale is split, sc = 8a + b with a, b in [0, 7], and every product stays an
// exact int8 x int8 MFMA term: three accumulators per output over each
// superblock,
//   lo = sum_k q8 * (q * b_s),  hi = sum_k q8 * (q * a_s),  mn = sum_k q8 * m_s,
// so S = lo + 8 hi and Mn = mn exactly, and the fp32 combine happens once per
// superblock.  v_mfma_i32_32x32x32_i8 has K = 32 = one sub-block, so the
// weight operand of a sub-block is its nibbles times a per-column constant
// (v_pk_mul_lo_u16 on packed bytes: 105 * 256 + 105 < 2^16, no carries).
//
// Tiling: a workgroup computes a 64 (tokens) x 128 (weight rows) tile with
// four waves, each 64 x 32 = two 32x32 MFMA tiles sharing one weight operand.
// Per superblock the quantized activation tile (64 x 256 int8, padded rows)
// and the raw Q4_K weight tile (128 x 144 B) are staged in LDS; the next
// superblock's global loads are issued before the current one is computed.
// The activation is quantized first, into the caller's Xq, by q8_K_quantize's
// kernel (Xq is part of the ABI), then read back from L2.
#include <algorithm>

#include "kernels.h"
#include "runtime.h"
#include "weft_common.h"
#include "weft_hip.h"

namespace weft {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));

constexpr int kMT = 64;          // tokens per workgroup tile
constexpr int kNT = 128;         // weight rows per workgroup tile
constexpr int kThreads = 256;
constexpr int kAStride = 272;    // LDS bytes per activation row (256 + 16 pad)
constexpr int kALoads = kMT * 256 / 16 / kThreads;       // 16-byte loads per thread: 4
constexpr int kWChunks = kNT * kQ4_KBytes / 16;           // 1152
constexpr int kWLoads = (kWChunks + kThreads - 1) / kThreads;  // 5

struct GemmArgs {
  const uint8_t* W;
  const uint8_t* Xq;
  float* Y;
  int N, K, M;
};

__device__ __forceinline__ uint32_t mul_bytes(uint32_t packed, uint32_t c) {
  // four bytes (each <= 15) times c (<= 7): no byte overflows into the next
  v2u16 v = __builtin_bit_cast(v2u16, packed);
  v2u16 r = v * (v2u16){(unsigned short)c, (unsigned short)c};
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ v4u ldg16_a4(const uint8_t* p) {
  // 16 bytes at a 4-byte aligned address
  const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
  return (v4u){q[0], q[1], q[2], q[3]};
}

__global__ void __launch_bounds__(kThreads, 2) q4k_mfma_gemm(GemmArgs a) {
  __shared__ __align__(16) int8_t As[kMT * kAStride];
  __shared__ __align__(16) float Dx[kMT];
  __shared__ __align__(16) uint8_t Ws[kNT * kQ4_KBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int col = lane & 31, kg = lane >> 5;
  const int m0 = blockIdx.y * kMT, n0 = blockIdx.x * kNT;
  const int nsb = a.K >> 8;
  const size_t wrb = (size_t)nsb * kQ4_KBytes;   // bytes per weight row
  const size_t xrb = (size_t)nsb * kQ8_KBytes;   // bytes per activation row

  // Per-thread staging sources (superblock 0) and LDS destinations: the
  // activation tile is 64 rows x 16 chunks of 16 B, the weight tile 1152
  // chunks; superblock b adds b * record size.
  const uint8_t* asrc[kALoads];
  int adst[kALoads];
#pragma unroll
  for (int i = 0; i < kALoads; ++i) {
    const int c = tid + i * kThreads;
    const int row = c >> 4, part = c & 15;
    asrc[i] = a.Xq + (size_t)min(m0 + row, a.M - 1) * xrb + 4 + 16 * part;
    adst[i] = row * kAStride + 16 * part;
  }
  const uint8_t* dsrc = a.Xq + (size_t)min(m0 + (tid & (kMT - 1)), a.M - 1) * xrb;
  const uint8_t* wsrc[kWLoads];
#pragma unroll
  for (int i = 0; i < kWLoads; ++i) {
    const int c = min(tid + i * kThreads, kWChunks - 1);
    const int row = c / 9, part = c - 9 * row;
    wsrc[i] = a.W + (size_t)min(n0 + row, a.N - 1) * wrb + 16 * part;
  }
  const bool w_last = tid + (kWLoads - 1) * kThreads < kWChunks;

  v4u ar[kALoads], wr[kWLoads];
  float dxr;
#define WEFT_FETCH(b)                                                                   \
  do {                                                                                  \
    const size_t ao = (size_t)(b) * kQ8_KBytes, wo = (size_t)(b) * kQ4_KBytes;          \
    _Pragma("unroll") for (int i = 0; i < kALoads; ++i) ar[i] = ldg16_a4(asrc[i] + ao); \
    dxr = *reinterpret_cast<const float*>(dsrc + ao);                                   \
    _Pragma("unroll") for (int i = 0; i < kWLoads; ++i)                                 \
        wr[i] = *reinterpret_cast<const v4u*>(wsrc[i] + wo);                            \
  } while (0)

  v16i lo[2], hi[2], mn[2];
  float y[2][16];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) y[t][r] = 0.f;

  const v16i zero = {};
  WEFT_FETCH(0);
  for (int b = 0; b < nsb; ++b) {
    __syncthreads();  // the previous superblock's LDS reads are done
#pragma unroll
    for (int i = 0; i < kALoads; ++i) *reinterpret_cast<v4u*>(As + adst[i]) = ar[i];
    if (tid < kMT) Dx[tid] = dxr;
#pragma unroll
    for (int i = 0; i < kWLoads - 1; ++i) *reinterpret_cast<v4u*>(Ws + 16 * (tid + i * kThreads)) = wr[i];
    if (w_last) *reinterpret_cast<v4u*>(Ws + 16 * (tid + (kWLoads - 1) * kThreads)) = wr[kWLoads - 1];
    __syncthreads();
    if (b + 1 < nsb) WEFT_FETCH(b + 1);  // in flight while this superblock computes

    // this lane's weight row (tile column) and its header
    const uint8_t* wrow = Ws + (32 * wave + col) * kQ4_KBytes;
    const uint4 h = *reinterpret_cast<const uint4*>(wrow);
    const uint32_t sc03 = h.y & 0x3f3f3f3fu;
    const uint32_t sc47 = (h.w & 0x0f0f0f0fu) | (((h.y >> 6) & 0x03030303u) << 4);
    const uint32_t mn03 = h.z & 0x3f3f3f3fu;
    const uint32_t mn47 = ((h.w >> 4) & 0x0f0f0f0fu) | (((h.z >> 6) & 0x03030303u) << 4);
    const float dw = fp16_to_fp32(h.x & 0xffffu);
    const float dmin = fp16_to_fp32(h.x >> 16);

#pragma unroll
    for (int g = 0; g < 4; ++g) {
      // 16 qs bytes: elements 64g + 16kg + i (low nibble) and 64g + 32 + 16kg + i (high)
      const uint4 q = *reinterpret_cast<const uint4*>(wrow + 16 + 32 * g + 16 * kg);
      const uint32_t scw = g < 2 ? sc03 : sc47;
      const uint32_t mnw = g < 2 ? mn03 : mn47;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int s = 2 * g + hf;
        const int sh = 8 * (s & 3);
        const uint32_t sc = (scw >> sh) & 0xffu, mm = (mnw >> sh) & 0xffu;
        const uint32_t n0w = hf ? (q.x >> 4) & 0x0f0f0f0fu : q.x & 0x0f0f0f0fu;
        const uint32_t n1w = hf ? (q.y >> 4) & 0x0f0f0f0fu : q.y & 0x0f0f0f0fu;
        const uint32_t n2w = hf ? (q.z >> 4) & 0x0f0f0f0fu : q.z & 0x0f0f0f0fu;
        const uint32_t n3w = hf ? (q.w >> 4) & 0x0f0f0f0fu : q.w & 0x0f0f0f0fu;
        const uint32_t cb = sc & 7u, ca = sc >> 3;
        const v4i b_lo = {(int)mul_bytes(n0w, cb), (int)mul_bytes(n1w, cb), (int)mul_bytes(n2w, cb),
                          (int)mul_bytes(n3w, cb)};
        const v4i b_hi = {(int)mul_bytes(n0w, ca), (int)mul_bytes(n1w, ca), (int)mul_bytes(n2w, ca),
                          (int)mul_bytes(n3w, ca)};
        const int mrep = (int)(mm * 0x01010101u);
        const v4i b_mn = {mrep, mrep, mrep, mrep};
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const v4i av = *reinterpret_cast<const v4i*>(As + (32 * t + col) * kAStride + 32 * s + 16 * kg);
          lo[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b_lo, s == 0 ? zero : lo[t], 0, 0, 0);
          hi[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b_hi, s == 0 ? zero : hi[t], 0, 0, 0);
          mn[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b_mn, s == 0 ? zero : mn[t], 0, 0, 0);
        }
      }
    }
    // fp32 combine of this superblock: D[i][j] lives in lane j (+32 for the
    // odd 4-row groups), register r holds row 8*(r/4) + 4*kg + r%4
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const float4 dx4 = *reinterpret_cast<const float4*>(Dx + 32 * t + 8 * r4 + 4 * kg);
        const float dxv[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = 4 * r4 + q;
          const int S = lo[t][r] + 8 * hi[t][r];
          y[t][r] += dxv[q] * (dw * (float)S - dmin * (float)mn[t][r]);
        }
      }
    }
  }
#undef WEFT_FETCH
  // store: for a fixed register the 32 lanes of a half cover 32 consecutive columns
  const int gn = n0 + 32 * wave + col;
  if (gn < a.N) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gm = m0 + 32 * t + 8 * (r >> 2) + 4 * kg + (r & 3);
        if (gm < a.M) a.Y[(size_t)gm * a.N + gn] = y[t][r];
      }
  }
}

void prefill_q4k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M) {
  if (N == 0 || M == 0 || K == 0) return;
  if (K % 256 || W == nullptr || X == nullptr || Xq == nullptr || Y == nullptr || !aligned(W, 16) ||
      !aligned(Xq, 4) || !aligned(Y, 4) || N > (size_t)INT32_MAX || K > (size_t)INT32_MAX ||
      M > (size_t)INT32_MAX) {
    set_error(hipErrorInvalidValue);
    return;
  }
  quantize_q8_k(X, Xq, M * K);
  GemmArgs a{W, Xq, Y, (int)N, (int)K, (int)M};
  dim3 grid((unsigned)((N + kNT - 1) / kNT), (unsigned)((M + kMT - 1) / kMT));
  q4k_mfma_gemm<<<grid, kThreads, 0, current_stream()>>>(a);
  check_launch();
}

}  // namespace

// Prefill entry: MFMA GEMM when the shape suits it, the decode GEMV otherwise.
void mul_mat_q4k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M) {
  if (M >= 16 && aligned(W, 16))
    prefill_q4k(W, X, Xq, Y, N, K, M);
  else
    decode_q4k(W, X, Xq, Y, N, K, M);
}

}  // namespace weft
