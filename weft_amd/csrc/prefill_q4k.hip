// Q4_K x Q8_K prefill GEMM on MFMA (production_mul_mat_q4_k_staged,
// production_mul_mat_q4_k; examples/kernels/mul_mat/q4_k_staged.py:9-37).
//
//   Y[m, n] = sum_b dx[m,b] * (dw[n,b] * S[m,n,b] - dmin[n,b] * Mn[m,n,b])
//   S  = sum_s sc[n,b,s] * sum_{k in s} q8[m,k] * q4[n,k]     (exact int32)
//   Mn = sum_s m[n,b,s]  * BS[m,b,s],  BS = Q8_K bsums[2s] + bsums[2s+1]
//
// S on int8 MFMA.  The 6-bit sub-block scale sc does not fit an int8 operand
// once multiplied by a nibble (sc*q <= 945), and applying it per sub-block on
// VALU costs one instruction per output per 32 products.  So the scale is
// split, sc = 8a + b with a, b in [0, 7], and every product stays an exact
// int8 x int8 term: two accumulators per output over each superblock,
//   lo = sum_k q8 * (q * b_s),   hi = sum_k q8 * (q * a_s),   S = lo + 8 hi,
// combined in fp32 once per superblock.  v_mfma_i32_32x32x32_i8 has K = 32 =
// one sub-block, so a sub-block's weight operand is its nibbles times a
// per-column constant (v_pk_mul_lo_u16 on packed bytes: 105*256+105 < 2^16).
//
// Mn on fp32 MFMA.  The min term is a GEMM over (superblock, sub-block) with
// operands A' = dx * BS (per token) and B' = -dmin * m (per weight row), so
// v_mfma_f32_32x32x2_f32 accumulates it straight into the fp32 outputs:
// 4 instructions per superblock and tile, no per-output combine.
//
// Tiling: a workgroup computes 64 (tokens) x 128 (weight rows) with 8 waves.
// Waves 0-3 take the even superblocks and waves 4-7 the odd ones; wave w owns
// weight rows 32*(w%4)..+31 for all 64 tokens (two 32x32 tiles sharing one
// weight operand).  Each superblock pair is staged by direct global->LDS
// loads (global_load_lds_dwordx4) into one of two ring slots, issued a pair
// ahead; one barrier per pair.  The odd waves run their fp32 combine one
// superblock late, so on every SIMD one wave's combine overlaps the other's
// MFMAs.  Odd partial sums are added to the even waves' through LDS at the
// end: every output is written once, in a fixed order.
//
// LDS per superblock stage (37,888 B; 4 stages):
//   AQ  64 rows x 256 qs bytes; row r keeps 16-byte chunk c at position
//       c ^ (r & 15), so the 8 lanes of an A-operand read hit distinct banks
//   AX  64 rows x 3 chunks: record bytes [0,16) (d), [260,276), [276,292) (bsums)
//   WT  128 rows x the 144-byte Q4_K record
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
typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
typedef short v2i16 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_ptr;

constexpr int kMT = 64;          // tokens per workgroup tile
constexpr int kNT = 128;         // weight rows per workgroup tile
constexpr int kThreads = 512;    // 8 waves: 4 column groups x 2 superblock parities
constexpr int kAQ = kMT * 256;                 // 16384
constexpr int kAX = kMT * 48;                  // 3072
constexpr int kWT = kNT * kQ4_KBytes;          // 18432
constexpr int kStage = kAQ + kAX + kWT;        // 37888
constexpr int kSlots = (kAQ + kAX + kWT) / 1024;  // 37 wave-wide 1 KB loads per superblock
constexpr int kSlotsPerWave = (kSlots + 3) / 4;   // 10
static_assert(kStage % 1024 == 0, "a stage is a whole number of wave loads");
static_assert(4 * 32 * 64 * 4 <= 2 * kStage, "reduction buffer fits one ring slot");

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

// Direct global->LDS load of 16 bytes per lane: lane l writes LDS bytes
// [lds + 16 l, lds + 16 l + 16) (lds wave-uniform).  Issued as inline asm so
// that the compiler does not make the following LDS reads, which never touch
// a slot being filled, wait for it; the kernel waits (s_waitcnt) itself.  One
// wait state separates the M0 write from the load that reads it.
// Nothing else in this file's kernel uses M0, so clobbering it is safe (the
// backend's note that a reserved register "may not be preserved" is moot).
__device__ __forceinline__ void lds_dma16(const uint8_t* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds), "v"(g)
               : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_ptr)p;
}

__device__ __forceinline__ int bsum_pair(uint32_t w) {
  // bsums[2s] + bsums[2s+1], two int16 in one dword
  return __builtin_amdgcn_sdot2(__builtin_bit_cast(v2i16, w), (v2i16){1, 1}, 0, false);
}

__global__ void __launch_bounds__(kThreads, 1) q4k_mfma_gemm(GemmArgs a) {
  // two ring slots as separate objects: a slot being filled by direct loads
  // never aliases the slot being read
  __shared__ __align__(16) uint8_t ring0[2 * kStage];
  __shared__ __align__(16) uint8_t ring1[2 * kStage];
  __shared__ __align__(16) float dxr[8 * 2 * 64];  // per wave, 2 slots, 64 token scales

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int par = wave >> 2, wcol = wave & 3;  // superblock parity, column group
  const int col = lane & 31, kg = lane >> 5;
  // Workgroups are dealt round-robin to the 8 XCDs (linear id % 8), each with
  // its own L2.  Give XCD x a contiguous run of tiles, ordered token-tile
  // fastest, so the workgroups resident on one XCD share weight rows and
  // the whole activation block while they sweep K together.
  int m0, n0;
  {
    const int ntm = (a.M + kMT - 1) / kMT;
    const int T = ntm * ((a.N + kNT - 1) / kNT);
    const int L = blockIdx.x, x = L & 7, j = L >> 3;
    const int t = x * (T >> 3) + min(x, T & 7) + j;
    m0 = (t % ntm) * kMT;
    n0 = (t / ntm) * kNT;
  }
  const int nsb = a.K >> 8;
  const size_t wrb = (size_t)nsb * kQ4_KBytes;  // bytes per weight row
  const size_t xrb = (size_t)nsb * kQ8_KBytes;  // bytes per activation row

  // Direct loads: the waves of parity P stage superblock 2*pair + P.  Wave
  // wcol issues slots k = wcol + 4i; slot k writes LDS bytes [1024k, 1024k +
  // 1024) of the stage, lane l the 16 bytes at 1024k + 16l.  src[i] is this
  // lane's source for superblock 0; superblock b adds b * record size.
  const uint8_t* src[kSlotsPerWave];
#pragma unroll
  for (int i = 0; i < kSlotsPerWave; ++i) {
    const int k = min(wcol + 4 * i, kSlots - 1);
    const uint8_t* p;
    if (k < 16) {
      const int q = 64 * k + lane, r = q >> 4, c = (q & 15) ^ (r & 15);
      p = a.Xq + (size_t)min(m0 + r, a.M - 1) * xrb + 4 + 16 * c;
    } else if (k < 19) {
      const int q = 64 * (k - 16) + lane, r = q / 3, e = q - 3 * r;
      p = a.Xq + (size_t)min(m0 + r, a.M - 1) * xrb + (e == 0 ? 0 : 244 + 16 * e);
    } else {
      const int q = 64 * (k - 19) + lane, row = q / 9, part = q - 9 * row;
      p = a.W + (size_t)min(n0 + row, a.N - 1) * wrb + 16 * part;
    }
    src[i] = p;
  }
  // issue this wave's slots i in [i0, i1) of `pair` into `ring`
  auto issue = [&](int pair, uint8_t* ring, int i0, int i1) {
    const int b = min(2 * pair + par, nsb - 1);
    uint8_t* stage = ring + par * kStage;
#pragma unroll
    for (int i = i0; i < i1; ++i) {
      const int k = wcol + 4 * i;
      if (k < kSlots) {
        const size_t off = (size_t)b * (k < 19 ? kQ8_KBytes : kQ4_KBytes);
        lds_dma16(src[i] + off, __builtin_amdgcn_readfirstlane(lds_addr(stage + 1024 * k)));
      }
    }
  };

  v16i lo[2], hi[2];
  v16f y[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) y[t][r] = 0.f;

  // y[t] += dx[row] * dw * (lo + 8 hi); D[i][j] of a 32x32 tile lives in lane
  // j (+32 for the odd 4-row groups), register r holds row 8*(r/4) + 4*kg + r%4
  auto combine = [&](float dwv, const float* dxs) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const float4 d4 = *reinterpret_cast<const float4*>(dxs + 32 * t + 8 * r4 + 4 * kg);
        const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = 4 * r4 + q;
          y[t][r] += (dv[q] * dwv) * (float)(lo[t][r] + 8 * hi[t][r]);
        }
      }
    }
  };

  const v16i zero = {};
  const int npair = (nsb + 1) >> 1;
  const int sw = col & 15;  // A-operand chunk swizzle of this lane's rows
  bool pending = false;     // odd waves: a combine is owed from the previous pair
  float dw_prev = 0.f;
  // one superblock pair: compute from ring slot `cur` while slot `nxt` fills
  auto step = [&](int pair, const uint8_t* cur, uint8_t* nxt) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of this pair have landed
    __syncthreads();                // everyone's have; the previous pair is consumed
    // the next pair's loads are spread over this pair's compute, a few per
    // weight-byte group, so no wave stalls on a burst of ten
    const bool refill = pair + 1 < npair;
    float* dxs = dxr + (2 * wave + (pair & 1)) * 64;
    if (pending) {  // odd waves: combine of the previous superblock
      combine(dw_prev, dxr + (2 * wave + ((pair - 1) & 1)) * 64);
      pending = false;
    }
    if (2 * pair + par >= nsb) {  // odd nsb: the last pair has one superblock
      if (refill) issue(pair + 1, nxt, 0, kSlotsPerWave);
      return;
    }

    const uint8_t* stage = cur + par * kStage;
    const uint8_t* AQ = stage;
    const uint8_t* AX = stage + kAQ;
    const uint8_t* wrow = stage + kAQ + kAX + (32 * wcol + col) * kQ4_KBytes;

    const uint4 h = *reinterpret_cast<const uint4*>(wrow);
    const uint32_t sc03 = h.y & 0x3f3f3f3fu;
    const uint32_t sc47 = (h.w & 0x0f0f0f0fu) | (((h.y >> 6) & 0x03030303u) << 4);
    const uint32_t mn03 = h.z & 0x3f3f3f3fu;
    const uint32_t mn47 = ((h.w >> 4) & 0x0f0f0f0fu) | (((h.z >> 6) & 0x03030303u) << 4);
    const float dw = fp16_to_fp32(h.x & 0xffffu);
    const float dmin = fp16_to_fp32(h.x >> 16);

    // min term: k index of v_mfma_f32_32x32x2f32 = lane / 32, so instruction j
    // covers sub-blocks s = 2j + kg
    float dxa[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) dxa[t] = *reinterpret_cast<const float*>(AX + (32 * t + col) * 48);
    dxs[32 * kg + col] = dxa[kg];  // token scales for the combine (this wave only)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t mw = j < 2 ? mn03 : mn47;
      const float bm = -dmin * (float)((mw >> (8 * (2 * (j & 1) + kg))) & 0xffu);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint32_t bw = *reinterpret_cast<const uint32_t*>(AX + (32 * t + col) * 48 + 16 + 4 * (2 * j + kg));
        const float am = dxa[t] * (float)bsum_pair(bw);
        y[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(am, bm, y[t], 0, 0, 0);
      }
    }

#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (refill) issue(pair + 1, nxt, (kSlotsPerWave * g) / 4, (kSlotsPerWave * (g + 1)) / 4);
      // 16 qs bytes: elements 64g + 16kg + i (low nibble) and 64g + 32 + 16kg + i (high)
      const uint4 q = *reinterpret_cast<const uint4*>(wrow + 16 + 32 * g + 16 * kg);
      const uint32_t scw = g < 2 ? sc03 : sc47;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int s = 2 * g + hf;
        const uint32_t sc = (scw >> (8 * (s & 3))) & 0xffu;
        const uint32_t n0w = hf ? (q.x >> 4) & 0x0f0f0f0fu : q.x & 0x0f0f0f0fu;
        const uint32_t n1w = hf ? (q.y >> 4) & 0x0f0f0f0fu : q.y & 0x0f0f0f0fu;
        const uint32_t n2w = hf ? (q.z >> 4) & 0x0f0f0f0fu : q.z & 0x0f0f0f0fu;
        const uint32_t n3w = hf ? (q.w >> 4) & 0x0f0f0f0fu : q.w & 0x0f0f0f0fu;
        const uint32_t cb = sc & 7u, ca = sc >> 3;
        const v4i b_lo = {(int)mul_bytes(n0w, cb), (int)mul_bytes(n1w, cb), (int)mul_bytes(n2w, cb),
                          (int)mul_bytes(n3w, cb)};
        const v4i b_hi = {(int)mul_bytes(n0w, ca), (int)mul_bytes(n1w, ca), (int)mul_bytes(n2w, ca),
                          (int)mul_bytes(n3w, ca)};
        const int chunk = (2 * s + kg) ^ sw;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const v4i av = *reinterpret_cast<const v4i*>(AQ + (32 * t + col) * 256 + 16 * chunk);
          lo[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b_lo, s == 0 ? zero : lo[t], 0, 0, 0);
          hi[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b_hi, s == 0 ? zero : hi[t], 0, 0, 0);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (par == 0) {
      combine(dw, dxs);
    } else {
      pending = true;
      dw_prev = dw;
    }
  };
  issue(0, ring0, 0, kSlotsPerWave);
  for (int pair = 0; pair < npair; pair += 2) {
    step(pair, ring0, ring1);
    if (pair + 1 < npair) step(pair + 1, ring1, ring0);
  }
  if (pending) combine(dw_prev, dxr + (2 * wave + ((npair - 1) & 1)) * 64);

  // odd-parity partial sums -> LDS (reusing the stages) -> even waves
  __syncthreads();
  float* red = reinterpret_cast<float*>(ring0) + wcol * (32 * 64) + lane;
  if (par == 1) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[(16 * t + r) * 64] = y[t][r];
  }
  __syncthreads();
  if (par == 1) return;
  // store: for a fixed register the 32 lanes of a half cover 32 consecutive columns
  const int gn = n0 + 32 * wcol + col;
  if (gn < a.N) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gm = m0 + 32 * t + 8 * (r >> 2) + 4 * kg + (r & 3);
        if (gm < a.M) a.Y[(size_t)gm * a.N + gn] = y[t][r] + red[(16 * t + r) * 64];
      }
  }
}

void prefill_q4k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M) {
  if (N == 0 || M == 0 || K == 0) return;
  if (K % 256 || W == nullptr || X == nullptr || Xq == nullptr || Y == nullptr || !aligned(W, 4) ||
      !aligned(Xq, 4) || !aligned(Y, 4) || N > (size_t)INT32_MAX || K > (size_t)INT32_MAX ||
      M > (size_t)INT32_MAX || ((N + kNT - 1) / kNT) * ((M + kMT - 1) / kMT) > (size_t)INT32_MAX) {
    set_error(hipErrorInvalidValue);
    return;
  }
  quantize_q8_k(X, Xq, M * K);
  GemmArgs a{W, Xq, Y, (int)N, (int)K, (int)M};
  const size_t tiles = ((N + kNT - 1) / kNT) * ((M + kMT - 1) / kMT);
  q4k_mfma_gemm<<<dim3((unsigned)tiles), kThreads, 0, current_stream()>>>(a);
  check_launch();
}

}  // namespace

// Prefill entry: MFMA GEMM when the shape suits it, the decode GEMV otherwise.
void mul_mat_q4k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M) {
  if (M >= 16 && aligned(W, 4))
    prefill_q4k(W, X, Xq, Y, N, K, M);
  else
    decode_q4k(W, X, Xq, Y, N, K, M);
}

}  // namespace weft
