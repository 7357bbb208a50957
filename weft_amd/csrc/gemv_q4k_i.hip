// Q4_K x Q8_K GEMV over the persisted 16-row interleaved layout Q4K_I[16]
// (q4_k_q8_k_gemv, examples/kernels/gemv/q4_k.py:8-26; the _groups4 and
// _contract variants, gemv/q4_k_groups4.py and gemv/q4_k_contract.py, compute
// the same function with other RVV loop orders and share this kernel), plus
// the layout's artifact-phase entry points <symbol>_W_packed_size and
// <symbol>_W_pack (lib/Target/Emission/Emitter.h:231-272).
//
// Layout (examples/formats/ggml.py:286-290, doc/dsl/encoding-and-artifacts.md
// :180-209; record address of lib/Target/Emission/Memory.cpp:984-991): rows
// are grouped in cohorts of 16; superblock j of cohort c is a 2304-byte block
// at ((c * nsb) + j) * 2304 whose byte 16 b + r is byte b of row 16 c + r's
// 144-byte Q4_K record.  M must be a multiple of 16.
//
// Semantics per row (q4_k.py:15-25 = ggml_vec_dot_q4_K_q8_K_generic,
// ggml-cpu/quants.c:645-718): y = sum_b ds_b (d_b S_b - dmin_b Mn_b) with
// exact int32 S_b = sum_s sc_s sum_{32} q x and Mn_b = sum_s m_s
// (bsum_2s + bsum_2s+1).  X is a quantized Q8_K activation (K / 256 records).
//
// gfx950 mapping.  The interleave puts byte b of 16 rows in one 16-byte
// line.  ds_read_b64_tr_b8 reads such lines transposed: within each group of
// 16 lanes, lane i receives bytes b0 .. b0 + 7 of row i from eight
// consecutive 16-byte lines.  So a workgroup takes one cohort, its four waves
// split the superblocks round-robin, and in every wave lane (r, g) = (lane %
// 16, lane / 16) owns row r and 64-element group g of each of its
// superblocks: six transposed reads give it the row's 16-byte header and the
// group's 32 nibble bytes, which meet the activation (staged in LDS once per
// workgroup, read as broadcasts) in sixteen v_dot4_i32_i8.  Each wave streams
// its superblocks from global memory into a private LDS ring by direct loads
// (three per 2304-byte block), kRing blocks ahead, and waits on its own
// counters: no barrier inside the loop.  Lane groups are summed with two
// cross-lane steps and the four waves' partial sums through LDS, in a fixed
// order, so every output is written once.
#include <algorithm>

#include "runtime.h"
#include "weft_common.h"
#include "weft_hip.h"

namespace weft {
namespace {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_ptr;
typedef __attribute__((address_space(3))) v2i lds_v2i;

constexpr int kCohort = 16;                          // rows per interleaved cohort
constexpr int kBlock = kCohort * kQ4_KBytes;          // 2304 bytes per cohort superblock
// Blocks per wave in LDS: one being computed, one in flight.  Deeper rings
// measured slower on this chip (more requests in flight per wave queue in
// front of the ones needed next); parallelism comes from waves instead.
constexpr int kRing = 2;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_ptr)p;
}

// direct global->LDS loads: lane l writes [lds + 16 l, +16) / [lds + 4 l, +4)
__device__ __forceinline__ void dma16(const uint8_t* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds), "v"(voff), "s"(sbase)
               : "memory", "m0");
}
__device__ __forceinline__ void dma4(const uint8_t* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2"
               :
               : "s"(lds), "v"(voff), "s"(sbase)
               : "memory", "m0");
}

typedef __attribute__((address_space(3))) uint8_t lds_u8;

// Eight bytes of row (lane % 16) of eight consecutive 16-byte lines: lane i
// of each 16-lane group addresses half line i (byte offset 8 i of the
// 128-byte window) and receives row i's eight bytes, one per line.
__device__ __forceinline__ v2i tr8(const uint8_t* base, uint32_t offset) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)((lds_u8*)base + offset));
}

// s_waitcnt for "at most n younger blocks (3 loads each) still in flight"
__device__ __forceinline__ void wait_blocks_younger(int n) {
  switch (n) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(9)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(12)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(18)" ::: "memory"); break;
  }
}

struct GemvArgs {
  const uint8_t* W;   // packed Q4K_I[16]
  const uint8_t* X;   // Q8_K records
  float* Y;
  int M, K;
};

// kWaves waves per workgroup split the cohort's superblocks round-robin.
template <int kWaves>
__global__ void __launch_bounds__(64 * kWaves) q4k_i16_gemv_kernel(GemvArgs a) {
  constexpr int kThreads = 64 * kWaves;
  constexpr int kRingBytes = kWaves * kRing * kBlock;
  extern __shared__ __align__(16) uint8_t lds[];
  const int nsb = a.K >> 8;
  uint8_t* ring = lds;                                                // [wave][kRing][2304]
  int8_t* xqs = reinterpret_cast<int8_t*>(lds + kRingBytes);          // nsb x 256
  int* xbp = reinterpret_cast<int*>(lds + kRingBytes + 256 * nsb);    // nsb x 8 pair sums
  float* xd = reinterpret_cast<float*>(xbp + 8 * nsb);               // nsb
  float* part = xd + nsb;                                             // kWaves x 16

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int r = lane & 15, g = lane >> 4;
  const int c = blockIdx.x;

  // ---- this wave's superblocks j = wave, wave + 4, ...: direct loads of the
  // 2304-byte blocks into its ring (two 1 KB loads and one 256-byte load)
  const uint8_t* wc = a.W + (size_t)c * nsb * kBlock;
  const int my = nsb > wave ? (nsb - wave + kWaves - 1) / kWaves : 0;
  uint8_t* wring = ring + wave * (kRing * kBlock);
  auto issue = [&](int i) {
    const int j = min(wave + kWaves * i, nsb - 1);  // past the end: a valid block, never read
    const uint8_t* src = wc + (size_t)j * kBlock;
    const uint32_t dst = lds_addr(wring + (i % kRing) * kBlock);
    dma16(src, 16u * lane, __builtin_amdgcn_readfirstlane(dst));
    dma16(src, 1024u + 16u * lane, __builtin_amdgcn_readfirstlane(dst + 1024u));
    dma4(src, 2048u + 4u * lane, __builtin_amdgcn_readfirstlane(dst + 2048u));
  };
  // the first kRing - 1 blocks go out before the activation is staged
#pragma unroll
  for (int i = 0; i < kRing - 1; ++i) issue(i);

  // ---- the Q8_K activation into LDS: qs at 256 j, d, and the 8 sub-block
  // sums bsum_2s + bsum_2s+1 (GGML's min-term operand, quants.c:693-699)
  for (int idx = tid; idx < nsb * 64; idx += kThreads) {
    const int j = idx >> 6, w = idx & 63;
    const uint8_t* rec = a.X + (size_t)j * kQ8_KBytes;
    reinterpret_cast<uint32_t*>(xqs + 256 * j)[w] = reinterpret_cast<const uint32_t*>(rec + 4)[w];
    if (w < 8) {
      const int16_t* bs = reinterpret_cast<const int16_t*>(rec + 260);
      xbp[8 * j + w] = (int)bs[2 * w] + (int)bs[2 * w + 1];
    } else if (w == 8) {
      xd[j] = *reinterpret_cast<const float*>(rec);
    }
  }
  __syncthreads();

  // this lane's half-line address within a block: lane i of the 16-lane
  // group covers bytes 8 i .. 8 i + 7 of each 128-byte (8-line) window
  const uint32_t lofs = 8u * (uint32_t)r;
  const uint32_t qofs = (uint32_t)(16 * (16 + 32 * g)) + lofs;  // first nibble line of group g

  float acc = 0.f;
  for (int i = 0; i < my; ++i) {
    // block i has landed once only the younger blocks' loads (three per
    // block, completing in order) are outstanding
    wait_blocks_younger(min(kRing - 2, my - 1 - i));
    const uint8_t* blk = wring + (i % kRing) * kBlock;
    // header: bytes 0..7 (d, dmin, scales 0..3) and 8..15 (scales 4..11) of row r
    const v2i h0 = tr8(blk, lofs);
    const v2i h1 = tr8(blk, 128u + lofs);
    // group g's 32 nibble bytes: 16 + 32 g .. 16 + 32 g + 31
    const v2i q0 = tr8(blk, qofs);
    const v2i q1 = tr8(blk, qofs + 128u);
    const v2i q2 = tr8(blk, qofs + 256u);
    const v2i q3 = tr8(blk, qofs + 384u);
    // every lane has read its block: the slot can be refilled
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (i + kRing - 1 < my) issue(i + kRing - 1);

    const int j = wave + kWaves * i;
    const int8_t* xs = xqs + 256 * j + 64 * g;
    const int4 xl0 = *reinterpret_cast<const int4*>(xs);
    const int4 xl1 = *reinterpret_cast<const int4*>(xs + 16);
    const int4 xh0 = *reinterpret_cast<const int4*>(xs + 32);
    const int4 xh1 = *reinterpret_cast<const int4*>(xs + 48);
    const int2 bp = *reinterpret_cast<const int2*>(xbp + 8 * j + 2 * g);
    const float dx = xd[j];

    // 6-bit scale and min of sub-blocks 2g, 2g + 1 (the utmp unpack of
    // ggml-cpu/quants.c:676-681): u0 = scale bytes 0-3, u1 = 4-7, u2 = 8-11
    const uint32_t u0 = (uint32_t)h0.y, u1 = (uint32_t)h1.x, u2 = (uint32_t)h1.y;
    const uint32_t scw = g < 2 ? (u0 & 0x3f3f3f3fu) : ((u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4));
    const uint32_t mnw = g < 2 ? (u1 & 0x3f3f3f3fu) : (((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4));
    const int sh = 16 * (g & 1);
    const int sc_lo = (scw >> sh) & 0xff, sc_hi = (scw >> (sh + 8)) & 0xff;
    const int m_lo = (mnw >> sh) & 0xff, m_hi = (mnw >> (sh + 8)) & 0xff;

    const uint32_t qw[8] = {(uint32_t)q0.x, (uint32_t)q0.y, (uint32_t)q1.x, (uint32_t)q1.y,
                            (uint32_t)q2.x, (uint32_t)q2.y, (uint32_t)q3.x, (uint32_t)q3.y};
    const int xlw[8] = {xl0.x, xl0.y, xl0.z, xl0.w, xl1.x, xl1.y, xl1.z, xl1.w};
    const int xhw[8] = {xh0.x, xh0.y, xh0.z, xh0.w, xh1.x, xh1.y, xh1.z, xh1.w};
    int pl = 0, ph = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      pl = dot4((int)(qw[k] & 0x0f0f0f0fu), xlw[k], pl);
      ph = dot4((int)((qw[k] >> 4) & 0x0f0f0f0fu), xhw[k], ph);
    }
    // |pl|, |ph| <= 32 * 15 * 127 and scales <= 63: 24-bit multiplies are exact
    const int S = __mul24(sc_lo, pl) + __mul24(sc_hi, ph);
    const int Mn = __mul24(m_lo, bp.x) + __mul24(m_hi, bp.y);
    const float dw = fp16_to_fp32((uint32_t)h0.x & 0xffffu);
    const float dmin = fp16_to_fp32((uint32_t)h0.x >> 16);
    acc += dx * (dw * (float)S - dmin * (float)Mn);
  }

  // sum the four lane groups of each row (lanes r, r + 16, r + 32, r + 48)
  acc += __shfl_xor(acc, 16, kWave);
  acc += __shfl_xor(acc, 32, kWave);
  if (lane < kCohort) part[wave * kCohort + lane] = acc;
  __syncthreads();
  if (wave == 0 && lane < kCohort) {
    float y = part[lane];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) y += part[w * kCohort + lane];
    a.Y[(size_t)c * kCohort + lane] = y;
  }
}

// Pack: thread t writes output line t (16 bytes = byte b of the 16 rows of a
// cohort superblock), gathering the bytes from the 16 source records.
__global__ void __launch_bounds__(256) q4k_i16_pack_kernel(const uint8_t* __restrict__ src,
                                                          uint8_t* __restrict__ dst, long long lines,
                                                          int nsb) {
  const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= lines) return;
  const long long blockid = t / kQ4_KBytes;   // c * nsb + j
  const int b = (int)(t - blockid * kQ4_KBytes);
  const long long c = blockid / nsb;
  const int j = (int)(blockid - c * nsb);
  const size_t rowbytes = (size_t)nsb * kQ4_KBytes;
  const uint8_t* s = src + (size_t)(c * kCohort) * rowbytes + (size_t)j * kQ4_KBytes + b;
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t v = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) v |= (uint32_t)s[(size_t)(4 * q + k) * rowbytes] << (8 * k);
    w[q] = v;
  }
  *reinterpret_cast<uint4*>(dst + 16 * t) = make_uint4(w[0], w[1], w[2], w[3]);
}

}  // namespace

namespace {
// waves per cohort: the power of two (up to 16, and at most one per
// superblock) nearest to 4096 waves in all, which measured best from 14 to
// 22 waves per CU at the reference's shapes
int i16_waves(size_t cohorts, size_t nsb) {
  int waves = 1;
  while (waves < 16 && (size_t)waves * 2 <= nsb && (double)cohorts * waves * 1.41421356 < 4096.0) waves *= 2;
  return waves;
}
// LDS of one workgroup: the waves' rings, the Q8_K row (qs, pair sums, d)
// and the partial sums
size_t i16_lds(int waves, size_t nsb) {
  return (size_t)waves * kRing * kBlock + nsb * (256 + 32 + 4) + (size_t)waves * kCohort * 4;
}

bool gemv_shape_ok(size_t M, size_t K) {
  return K % 256 == 0 && M % kCohort == 0 && M <= (size_t)INT32_MAX && K <= (size_t)INT32_MAX;
}

}  // namespace

bool q4k_i16_gemv_fits(size_t M, size_t K) {
  const size_t nsb = K / 256;
  return i16_lds(i16_waves(M / kCohort, nsb), nsb) <= max_lds_per_block();
}

size_t q4k_i16_packed_size(size_t M, size_t K) {
  if (!gemv_shape_ok(M, K)) {
    set_error(hipErrorInvalidValue);
    return 0;
  }
  return M * (K / 256) * kQ4_KBytes;
}

void q4k_i16_pack(const uint8_t* source, uint8_t* target, size_t M, size_t K) {
  if (M == 0 || K == 0) return;
  if (!gemv_shape_ok(M, K) || source == nullptr || target == nullptr || !aligned(target, 16)) {
    set_error(hipErrorInvalidValue);
    return;
  }
  const long long lines = (long long)(M / kCohort) * (long long)(K / 256) * kQ4_KBytes;
  const long long blocks = (lines + 255) / 256;
  if (blocks > INT32_MAX) {
    set_error(hipErrorInvalidValue);
    return;
  }
  q4k_i16_pack_kernel<<<(unsigned)blocks, 256, 0, current_stream()>>>(source, target, lines,
                                                                       (int)(K / 256));
  check_launch("q4k_i16_pack_kernel");
}

void q4k_i16_gemv(const uint8_t* W, const uint8_t* X, float* Y, size_t M, size_t K) {
  if (M == 0 || K == 0) return;
  if (!gemv_shape_ok(M, K) || W == nullptr || X == nullptr || Y == nullptr || !aligned(W, 16) ||
      !aligned(X, 4) || !aligned(Y, 4)) {
    set_error(hipErrorInvalidValue);
    return;
  }
  const size_t nsb = K / 256, cohorts = M / kCohort;
  const int waves = i16_waves(cohorts, nsb);
  const size_t lds = i16_lds(waves, nsb);
  if (lds > max_lds_per_block()) {
    set_error(hipErrorInvalidValue);  // the activation does not fit in LDS
    return;
  }
  if (cohorts > (size_t)INT32_MAX) {
    set_error(hipErrorInvalidValue);
    return;
  }
  GemvArgs a{W, X, Y, (int)M, (int)K};
  const dim3 grid((unsigned)cohorts);
  switch (waves) {
    case 1: q4k_i16_gemv_kernel<1><<<grid, 64, lds, current_stream()>>>(a); break;
    case 2: q4k_i16_gemv_kernel<2><<<grid, 128, lds, current_stream()>>>(a); break;
    case 4: q4k_i16_gemv_kernel<4><<<grid, 256, lds, current_stream()>>>(a); break;
    case 8: q4k_i16_gemv_kernel<8><<<grid, 512, lds, current_stream()>>>(a); break;
    default: q4k_i16_gemv_kernel<16><<<grid, 1024, lds, current_stream()>>>(a); break;
  }
  check_launch("q4k_i16_gemv_kernel");
}

}  // namespace weft

extern "C" {

size_t q4_k_q8_k_gemv_W_packed_size(size_t M, size_t K) { return weft::q4k_i16_packed_size(M, K); }
void q4_k_q8_k_gemv_W_pack(const uint8_t* source, uint8_t* target, size_t M, size_t K) {
  weft::q4k_i16_pack(source, target, M, K);
}
void q4_k_q8_k_gemv(const uint8_t* W, const uint8_t* X, float* Y, size_t M, size_t K) {
  weft::q4k_i16_gemv(W, X, Y, M, K);
}

size_t q4_k_q8_k_gemv_groups4_W_packed_size(size_t M, size_t K) {
  return weft::q4k_i16_packed_size(M, K);
}
void q4_k_q8_k_gemv_groups4_W_pack(const uint8_t* source, uint8_t* target, size_t M, size_t K) {
  weft::q4k_i16_pack(source, target, M, K);
}
void q4_k_q8_k_gemv_groups4(const uint8_t* W, const uint8_t* X, float* Y, size_t M, size_t K) {
  weft::q4k_i16_gemv(W, X, Y, M, K);
}

size_t q4_k_q8_k_gemv_contract_W_packed_size(size_t M, size_t K) {
  return weft::q4k_i16_packed_size(M, K);
}
void q4_k_q8_k_gemv_contract_W_pack(const uint8_t* source, uint8_t* target, size_t M, size_t K) {
  weft::q4k_i16_pack(source, target, M, K);
}
void q4_k_q8_k_gemv_contract(const uint8_t* W, const uint8_t* X, float* Y, size_t M, size_t K) {
  weft::q4k_i16_gemv(W, X, Y, M, K);
}

}  // extern "C"
