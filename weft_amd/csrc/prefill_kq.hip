// Q6_K and Q5_K x Q8_K prefill GEMMs on int8 MFMA (production_mul_mat_q6_k,
// production_mul_mat_q5_k; examples/kernels/mul_mat/q6_k.py:9-37,
// q5_k.py:9-37), with a grouped MUL_MAT_ID mode.
//
// Q6_K (ggml-cpu/quants.c:800-853):
//   Y[m,n] = sum_b (dw[n,b] dx[m,b]) * sum_{j<16} sc[n,b,j] * P[m,n,b,j]
//   P = sum_{k in 16-group j} q8[m,k] * (q6[n,k] - 32)                (exact int32)
// The signed 8-bit scale times a 6-bit value does not fit an int8 operand,
// so it is applied after the product: one v_mfma_i32_32x32x32_i8 covers a
// 32-group, and it runs twice with the weight operand of one 16-element half
// (the lanes of the other half hold zeros); each product tile takes its
// half's scale in one v_mad_i32_i24 per output (|P| <= 65536, |sc| <= 128,
// eight groups < 2^27).  The weight operand is q6 - 32 as a signed byte,
// formed four at a time: ((q | 0x80) - 0x20) ^ 0x80 never borrows.
//
// Q5_K (ggml-cpu/quants.c:720-798):
//   Y[m,n] = sum_b (dw dx) * S - (dmin dx) * Mn
//   S  = sum_{g<8} sc[n,b,g] * sum_{k in 32-group g} q8 * q5            (exact int32)
//   Mn = sum_{j<16} m[n,b,j/2] * bsum[m,b,j]                             (exact)
// q5 in [0, 31] is the weight operand as it is; one MFMA per 32-group and
// one multiply-add of its 6-bit scale per output.  Mn comes from one
// v_mfma_f32_32x32x8_f16 per half superblock: Q8_K's bsums are sums of 16
// int8 (|bsum| <= 2032) and the mins 6-bit, so both are exact f16 operands
// and the fp32 result is exact (|Mn| < 2^21).
//
// The superblock's fp32 factors dx dw (and dx dmin) of every output come from
// one bf16 outer-product MFMA per tile each (dx = h + m + l in bf16 parts
// against the fp16 scale's two bf16 parts: six exact products summed in
// fp32), so the combine is a convert and one FMA per output (two for Q5_K).
//
// Tiling: 64 tokens x 128 weight rows per workgroup, 8 waves; wave w takes
// weight rows 32 (w % 4) .. +31 and the half superblock w / 4 (elements
// 128 h .. +127: Q6_K's ql/qh half, Q5_K's groups 4h .. 4h+3) for all 64
// tokens as two 32x32 tiles that share the weight operand.  One superblock
// per ring slot, two slots: the waves stage superblock b+1 by direct
// global->LDS loads while computing b (Q5_K's 176-byte records as 16-byte
// chunks when the rows are aligned).  A Q6_K record (210 bytes) is 2-byte
// aligned for odd b, so its row is staged from the dword holding its first
// byte (54 dwords, 216 bytes per LDS row) and the odd superblocks read with
// a 2-byte alignment; the even/odd slots are the two instantiations of the
// step.  Both halves' partial sums meet in LDS at the end and every output
// is written once, even + odd, with 16-byte stores (tile_store.h).
#include <algorithm>
#include <type_traits>

#include "kernels.h"
#include "runtime.h"
#include "tile_store.h"
#include "weft_common.h"
#include "weft_hip.h"

namespace weft {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void* lds_ptr;

constexpr int kMT = 64;        // tokens per workgroup tile
constexpr int kNT = 128;       // weight rows per workgroup tile
constexpr int kThreads = 512;  // 8 waves: 4 column groups x 2 half superblocks
constexpr int kAQ = kMT * 256;  // activation int8 of one superblock

enum class KQ { Q6_K, Q5_K };

template <KQ F>
struct KTile {
  static constexpr bool k6 = F == KQ::Q6_K;
  static constexpr int kRec = k6 ? kQ6_KBytes : kQ5_KBytes;  // 210 / 176
  static constexpr int kLoadD = k6 ? 54 : 44;                // dwords staged per weight row
  static constexpr int kRowB = 4 * kLoadD;                   // LDS bytes per weight row: 216 / 176
  static constexpr int kBS = k6 ? 0 : kMT * 32;              // Q5_K: the tokens' bsums
  static constexpr int kWT = kNT * kRowB;
  static constexpr int kSlot = kAQ + kBS + kWT;              // 44,032 / 40,960
  static constexpr int kWSlots = kNT * kLoadD / 64;          // 108 / 88 wave-wide dword loads
  static_assert(kNT * kLoadD % 64 == 0, "weight tile is whole wave loads");
  static_assert(kTilePlaneBytes <= kSlot, "an output plane fits one ring slot");
};

struct GemmArgs {
  const uint8_t* W;
  const uint8_t* Xq;
  float* Y;
  int N, K, M;
  size_t ldw;      // bytes between weight rows
  long long ldy;   // floats between output rows
  GroupTiles grp;  // grouped (MUL_MAT_ID) mode
};

// Direct global->LDS loads; lane l writes [lds + size*l, +size).  Inline asm
// keeps the compiler from making unrelated LDS reads wait for them; the
// kernel waits (s_waitcnt) itself.  Nothing else in this kernel uses M0.
__device__ __forceinline__ void lds_dma16(const uint8_t* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds), "v"(g)
               : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4(const uint8_t* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off"
               :
               : "s"(lds), "v"(g)
               : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_ptr)p;
}
__device__ __forceinline__ void pin(int& v) { asm volatile("" : "+v"(v)); }

// 16 bytes that start kSh (0 or 2) bytes past the 8-byte aligned LDS address p
template <int kSh>
__device__ __forceinline__ uint4 ld16(const uint8_t* p) {
  const uint2 a = *reinterpret_cast<const uint2*>(p);
  const uint2 b = *reinterpret_cast<const uint2*>(p + 8);
  if constexpr (kSh == 0) {
    return make_uint4(a.x, a.y, b.x, b.y);
  } else {
    const uint32_t c = *reinterpret_cast<const uint32_t*>(p + 16);
    return make_uint4(__builtin_amdgcn_alignbyte(a.y, a.x, kSh), __builtin_amdgcn_alignbyte(b.x, a.y, kSh),
                      __builtin_amdgcn_alignbyte(b.y, b.x, kSh), __builtin_amdgcn_alignbyte(c, b.y, kSh));
  }
}

template <bool kGroup, KQ F>
__global__ void __launch_bounds__(kThreads, 1) kq_mfma_gemm(GemmArgs a) {
  using TT = KTile<F>;
  constexpr bool k6 = TT::k6;
  constexpr int kRowB = TT::kRowB, kLoadD = TT::kLoadD, kWSlots = TT::kWSlots;
  __shared__ __align__(16) uint8_t ring0[TT::kSlot];
  __shared__ __align__(16) uint8_t ring1[TT::kSlot];
  // [slot][token]: the token's Q8_K d as the bf16 parts of the outer-product
  // factor MFMA ((h,h), (m,m), (l,l), 0)
  __shared__ __align__(16) uint4 dxq[2][kMT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int h = wave >> 2, wcol = wave & 3;
  const int col = lane & 31, kg = lane >> 5;
  const int nsb = a.K >> 8;
  const size_t wrb = a.ldw;
  const size_t xrb = (size_t)nsb * kQ8_KBytes;

  // XCD-aware tile order (workgroups are dealt round-robin to 8 XCDs);
  // grouped: m0 indexes the pair list, mrows pairs, W the tile's expert
  int m0, n0, mrows;
  const uint8_t* W = a.W;
  {
    const int ntm = kGroup ? a.grp.tmax : (a.M + kMT - 1) / kMT;
    const int Tn = ntm * ((a.N + kNT - 1) / kNT);
    const int L = blockIdx.x, x = L & 7, j = L >> 3;
    const int t = x * (Tn >> 3) + min(x, Tn & 7) + j;
    n0 = (t / ntm) * kNT;
    if constexpr (kGroup) {
      long long w_off;
      if (!group_tile(a.grp, t % ntm, m0, mrows, w_off)) return;  // no barrier yet
      W += w_off;
    } else {
      m0 = (t % ntm) * kMT;
      mrows = min(kMT, a.M - m0);
    }
  }
  auto act_row = [&](int r) -> int {
    if constexpr (kGroup)
      return group_act_row(a.grp, m0, r);
    else
      return m0 + r;
  };

  // activation int8 of one superblock: 16 wave-wide 16-byte loads, 2 per
  // wave; token r's chunk c lands at 256 r + 16 (c ^ (r & 15))
  const uint8_t* asrc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = 64 * (wave + 8 * i) + lane, r = q >> 4, c = (q & 15) ^ (r & 15);
    asrc[i] = a.Xq + (size_t)act_row(min(r, mrows - 1)) * xrb + 4 + 16 * c;
  }
  // Q5_K: the 32 bsum bytes of each token, 2 wave loads (waves 0, 1)
  const uint8_t* bsrc = a.Xq + (size_t)act_row(min((64 * (wave & 1) + lane) >> 1, mrows - 1)) * xrb + 260 +
                        16 * (lane & 1);
  const uint8_t* dsrc = a.Xq + (size_t)act_row(min(lane, mrows - 1)) * xrb;  // Q8_K d of token lane

  const bool w16 = ((reinterpret_cast<uintptr_t>(W) | wrb) & 15) == 0;  // Q5_K: 16-byte weight loads
  const uint32_t ring_lds[2] = {(uint32_t)__builtin_amdgcn_readfirstlane(lds_addr(ring0)),
                                (uint32_t)__builtin_amdgcn_readfirstlane(lds_addr(ring1))};
  auto issue = [&](int b, int slot) {
    const uint32_t base = ring_lds[slot];
#pragma unroll
    for (int i = 0; i < 2; ++i)
      lds_dma16(asrc[i] + (size_t)b * kQ8_KBytes, base + 1024 * (wave + 8 * i));
    if constexpr (!k6) {
      if (wave < 2) lds_dma16(bsrc + (size_t)b * kQ8_KBytes, base + kAQ + 1024 * wave);
    }
    // weight rows: Q6_K from the dword holding the record's first byte (2
    // bytes before it for odd b); dword 53 is padding and re-reads dword 52
    const size_t wb = (size_t)b * TT::kRec - (k6 ? 2 * (b & 1) : 0);
    if constexpr (!k6) {
      // Q5_K records are 11 chunks of 16 bytes: 22 wave-wide 16-byte loads
      // when the rows are 16-byte aligned (row q / 11, chunk q % 11)
      if (w16) {
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          const int k = wave + 8 * i;
          if (k < kNT * 11 / 64) {
            const int q = 64 * k + lane, row = q / 11;
            const uint8_t* g = W + (size_t)min(n0 + row, a.N - 1) * wrb + wb + 16 * (q - 11 * row);
            lds_dma16(g, base + kAQ + TT::kBS + 1024 * k);
          }
        }
        return;
      }
    }
#pragma unroll
    for (int i = 0; i < (kWSlots + 7) / 8; ++i) {
      const int k = wave + 8 * i;
      if (k < kWSlots) {
        const int q = 64 * k + lane, row = q / kLoadD, part = q - kLoadD * row;
        const uint8_t* g = W + (size_t)min(n0 + row, a.N - 1) * wrb + wb + 4 * (k6 ? min(part, 52) : part);
        lds_dma4(g, base + kAQ + TT::kBS + 256 * k);
      }
    }
  };
  float dxr = 0.f;
  auto load_dx = [&](int b) { dxr = *reinterpret_cast<const float*>(dsrc + (size_t)b * kQ8_KBytes); };

  v16i acc[2];
  v16f y[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) y[t][r] = 0.f;
  const v16i zero = {};
  const int sw = col & 15;

  auto step = [&](int b, const uint8_t* cur, int nxt, auto shift) {
    constexpr int kSh = decltype(shift)::value;  // byte offset of the Q6_K record in its LDS row
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of superblock b have landed
    __syncthreads();                // everyone's; superblock b - 1 is consumed
    const bool refill = b + 1 < nsb;
    if (refill && wave == 0) load_dx(b + 1);
    // this wave's share of superblock b + 1's direct loads goes out after
    // the half's second group (below): issued right after the barrier, every
    // wave's first group waited behind the workgroup's queued loads (the
    // MXFP4 GEMM measured 39.5 -> 37.8 us per call for the move)
    const uint8_t* AQ = cur;
    const uint8_t* row = cur + kAQ + TT::kBS + (32 * wcol + col) * kRowB;  // this lane's weight row
    const uint4* dxb = &dxq[b & 1][0];
    float dw, dmin = 0.f;
    v16f mn[2];
    if constexpr (k6) {
      // ql of groups s = 0, 2 (P0) and 1, 3 (P1), qh of all four, the 8 scales of the half
      const uint4 P0 = ld16<kSh>(row + 64 * h + 16 * kg);
      const uint4 P1 = ld16<kSh>(row + 64 * h + 32 + 16 * kg);
      const uint4 Q = ld16<kSh>(row + 128 + 32 * h + 16 * kg);
      const uint2 s8 = *reinterpret_cast<const uint2*>(row + 192 + 8 * h);
      uint32_t sc0 = s8.x, sc1 = s8.y;
      if constexpr (kSh != 0) {
        const uint32_t s2 = *reinterpret_cast<const uint32_t*>(row + 200 + 8 * h);
        sc0 = __builtin_amdgcn_alignbyte(s8.y, s8.x, kSh);
        sc1 = __builtin_amdgcn_alignbyte(s2, s8.y, kSh);
      }
      const uint32_t dword = *reinterpret_cast<const uint32_t*>(row + 208);
      dw = fp16_to_fp32(kSh ? dword >> 16 : dword & 0xffffu);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint4 L = (s & 1) ? P1 : P0;
        const uint32_t lq[4] = {L.x, L.y, L.z, L.w}, hq[4] = {Q.x, Q.y, Q.z, Q.w};
        v4i bv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t lo = ((lq[i] >> (4 * (s >> 1))) & 0x0f0f0f0fu) | 0x80808080u;
          const uint32_t hi = (s < 3 ? hq[i] << (4 - 2 * s) : hq[i] >> 2) & 0x30303030u;
          bv[i] = (int)(((lo | hi) - 0x20202020u) ^ 0x80808080u);  // q6 - 32, four signed bytes
        }
        const v4i bz = {};
        const uint32_t sb = ((s < 2 ? sc0 : sc1) >> (16 * (s & 1))) & 0xffffu;
        const int sc_lo = (int)(int8_t)(sb & 0xffu), sc_hi = (int)(int8_t)(sb >> 8);
        const int chunk = (2 * (4 * h + s) + kg) ^ sw;
        v16i I[2], I2[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const v4i av = *reinterpret_cast<const v4i*>(AQ + (32 * t + col) * 256 + 16 * chunk);
          I[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, kg ? bz : bv, zero, 0, 0, 0);
          I2[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, kg ? bv : bz, zero, 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            int v = __mul24(I[t][r], sc_lo) + __mul24(I2[t][r], sc_hi) + (s == 0 ? 0 : acc[t][r]);
            pin(v);
            acc[t][r] = v;
          }
        if (s == 1 && refill) issue(b + 1, nxt);
      }
    } else {
      const uint4 hd = *reinterpret_cast<const uint4*>(row);  // d, dmin, 12 scale bytes
      dw = fp16_to_fp32(hd.x & 0xffffu);
      dmin = fp16_to_fp32(hd.x >> 16);
      const uint4 Q = *reinterpret_cast<const uint4*>(row + 16 + 16 * kg);  // qh bytes 16kg .. +15
      const uint4 L0 = *reinterpret_cast<const uint4*>(row + 48 + 64 * h + 16 * kg);       // qs of j = 2h
      const uint4 L1 = *reinterpret_cast<const uint4*>(row + 48 + 64 * h + 32 + 16 * kg);  // j = 2h + 1
      const uint32_t hq[4] = {Q.x, Q.y, Q.z, Q.w};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int g = 4 * h + s;
        const uint4 L = (s >> 1) ? L1 : L0;
        const uint32_t lq[4] = {L.x, L.y, L.z, L.w};
        v4i bv;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          bv[i] = (int)(((lq[i] >> (4 * (s & 1))) & 0x0f0f0f0fu) | (((hq[i] >> g) & 0x01010101u) << 4));
        int sc, m;
        q4k_scale_min(g, hd.y, hd.z, hd.w, sc, m);
        const int chunk = (2 * g + kg) ^ sw;
        v16i I[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const v4i av = *reinterpret_cast<const v4i*>(AQ + (32 * t + col) * 256 + 16 * chunk);
          I[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, zero, 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            int v = __mul24(I[t][r], sc) + (s == 0 ? 0 : acc[t][r]);
            pin(v);
            acc[t][r] = v;
          }
        if (s == 1 && refill) issue(b + 1, nxt);
      }
      // Mn of this half: bsums 8h + 4kg .. +3 of token 32t + col against the
      // mins of groups 4h + 2kg, 4h + 2kg + 1 (two bsums each) of row col
      int m_a, m_b, sdummy;
      q4k_scale_min(4 * h + 2 * kg, hd.y, hd.z, hd.w, sdummy, m_a);
      q4k_scale_min(4 * h + 2 * kg + 1, hd.y, hd.z, hd.w, sdummy, m_b);
      const v4h bm = {(_Float16)m_a, (_Float16)m_a, (_Float16)m_b, (_Float16)m_b};
      const v16f fz = {};
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint2 bs = *reinterpret_cast<const uint2*>(AQ + kAQ + (32 * t + col) * 32 + 16 * h + 8 * kg);
        const v4h am = {(_Float16)(short)(bs.x & 0xffffu), (_Float16)(short)(bs.x >> 16),
                        (_Float16)(short)(bs.y & 0xffffu), (_Float16)(short)(bs.y >> 16)};
        mn[t] = __builtin_amdgcn_mfma_f32_32x32x8f16(am, bm, fz, 0, 0, 0);
      }
    }
    // y += (dx dw) acc [- (dx dmin) Mn]: the factors of every output from a
    // bf16 outer-product MFMA per tile (token d = h + m + l against the
    // row's fp16 scale = f_h + f_l, K slots 0-5 of the kg = 0 lanes; the
    // kg = 1 lanes' slots are zero), then two VALU operations per output
    const uint32_t kz = kg ? 0u : 0xffffffffu;
    const uint32_t pw = bf16_split2(dw) & kz;
    const v4i bw = {(int)pw, (int)pw, (int)pw, 0};
    v4i bm = {};
    if constexpr (!k6) {
      const uint32_t pm = bf16_split2(dmin) & kz;
      bm = (v4i){(int)pm, (int)pm, (int)pm, 0};
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint4 d4 = dxb[32 * t + col];
      const v4i aq = {(int)(d4.x & kz), (int)(d4.y & kz), (int)(d4.z & kz), 0};
      const v16f fz = {};
      const v16f qw = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, aq),
                                                             __builtin_bit_cast(v8bf, bw), fz, 0, 0, 0);
      if constexpr (k6) {
#pragma unroll
        for (int r = 0; r < 16; ++r) y[t][r] = fmaf(qw[r], (float)acc[t][r], y[t][r]);
      } else {
        const v16f qm = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, aq),
                                                               __builtin_bit_cast(v8bf, bm), fz, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 16; ++r) y[t][r] = fmaf(-qm[r], mn[t][r], fmaf(qw[r], (float)acc[t][r], y[t][r]));
      }
    }
    if (refill && wave == 0) dxq[(b + 1) & 1][lane] = bf16_split3(dxr);  // slot last read a superblock ago
  };

  issue(0, 0);
  if (wave == 0) {
    load_dx(0);
    dxq[0][lane] = bf16_split3(dxr);
  }
  for (int b = 0; b < nsb; b += 2) {
    step(b, ring0, 1, std::integral_constant<int, 0>{});
    if (b + 1 < nsb) step(b + 1, ring1, 0, std::integral_constant<int, k6 ? 2 : 0>{});
  }

  // both parities' partial sums -> two LDS planes (reusing the ring) -> Y
  __syncthreads();
  float* even_plane = reinterpret_cast<float*>(ring0);
  float* odd_plane = reinterpret_cast<float*>(ring1);
  tile_partials_to_lds(y, wcol, lane, h ? odd_plane : even_plane);
  __syncthreads();
  tile_store_from_lds(
      wave, lane, even_plane, odd_plane, mrows, min(kNT, a.N - n0),
      [&](int rr) {
        return a.Y + (kGroup ? group_dst_row(a.grp, m0, rr) : (long long)(m0 + rr) * a.ldy) + n0;
      },
      [](float e, float o) { return e + o; });
}

// MFMA path: prefill shapes with 4-byte aligned weight rows; Q6_K also needs
// an even number of superblocks per row (its odd records start 2 bytes into
// a dword).  The GEMV kernels take everything else.
template <KQ F>
bool gemm_kq_ok(const uint8_t* W, const void* Xq, const float* Y, size_t N, size_t K, size_t M,
                const RowStrides& st) {
  constexpr size_t kRec = KTile<F>::kRec;
  const size_t ldw = N > 1 ? st.ldw : K / 256 * kRec;
  const size_t kq = F == KQ::Q6_K ? 512 : 256;
  // below 16 activation rows only when the GEMV's LDS cannot hold a row
  return (M >= 16 || !staged_gemv_fits(F == KQ::Q6_K ? 3 : 4, K)) && N > 0 && K > 0 && K % kq == 0 &&
         W != nullptr && Xq != nullptr && Y != nullptr &&
         aligned(W, 4) && ldw % 4 == 0 && aligned(Xq, 4) && aligned(Y, 4) && N <= (size_t)INT32_MAX &&
         K <= (size_t)INT32_MAX && M <= (size_t)INT32_MAX && strides_ok(st, K / 256 * kRec, 2, K, N, N, M) &&
         ((N + kNT - 1) / kNT) * ((M + kMT - 1) / kMT) <= (size_t)INT32_MAX;
}

template <KQ F>
void gemm_kq(const uint8_t* W, const uint8_t* Xq, float* Y, size_t N, size_t K, size_t M, const RowStrides& st) {
  const size_t ldw = N > 1 ? st.ldw : K / 256 * KTile<F>::kRec;
  GemmArgs ga{W, Xq, Y, (int)N, (int)K, (int)M, ldw, (long long)st.ldy, GroupTiles{}};
  const size_t tiles = ((N + kNT - 1) / kNT) * ((M + kMT - 1) / kMT);
  kq_mfma_gemm<false, F><<<dim3((unsigned)tiles), kThreads, 0, current_stream()>>>(ga);
  check_launch(F == KQ::Q6_K ? "q6k_mfma_gemm" : "q5k_mfma_gemm");
}

}  // namespace

void mul_mat_q6k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K, size_t M,
                 const RowStrides& st) {
  if (X == nullptr || !aligned(X, 4) || !gemm_kq_ok<KQ::Q6_K>(W, Xq, Y, N, K, M, st))
    return decode_q6_k(W, X, Xq, Y, N, K, M, st);
  quantize_q8_k_rows(X, st.ldx, Xq, M, K);
  gemm_kq<KQ::Q6_K>(W, Xq, Y, N, K, M, st);
}

bool gemm_kq_try(bool q6, const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M, const RowStrides& st) {
  if (X == nullptr || !aligned(X, 4)) return false;
  if (q6) {
    if (!gemm_kq_ok<KQ::Q6_K>(W, Xq, Y, N, K, M, st)) return false;
    quantize_q8_k_rows(X, st.ldx, Xq, M, K);
    gemm_kq<KQ::Q6_K>(W, Xq, Y, N, K, M, st);
  } else {
    if (!gemm_kq_ok<KQ::Q5_K>(W, Xq, Y, N, K, M, st)) return false;
    quantize_q8_k_rows(X, st.ldx, Xq, M, K);
    gemm_kq<KQ::Q5_K>(W, Xq, Y, N, K, M, st);
  }
  return true;
}

void mul_mat_q5k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K, size_t M,
                 const RowStrides& st) {
  if (X == nullptr || !aligned(X, 4) || !gemm_kq_ok<KQ::Q5_K>(W, Xq, Y, N, K, M, st))
    return decode_q5_k(W, X, Xq, Y, N, K, M, st);
  quantize_q8_k_rows(X, st.ldx, Xq, M, K);
  gemm_kq<KQ::Q5_K>(W, Xq, Y, N, K, M, st);
}

void mul_mat_q6k_quantized(const uint8_t* W, const uint8_t* Xq, float* Y, size_t N, size_t K, size_t M,
                           const RowStrides& st) {
  if (!gemm_kq_ok<KQ::Q6_K>(W, Xq, Y, N, K, M, st))
    return decode_quantized(3, W, Xq, nullptr, nullptr, Y, N, K, M, st);
  gemm_kq<KQ::Q6_K>(W, Xq, Y, N, K, M, st);
}

void mul_mat_q5k_quantized(const uint8_t* W, const uint8_t* Xq, float* Y, size_t N, size_t K, size_t M,
                           const RowStrides& st) {
  if (!gemm_kq_ok<KQ::Q5_K>(W, Xq, Y, N, K, M, st))
    return decode_quantized(4, W, Xq, nullptr, nullptr, Y, N, K, M, st);
  gemm_kq<KQ::Q5_K>(W, Xq, Y, N, K, M, st);
}

bool mul_mat_id_kq_grouped_ok(bool q6, const uint8_t* W, size_t xq_bytes, const float* Y, size_t N, size_t K,
                              const RowStrides& st, const PairArgs& pr, int n_pairs, const void* ws,
                              size_t ws_bytes) {
  const size_t rb = K / 256 * (q6 ? kQ6_KBytes : kQ5_KBytes);
  const size_t ldw = N > 1 ? st.ldw : rb;
  return N > 0 && n_pairs > 0 && K > 0 && K % (q6 ? 512 : 256) == 0 && W != nullptr && Y != nullptr &&
         aligned(W, 4) && ldw % 4 == 0 && aligned(Y, 4) && xq_bytes < ((size_t)1 << 32) && aligned(ws, 16) &&
         ws_bytes >= moe_group_bytes(n_pairs, pr.n_as) && pr.w_es % 4 == 0 && pr.n_as <= kMaxExperts &&
         N <= (size_t)INT32_MAX && K <= (size_t)INT32_MAX && strides_ok(st, rb, 2, K, N, N, 1) &&
         (size_t)moe_tile_bound(n_pairs, pr.n_as) * ((N + kNT - 1) / kNT) <= (size_t)INT32_MAX;
}

void mul_mat_id_kq_grouped(bool q6, const uint8_t* W, const uint8_t* Xq, float* Y, size_t N, size_t K,
                           const RowStrides& st, const PairArgs& pr, int n_pairs, void* ws) {
  const MoeGroups g = moe_group(pr, n_pairs, ws);
  const size_t ldw = N > 1 ? st.ldw : K / 256 * (q6 ? kQ6_KBytes : kQ5_KBytes);
  GemmArgs ga{W, Xq, Y, (int)N, (int)K, kMT, ldw, 0, group_tiles(g, pr)};
  const size_t wgs = (size_t)g.tmax * ((N + kNT - 1) / kNT);
  if (q6) {
    kq_mfma_gemm<true, KQ::Q6_K><<<dim3((unsigned)wgs), kThreads, 0, current_stream()>>>(ga);
    check_launch("q6k_mfma_gemm");
  } else {
    kq_mfma_gemm<true, KQ::Q5_K><<<dim3((unsigned)wgs), kThreads, 0, current_stream()>>>(ga);
    check_launch("q5k_mfma_gemm");
  }
}

}  // namespace weft
