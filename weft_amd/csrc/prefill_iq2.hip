// IQ2_XXS x Q8_K prefill GEMM on int8 MFMA (production_mul_mat_iq2_xxs,
// production_mul_mat_iq2_xxs_staged; examples/kernels/mul_mat/iq2_xxs_staged.py:9-97),
// and its IQ2_XS variant (production_mul_mat_iq2_xs{,_staged};
// examples/kernels/mul_mat/iq2_xs.py:26-56, iq2_xs_staged.py:29-75).
//
//   Y[m, n] = 1/8 * sum_b dw[n,b] * dx[m,b] * sum_g ls[n,b,g] * I[m,n,b,g]
//   I = sum_{k in group g} q8[m,k] * grid[idx][j] * sign      (exact int32)
//   ls = 2 s + 1 (4-bit s)              (ggml-cpu/quants.c:855-895)
// One v_mfma_i32_32x32x32_i8 per 32x32 tile and 32-group gives I (weight
// operand bytes are +-{8, 25, 43}); the small integer group scale folds in
// with one v_mad_i32_i24 per output, exact in int32 (|I| < 2^18, ls <= 31,
// eight groups < 2^26), and the fp32 combine runs once per superblock on the
// same integer GGML converts, its factor dx dw from a bf16 outer-product
// MFMA per tile (as in the K-quant GEMMs).
//
// Tiling as in the Q4_K prefill: 64 tokens x 128 weight rows per workgroup,
// 8 waves (superblock parity x 4 column groups), each wave two 32x32 tiles.
// A 66-byte record is only 2-byte aligned, so the weight rows of a superblock
// PAIR (132 bytes, 4-byte aligned when K/256 is even) are staged together,
// each parity's record in a 16-byte aligned segment of its own (Tile
// below); a parity reads its group bytes with five 16-byte LDS reads and
// byte alignment.
// Grid and sign tables live in LDS, the signs as byte masks (0xff per -1).
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
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void* lds_ptr;

constexpr int kMT = 64;        // tokens per workgroup tile
constexpr int kNT = 128;       // weight rows per workgroup tile
constexpr int kThreads = 512;  // 8 waves: 4 column groups x 2 superblock parities
constexpr int kAQ = kMT * 256;                    // activation int8 of one superblock

// Per format (kXs: IQ2_XS, else IQ2_XXS): record bytes and the weight tile
// of a superblock pair (4-byte aligned: 132 / 148 bytes per row).  A row's
// pair is 11 chunks of 16 bytes in LDS (176-byte stride: 16 lanes' 16-byte
// reads fall on all 64 banks), each copied by a 16-byte direct load from a
// 4-byte aligned source (P: the pair's first byte in the row, R = kRec):
//   chunks 0-4   bytes P + 16 c          record 0 from its first byte (d, then
//                                         its group bytes at 2 + 8 g)
//   chunks 5-8   bytes P + R + 2 + 16 j  record 1's group bytes from byte 0
//   chunk 9      IQ2_XS: P + R + 58      record 1's scales at bytes 8-15
//                IQ2_XXS: as chunk 10
//   chunk 10     bytes P + R - 2         record 1's d at bytes 2-3
// so both parities take group g's words from dwords 2g .. 2g + 2 of their
// five chunks, shifted by 2 bytes (parity 0) or 0 (parity 1).
template <bool kXs>
struct Tile {
  static constexpr int kRec = kXs ? kIq2xsBytes : kIq2xxsBytes;  // 74 / 66
  static constexpr int kPairB = 2 * kRec;
  static constexpr int kRowL = 176;                             // LDS bytes per weight row and pair
  static constexpr int kCh = kRowL / 16;                        // 11 chunks
  static constexpr int kW16 = kNT * kCh / 64;                   // 22 wave-wide 16-byte loads
  static constexpr int kWT = kNT * kRowL;                       // 22528
  static constexpr int kSlot = 2 * kAQ + kWT;                   // one ring slot: both parities + weights
  static constexpr int kSlotAlloc = kSlot + 16;
  static_assert((!kXs || kRec + 58 + 16 <= kPairB) && kRec + 66 <= kPairB && 80 <= kPairB &&
                    kNT * kCh % 64 == 0,
                "chunks within the pair");
  static constexpr int kGrid = kXs ? 512 : 256;                 // grid entries
  static_assert(kTilePlaneBytes <= kSlot, "an output plane fits one ring slot");
};

struct GemmArgs {
  const uint8_t* W;
  const uint8_t* Xq;
  const int8_t* grid;   // 256 x 8
  const int8_t* signs;  // 128 x 8 (+-1)
  float* Y;
  int N, K, M;
  size_t ldw;     // bytes between weight rows
  long long ldy;  // floats between output rows
  GroupTiles grp;  // grouped (MUL_MAT_ID) mode
};

// Direct global->LDS loads; lane l writes [lds + size*l, +size).  Inline asm
// keeps the compiler from making unrelated LDS reads wait for them; the
// kernel waits (s_waitcnt) itself.  Nothing else in this kernel uses M0.
// `lds` is wave-uniform; readfirstlane states it, so it is an SGPR operand
// in every instantiation.
__device__ __forceinline__ void lds_dma16(const uint8_t* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(g)
               : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_ptr)p;
}
__device__ __forceinline__ uint32_t ld32(const uint8_t* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}
// An empty asm that claims to modify v: the optimizer cannot re-associate a
// running sum through it.  Used on the eight-group sum, which it would
// otherwise turn into a tree holding every group's 16-register product tile
// live.  (It emits nothing, so the compiler still places the wait states a
// VALU read of an MFMA result needs.)
__device__ __forceinline__ void pin(int& v) { asm volatile("" : "+v"(v)); }
// negate the bytes of g whose mask byte in m is 0xff (the sign table is
// staged in LDS as byte masks: 0xff where the +-1 byte is -1): for a byte
// b != 0, (b ^ 0xff) + 1 = 256 - b never carries into the next byte (GGML's
// grid magnitudes are 8, 25 and 43)
__device__ __forceinline__ uint32_t apply_signs(uint32_t g, uint32_t m) {
  return (g ^ m) + (m & 0x01010101u);
}
// one operand's sixteen weight bytes (grid rows g0, g1 against sign rows
// z0, z1): the masks' negate, or, for tables outside its precondition, the
// i8 products of grid and sign bytes.  `canon` is wave-uniform; the branch
// keeps the rare path off the common one.
__device__ __forceinline__ v4i weight_bytes(uint2 g0, uint2 g1, uint2 z0, uint2 z1, bool canon) {
  v4i bv;
  if (__builtin_expect(canon, 1)) {
    bv = (v4i){(int)apply_signs(g0.x, z0.x), (int)apply_signs(g0.y, z0.y), (int)apply_signs(g1.x, z1.x),
               (int)apply_signs(g1.y, z1.y)};
  } else {
    bv = (v4i){(int)mul8x4(g0.x, z0.x), (int)mul8x4(g0.y, z0.y), (int)mul8x4(g1.x, z1.x),
               (int)mul8x4(g1.y, z1.y)};
  }
  return bv;
}

// kXs (IQ2_XS, ggml-cpu/quants.c:897-946): u16 entries (grid row bits 0-8,
// sign row bits 9-15) and a 4-bit scale per 16-element half, s_lo for
// entries 0-1 and s_hi for 2-3 of each 32-group (scale byte 66 + g).  A
// 32-group's MFMA runs twice with the weight operand of one half (the lanes
// kg of the other half hold zeros), and each product tile takes its half's
// 2 s + 1 in the same exact int32 multiply-add.
template <bool kGroup, bool kXs = false>
__global__ void __launch_bounds__(kThreads, 1) iq2_mfma_gemm(GemmArgs a) {
  using TT = Tile<kXs>;
  constexpr int kPairB = TT::kPairB;
  __shared__ __align__(16) uint8_t ring0[TT::kSlotAlloc];
  __shared__ __align__(16) uint8_t ring1[TT::kSlotAlloc];
  // [slot][parity][token]: the token's Q8_K d as the bf16 parts of the
  // outer-product factor MFMA ((h,h), (m,m), (l,l), 0)
  __shared__ __align__(16) uint4 dxq[2][2][kMT];
  __shared__ __align__(16) uint8_t tgrid[TT::kGrid * 8];
  __shared__ __align__(16) uint8_t tsign[128 * 8];  // sign rows as byte masks
  __shared__ __align__(16) uint8_t traw[128 * 8];   // sign rows as given
  __shared__ uint32_t tflag[kThreads / 64];          // per wave: a table byte outside the masks' precondition

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int par = wave >> 2, wcol = wave & 3;
  const int col = lane & 31, kg = lane >> 5;
  const int nsb = a.K >> 8;
  const int npair = nsb >> 1;  // nsb is even on this path
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

  // activation int8 of superblock 2*pair + par: 16 wave-wide 16-byte loads, 4 per wave
  const uint8_t* asrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = wcol + 4 * i;
    const int q = 64 * k + lane, r = q >> 4, c = (q & 15) ^ (r & 15);
    asrc[i] = a.Xq + (size_t)act_row(min(r, mrows - 1)) * xrb + 4 + 16 * c;
  }
  const uint8_t* dsrc = a.Xq + (size_t)act_row(min(lane, mrows - 1)) * xrb;  // Q8_K d of token lane

  // LDS byte addresses of the two ring slots, formed once from wave-uniform
  // pointers (no per-load generic-to-LDS casts)
  const uint32_t ring_lds[2] = {(uint32_t)__builtin_amdgcn_readfirstlane(lds_addr(ring0)),
                                (uint32_t)__builtin_amdgcn_readfirstlane(lds_addr(ring1))};
  // weight chunk q = 64 k + lane of load k = wave + 8 i (< 22): row q / 11,
  // chunk q % 11 at the byte offsets of the layout above
  uint32_t wv[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int q = 64 * min(wave + 8 * i, TT::kW16 - 1) + lane, row = q / TT::kCh, c = q - TT::kCh * row;
    const int off = c < 5 ? 16 * c : c < 9 ? TT::kRec + 2 + 16 * (c - 5) : (kXs && c == 9) ? TT::kRec + 58 : TT::kRec - 2;
    wv[i] = (uint32_t)min(row, a.N - 1 - n0) * (uint32_t)wrb + (uint32_t)off;
  }
  const uint8_t* wtile = W + (size_t)n0 * wrb;
  auto issue = [&](int pair, uint8_t* ring) {
    const int b = 2 * pair + par;
    const uint32_t base = ring == ring0 ? ring_lds[0] : ring_lds[1];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      lds_dma16(asrc[i] + (size_t)b * kQ8_KBytes, base + par * kAQ + 1024 * (wcol + 4 * i));
#pragma unroll
    for (int i = 0; i < (TT::kW16 + 7) / 8; ++i)
      if (wave + 8 * i < TT::kW16)
        lds_dma16(wtile + (size_t)pair * kPairB + wv[i], base + 2 * kAQ + 1024 * (wave + 8 * i));
  };
  float dxr = 0.f;
  auto load_dx = [&](int pair) {
    dxr = *reinterpret_cast<const float*>(dsrc + (size_t)(2 * pair + par) * kQ8_KBytes);
  };

  v16i I[2], I2[2], acc[2];
  v16f y[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) y[t][r] = 0.f;
  const v16i zero = {};
  const int sw = col & 15;

  auto step = [&](int pair, const uint8_t* cur, uint8_t* nxt) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of this pair have landed
    __syncthreads();                // everyone's; the previous pair is consumed
    // every wave has flagged its table words (before the first of these
    // barriers): canon = the sign masks' negate; otherwise (tables outside
    // its precondition) the i8 products of grid and sign bytes, on a scalar
    // branch around the operand's four words only
    const bool canon = iq2_flags_clear(tflag, kThreads / 64);
    const uint8_t* tsg = canon ? tsign : traw;
    const bool refill = pair + 1 < npair;
    if (refill && wcol == 0) load_dx(pair + 1);
    const uint8_t* AQ = cur + par * kAQ;
    const uint8_t* wrow = cur + 2 * kAQ + (32 * wcol + col) * TT::kRowL;
    const uint8_t* seg = wrow + 80 * par;  // this parity's five chunks
    const uint4* dxb = &dxq[pair & 1][par][0];
    // fp16 d: bytes 0-1 of chunk 0 (parity 0) or 2-3 of chunk 10 (parity 1)
    const uint32_t dword0 = ld32(par ? wrow + 160 : wrow);
    const float dw = fp16_to_fp32(par ? dword0 >> 16 : dword0 & 0xffffu);
    const int sh = 2 - 2 * par;  // byte offset of the group bytes in their dwords
    // IQ2_XS: the 8 scale bytes, at bytes 66-73 of parity 0's chunks and
    // 8-15 of parity 1's chunk 9 (dwords 16-18 / 18-19, shift sh)
    uint32_t scl0 = 0, scl1 = 0;
    if constexpr (kXs) {
      const uint8_t* sbase = seg + 64 + 8 * par;
      const uint32_t s0w = ld32(sbase), s1w = ld32(sbase + 4), s2w = ld32(sbase + 8);
      scl0 = __builtin_amdgcn_alignbyte(s1w, s0w, sh);
      scl1 = __builtin_amdgcn_alignbyte(s2w, s1w, sh);
    }
    // Groups G0 .. G0 + 3, from the segment's dwords 2 G0 .. 2 G0 + 8
    // (16-byte reads G0 / 2 .. G0 / 2 + 2).  A pair is groups 0-3, then this
    // wave's share of the next pair's direct loads, then groups 4-7: issued
    // right after the barrier, every wave's first group waited behind the
    // workgroup's queued loads (the MXFP4 GEMM measured 39.5 -> 37.8 us per
    // call for the move).
    auto groups = [&](auto g0_tag) {
      constexpr int G0 = decltype(g0_tag)::value;
      uint32_t wq[20];
#pragma unroll
      for (int i = G0 / 2; i < G0 / 2 + 3; ++i) {
        const uint4 v = *reinterpret_cast<const uint4*>(seg + 16 * i);
        wq[4 * i] = v.x, wq[4 * i + 1] = v.y, wq[4 * i + 2] = v.z, wq[4 * i + 3] = v.w;
      }
#pragma unroll
      for (int g = G0; g < G0 + 4; ++g) {
        if constexpr (kXs) {
          const uint32_t w0 = wq[2 * g], w1 = wq[2 * g + 1], w2 = wq[2 * g + 2];
          // this lane's 16 elements: entries 2kg, 2kg + 1 = one u16 pair
          const uint32_t ew = kg ? __builtin_amdgcn_alignbyte(w2, w1, sh) : __builtin_amdgcn_alignbyte(w1, w0, sh);
          const uint32_t e0 = ew & 0xffffu, e1 = ew >> 16;
          const uint2 g0 = *reinterpret_cast<const uint2*>(tgrid + 8 * (e0 & 511u));
          const uint2 g1 = *reinterpret_cast<const uint2*>(tgrid + 8 * (e1 & 511u));
          const uint2 z0 = *reinterpret_cast<const uint2*>(tsg + 8 * (e0 >> 9));
          const uint2 z1 = *reinterpret_cast<const uint2*>(tsg + 8 * (e1 >> 9));
          const v4i bv = weight_bytes(g0, g1, z0, z1, canon);
          const v4i bz = {};
          const uint32_t sb = ((g < 4 ? scl0 : scl1) >> (8 * (g & 3))) & 0xffu;
          const int ls_lo = 2 * (int)(sb & 15u) + 1, ls_hi = 2 * (int)(sb >> 4) + 1;
          const int chunk = (2 * g + kg) ^ sw;
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
              int v = __mul24(I[t][r], ls_lo) + __mul24(I2[t][r], ls_hi) + (g == 0 ? 0 : acc[t][r]);
              pin(v);
              acc[t][r] = v;
            }
          continue;
        }
        const uint32_t w0 = wq[2 * g], w1 = wq[2 * g + 1], w2 = wq[2 * g + 2];
        const uint32_t idx = __builtin_amdgcn_alignbyte(w1, w0, sh);   // 4 grid indices
        const uint32_t meta = __builtin_amdgcn_alignbyte(w2, w1, sh);  // 4 x 7-bit signs, 4-bit s
        // this lane's 16 elements: grid entries l = 2kg, 2kg+1 (8 elements each)
        const uint32_t i0 = (idx >> (16 * kg)) & 0xffu, i1 = (idx >> (16 * kg + 8)) & 0xffu;
        const uint32_t s0 = (meta >> (14 * kg)) & 127u, s1 = (meta >> (14 * kg + 7)) & 127u;
        const uint2 g0 = *reinterpret_cast<const uint2*>(tgrid + 8 * i0);
        const uint2 g1 = *reinterpret_cast<const uint2*>(tgrid + 8 * i1);
        const uint2 z0 = *reinterpret_cast<const uint2*>(tsg + 8 * s0);
        const uint2 z1 = *reinterpret_cast<const uint2*>(tsg + 8 * s1);
        const v4i bv = weight_bytes(g0, g1, z0, z1, canon);
        const int ls = 2 * (int)(meta >> 28) + 1;
        const int chunk = (2 * g + kg) ^ sw;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const v4i av = *reinterpret_cast<const v4i*>(AQ + (32 * t + col) * 256 + 16 * chunk);
          I[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, zero, 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            int v = __mul24(I[t][r], ls) + (g == 0 ? 0 : acc[t][r]);
            pin(v);
            acc[t][r] = v;
          }
      }
    };
    groups(std::integral_constant<int, 0>{});
    if (refill) issue(pair + 1, nxt);
    groups(std::integral_constant<int, 4>{});
    // y += (dx dw) acc: the factor of every output from a bf16 outer-product
    // MFMA per tile (token d = h + m + l against the row's fp16 dw = f_h +
    // f_l in K slots 0-5 of the kg = 0 lanes), then two VALU operations per
    // output
    const uint32_t kz = kg ? 0u : 0xffffffffu;
    const uint32_t pw = bf16_split2(dw) & kz;
    const v4i bw = {(int)pw, (int)pw, (int)pw, 0};
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint4 d4 = dxb[32 * t + col];
      const v4i aq = {(int)(d4.x & kz), (int)(d4.y & kz), (int)(d4.z & kz), 0};
      const v16f fz = {};
      const v16f qw = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, aq),
                                                             __builtin_bit_cast(v8bf, bw), fz, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 16; ++r) y[t][r] = fmaf(qw[r], (float)acc[t][r], y[t][r]);
    }
    if (refill && wcol == 0) dxq[(pair + 1) & 1][par][lane] = bf16_split3(dxr);  // slot last read a pair ago
  };

  issue(0, ring0);
  // the tables after the first stage's loads: their round trip overlaps it.
  // `bad` marks a grid byte of 0 or a sign byte other than +-1 (weft_common.h)
  bool bad = false;
  for (int i = tid; i < TT::kGrid * 8; i += kThreads) {
    const int8_t gb = a.grid[i];
    tgrid[i] = (uint8_t)gb;
    bad |= gb == 0;
  }
  for (int i = tid; i < 128 * 8; i += kThreads) {
    const int8_t sb = a.signs[i];
    tsign[i] = sb < 0 ? 0xffu : 0u;  // byte masks
    traw[i] = (uint8_t)sb;
    bad |= sb != 1 && sb != -1;
  }
  iq2_flag_wave(tflag, bad);  // read after the first pair's barrier (the same in every workgroup)
  if (wcol == 0) {
    load_dx(0);
    dxq[0][par][lane] = bf16_split3(dxr);
  }
  for (int pair = 0; pair < npair; pair += 2) {
    step(pair, ring0, ring1);
    if (pair + 1 < npair) step(pair + 1, ring1, ring0);
  }

  // both parities' partial sums -> two LDS planes (reusing the ring) -> Y
  __syncthreads();
  float* even_plane = reinterpret_cast<float*>(ring0);
  float* odd_plane = reinterpret_cast<float*>(ring1);
  tile_partials_to_lds(y, wcol, lane, par ? odd_plane : even_plane);
  __syncthreads();
  tile_store_from_lds(
      wave, lane, even_plane, odd_plane, mrows, min(kNT, a.N - n0),
      [&](int rr) {
        return a.Y + (kGroup ? group_dst_row(a.grp, m0, rr) : (long long)(m0 + rr) * a.ldy) + n0;
      },
      [](float e, float o) { return 0.125f * (e + o); });
}


template <bool kXs = false>
bool gemm_iq2_ok(const uint8_t* W, const void* Xq, const float* Y, const int8_t* grid,
                 const int8_t* signs, size_t N, size_t K, size_t M, const RowStrides& st) {
  // MFMA path: prefill shapes with an even number of superblocks per row and
  // 4-byte aligned weight rows whose tile of 128 rows stays within 32-bit
  // offsets; the GEMV kernels take everything else
  constexpr size_t kRec = Tile<kXs>::kRec;
  const size_t ldw = N > 1 ? st.ldw : K / 256 * kRec;
  // (below 16 activation rows only when the GEMV's LDS cannot hold a row)
  return (M >= 16 || !staged_gemv_fits(kXs ? 7 : 2, K)) && N > 0 && K > 0 && K % 512 == 0 &&
         W != nullptr && Xq != nullptr &&
         Y != nullptr && grid != nullptr && signs != nullptr && aligned(W, 4) && ldw % 4 == 0 &&
         (kNT - 1) * ldw + K / 256 * kRec < ((size_t)1 << 32) &&
         aligned(Xq, 4) && aligned(Y, 4) && N <= (size_t)INT32_MAX && K <= (size_t)INT32_MAX &&
         M <= (size_t)INT32_MAX && strides_ok(st, K / 256 * kRec, 2, K, N, N, M) &&
         ((N + kNT - 1) / kNT) * ((M + kMT - 1) / kMT) <= (size_t)INT32_MAX;
}

template <bool kXs = false>
void gemm_iq2(const uint8_t* W, const uint8_t* Xq, const int8_t* grid, const int8_t* signs, float* Y,
              size_t N, size_t K, size_t M, const RowStrides& st) {
  const size_t ldw = N > 1 ? st.ldw : K / 256 * Tile<kXs>::kRec;
  GemmArgs ga{W, Xq, grid, signs, Y, (int)N, (int)K, (int)M, ldw, (long long)st.ldy, GroupTiles{}};
  const size_t tiles = ((N + kNT - 1) / kNT) * ((M + kMT - 1) / kMT);
  iq2_mfma_gemm<false, kXs><<<dim3((unsigned)tiles), kThreads, 0, current_stream()>>>(ga);
  check_launch(kXs ? "iq2xs_mfma_gemm" : "iq2_mfma_gemm");
}

}  // namespace

bool mul_mat_id_iq2_grouped_ok(bool xs, const uint8_t* W, size_t xq_bytes, const float* Y, const int8_t* grid,
                               const int8_t* signs, size_t N, size_t K, const RowStrides& st,
                               const PairArgs& pr, int n_pairs, const void* ws, size_t ws_bytes) {
  const size_t rb = K / 256 * (xs ? kIq2xsBytes : kIq2xxsBytes);
  const size_t ldw = N > 1 ? st.ldw : rb;
  return N > 0 && n_pairs > 0 && K > 0 && K % 512 == 0 && W != nullptr && Y != nullptr &&
         grid != nullptr && signs != nullptr && aligned(W, 4) && ldw % 4 == 0 &&
         (kNT - 1) * ldw + rb < ((size_t)1 << 32) && aligned(Y, 4) &&
         xq_bytes < ((size_t)1 << 32) && aligned(ws, 16) && ws_bytes >= moe_group_bytes(n_pairs, pr.n_as) &&
         pr.w_es % 4 == 0 && pr.n_as <= kMaxExperts && N <= (size_t)INT32_MAX && K <= (size_t)INT32_MAX &&
         strides_ok(st, rb, 2, K, N, N, 1) &&
         (size_t)moe_tile_bound(n_pairs, pr.n_as) * ((N + kNT - 1) / kNT) <= (size_t)INT32_MAX;
}

void mul_mat_id_iq2_grouped(bool xs, const uint8_t* W, const uint8_t* Xq, const int8_t* grid, const int8_t* signs,
                            float* Y, size_t N, size_t K, const RowStrides& st, const PairArgs& pr,
                            int n_pairs, void* ws) {
  const MoeGroups g = moe_group(pr, n_pairs, ws);
  const size_t ldw = N > 1 ? st.ldw : K / 256 * (xs ? kIq2xsBytes : kIq2xxsBytes);
  GemmArgs ga{W, Xq, grid, signs, Y, (int)N, (int)K, kMT, ldw, 0, group_tiles(g, pr)};
  const size_t wgs = (size_t)g.tmax * ((N + kNT - 1) / kNT);
  if (xs) {
    iq2_mfma_gemm<true, true><<<dim3((unsigned)wgs), kThreads, 0, current_stream()>>>(ga);
    check_launch("iq2xs_mfma_gemm");
  } else {
    iq2_mfma_gemm<true><<<dim3((unsigned)wgs), kThreads, 0, current_stream()>>>(ga);
    check_launch("iq2_mfma_gemm");
  }
}

bool gemm_iq2_try(bool xs, const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid,
                  const int8_t* signs, float* Y, size_t N, size_t K, size_t M, const RowStrides& st) {
  if (X == nullptr || !aligned(X, 4)) return false;
  if (xs) {
    if (!gemm_iq2_ok<true>(W, Xq, Y, grid, signs, N, K, M, st)) return false;
    quantize_q8_k_rows(X, st.ldx, Xq, M, K);
    gemm_iq2<true>(W, Xq, grid, signs, Y, N, K, M, st);
  } else {
    if (!gemm_iq2_ok(W, Xq, Y, grid, signs, N, K, M, st)) return false;
    quantize_q8_k_rows(X, st.ldx, Xq, M, K);
    gemm_iq2(W, Xq, grid, signs, Y, N, K, M, st);
  }
  return true;
}

void mul_mat_iq2_xxs(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid,
                     const int8_t* signs, float* Y, size_t N, size_t K, size_t M,
                     const RowStrides& st) {
  if (X == nullptr || !aligned(X, 4) || !gemm_iq2_ok(W, Xq, Y, grid, signs, N, K, M, st))
    return decode_iq2_xxs(W, X, Xq, grid, signs, Y, N, K, M, st);
  quantize_q8_k_rows(X, st.ldx, Xq, M, K);
  gemm_iq2(W, Xq, grid, signs, Y, N, K, M, st);
}

// IQ2_XS: the same GEMM with per-half scales (M >= 16, K % 512 == 0), the GEMV otherwise
void mul_mat_iq2_xs(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid, const int8_t* signs,
                    float* Y, size_t N, size_t K, size_t M, const RowStrides& st) {
  if (X == nullptr || !aligned(X, 4) || !gemm_iq2_ok<true>(W, Xq, Y, grid, signs, N, K, M, st))
    return decode_iq2_xs(W, X, Xq, grid, signs, Y, N, K, M, st);
  quantize_q8_k_rows(X, st.ldx, Xq, M, K);
  gemm_iq2<true>(W, Xq, grid, signs, Y, N, K, M, st);
}

void mul_mat_iq2_xs_quantized(const uint8_t* W, const uint8_t* Xq, const int8_t* grid, const int8_t* signs,
                              float* Y, size_t N, size_t K, size_t M, const RowStrides& st) {
  if (!gemm_iq2_ok<true>(W, Xq, Y, grid, signs, N, K, M, st))
    return decode_quantized(7, W, Xq, grid, signs, Y, N, K, M, st);
  gemm_iq2<true>(W, Xq, grid, signs, Y, N, K, M, st);
}

void mul_mat_iq2_xxs_quantized(const uint8_t* W, const uint8_t* Xq, const int8_t* grid,
                               const int8_t* signs, float* Y, size_t N, size_t K, size_t M,
                               const RowStrides& st) {
  if (!gemm_iq2_ok(W, Xq, Y, grid, signs, N, K, M, st))
    return decode_quantized(2, W, Xq, grid, signs, Y, N, K, M, st);
  gemm_iq2(W, Xq, grid, signs, Y, N, K, M, st);
}

}  // namespace weft
