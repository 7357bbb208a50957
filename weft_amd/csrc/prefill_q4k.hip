// Q4_K x Q8_K prefill GEMM on MFMA (production_mul_mat_q4_k_staged,
// production_mul_mat_q4_k; examples/kernels/mul_mat/q4_k_staged.py:9-37).
//
//   Y[m, n] = sum_b dx[m,b] * (dw[n,b] * S[m,n,b] - dmin[n,b] * Mn[m,n,b])
//   S  = sum_s sc[n,b,s] * sum_{k in s} q8[m,k] * q4[n,k]     (exact int32)
//   Mn = sum_j m[n,b,j/2] * bsum[m,b,j], j = 0..15            (exact)
//
// S on int8 MFMA.  The 6-bit sub-block scale sc does not fit an int8 operand
// once multiplied by a nibble (sc*q <= 945), and applying it per sub-block on
// VALU costs one instruction per output per 32 products.  So the scale is
// split, sc = 8a + b with a, b in [0, 7], and every product stays an exact
// int8 x int8 term: two accumulators per output over each superblock,
//   lo = sum_k q8 * (q * b_s),   hi = sum_k q8 * (q * a_s),   S = lo + 8 hi.
// v_mfma_i32_32x32x32_i8 has K = 32 = one sub-block, so a sub-block's weight
// operand is its nibbles times a per-column constant (v_pk_mul_lo_u16 on
// packed bytes: 105*256+105 < 2^16).
//
// Mn on one f16 MFMA per superblock and 32x32 tile.  Q8_K's 16 bsums are
// sums of 16 int8 (|bsum| <= 2032 < 2^11) and the mins are 6-bit, so both
// are exact f16 operands and v_mfma_f32_32x32x16_f16 (K = 16 = the bsums)
// returns Mn exactly in fp32 (|Mn| <= 2.05e6 < 2^24).  The token scale times
// the column scale, Q = dx * f, comes from one bf16 MFMA per tile as an outer
// product: dx = h + m + l (three bf16, to 2^-24) against f = f_h + f_l (an
// fp16 value is exactly two bf16), six exact products summed in fp32.  Once
// per superblock every output then takes
//   D = (lo + 8 hi) - r * Mn,   y += Q * D
// with f = dw, r = dmin / dw; a superblock with dw == 0 zeroes its sc
// operands (S = 0) and uses f = dmin, r = 1.  The rounding of D, r and Q
// stays within 2^-21 of |dw S| + |dmin Mn|, far inside the tolerance.
//
// Tiling: a workgroup computes 64 (tokens) x 128 (weight rows) with 8 MFMA
// waves and 2 loader waves.  MFMA waves 0-3 take the even superblocks and
// 4-7 the odd ones; wave w owns weight rows 32*(w%4)..+31 for all 64 tokens
// (two 32x32 tiles sharing one weight operand).  The loader waves stage the
// next superblock pair into LDS by direct global->LDS loads
// (global_load_lds_dwordx4, SGPR base + per-lane constant offset) while the
// MFMA waves compute the current one, so no MFMA wave ever issues or waits on
// a global memory instruction.  Once a pair has landed, each loader rewrites
// its stage's per-token data in place, once for all four column groups: the
// bsums become f16 and the token scale becomes the outer product's bf16
// operand.  One barrier per pair hands the filled ring slots over.  At the
// end both parities' partial sums meet in LDS and every output is written
// once, even + odd, with 16-byte stores (tile_store.h).
//
// Launch: at most one workgroup per CU (the ring takes its LDS), each walking
// a share of the tiles.  The pairs of a workgroup's tiles form one stream
// through the ring, so the next tile's first superblocks load while the
// current tile finishes and stores (measured at 512 x 4096 x 11008: a
// tile's K loop takes 18-19.5 us and its output stage ~1.9 us; only a
// workgroup's first tile waits for its first pair, ~2.9 us).
//
// LDS per superblock stage (38,912 B; 2 pairs = 4 stages):
//   AQ  64 rows x 17 16-byte chunks: the 16 chunks of qs, then one pad chunk,
//       so row r starts at 272 r and the 8 lanes of an A-operand read (8
//       consecutive rows, one chunk) hit distinct banks with immediate offsets
//   AX  64 rows x 3 chunks: record bytes [0,16) (d), [260,276), [276,292)
//       (bsums), rewritten in place as described above
//   WT  128 rows x the 144-byte Q4_K record
// The activation is quantized first, into the caller's Xq, by q8_K_quantize's
// kernel (Xq is part of the ABI), then read back from L2.
//
// Grouped mode (kGroup, GGML's MUL_MAT_ID, ggml-cpu/ggml-cpu.c:1454-1698):
// the (token, slot) pairs are grouped by expert on the device
// (moe_group_kernel: a pair list per expert and a table of 64-row tiles), and
// each (tile, column block) runs the same GEMM on its tile's pairs: the
// loader gathers their activation rows through the pair list, W is the
// tile's expert matrix, and each output goes to the pair's dst row.  The
// workgroups walk the device's tile count (launched for the host's bound).
#include <algorithm>
#include <cstdio>

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
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_ptr;

constexpr int kLoaders = 2;                    // loader waves, one per parity
constexpr int kAQRow = 272;                    // 16 qs chunks + 1 pad chunk
constexpr int kCohortBlock = 16 * kQ4_KBytes;  // 2304: one superblock of a 16-row interleaved cohort

constexpr int round_kb(int b) { return (b + 1023) / 1024 * 1024; }

// A workgroup tile of kMT tokens x kNT weight rows (kMT 32 or 64, kNT 64 or
// 128): kNT / 32 column groups x 2 superblock parities of MFMA waves, each
// wave kMT tokens x 32 rows (kMT / 32 accumulator tiles sharing one weight
// operand), and the two loader waves.  The default and fastest at prefill
// sizes is 64 x 128; the others serve CompileOptions.meta's MC / NC and
// small M.
template <int kMT_, int kNT_>
struct Tiling {
  static constexpr int kMT = kMT_;
  static constexpr int kNT = kNT_;
  static constexpr int kCols = kNT / 32;          // column groups
  static constexpr int kT2 = kMT / 32;            // token tiles per wave
  static constexpr int kMfmaWaves = 2 * kCols;
  static constexpr int kThreads = 64 * (kMfmaWaves + kLoaders);
  static constexpr int kAQ = round_kb(kMT * kAQRow);  // 17408 at 64 tokens
  static constexpr int kAX = round_kb(kMT * 48);      // 3072
  static constexpr int kWT = kNT * kQ4_KBytes;        // 18432 at 128 rows
  static constexpr int kStage = kAQ + kAX + kWT;      // 38912
  static constexpr int kAQSlots = kAQ / 1024;
  static constexpr int kAXSlots = kAX / 1024;
  static constexpr int kSlots = kStage / 1024;        // wave-wide 1 KB loads per superblock
  static constexpr int kPlaneBytes = tile_plane_bytes<kMT, kNT>();
  static_assert((kMT == 32 || kMT == 64) && (kNT == 64 || kNT == 128), "supported tilings");
  static_assert(kWT == (kNT / 16) * kCohortBlock, "a weight stage is whole cohort blocks");
  static_assert(kWT % 1024 == 0, "every region is a whole number of wave loads");
  static_assert(2 * kPlaneBytes <= 2 * kStage, "the output planes fit one ring slot");
};
typedef Tiling<64, 128> DefaultTiling;

struct GemmArgs {
  const uint8_t* W;
  const uint8_t* Xq;
  float* Y;
  int N, K, M;
  uint32_t ldw;   // bytes between weight rows (a tile's 128 rows stay in 32-bit offsets)
  long long ldy;  // floats between output rows
  GroupTiles grp;  // grouped (MUL_MAT_ID) mode
};

// One 64 x 128 output tile: first activation row (grouped: pair-list index),
// activation rows present, first weight row, weight byte offset (grouped:
// the expert's matrix).
struct Tile {
  int m0, mrows, n0;
  long long w_off;
};

// Direct global->LDS load of 16 bytes per lane: lane l reads sbase + voff
// and writes LDS bytes [lds + 16 l, lds + 16 l + 16) (lds wave-uniform).
// Inline asm: the loader waves wait for these loads themselves (s_waitcnt
// vmcnt(0) before the step barrier).  One wait state separates the M0 write
// from the load that reads it; nothing else in this kernel uses M0.
__device__ __forceinline__ void lds_dma16(const uint8_t* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds), "v"(voff), "s"(sbase)
               : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_ptr)p;
}

// two int16 (one dword) -> two f16, exact for |v| <= 2048
__device__ __forceinline__ uint32_t i16x2_to_f16x2(uint32_t w) {
  const v2h h = {(_Float16)(short)(w & 0xffffu), (_Float16)(short)(w >> 16)};
  return __builtin_bit_cast(uint32_t, h);
}

// byte i of w (a 6-bit min) twice, as two f16
__device__ __forceinline__ uint32_t dup_byte_f16x2(uint32_t w, int i) {
  // v_perm: bytes [w.i, 0x64, w.i, 0x64] -> halves 0x6400 + m = 1024 + m
  const uint32_t sel = (uint32_t)i | (4u << 8) | ((uint32_t)i << 16) | (4u << 24);
  const uint32_t biased = __builtin_amdgcn_perm(0x64646464u, w, sel);
  const v2h h = __builtin_bit_cast(v2h, biased) - (v2h){(_Float16)1024.f, (_Float16)1024.f};
  return __builtin_bit_cast(uint32_t, h);
}

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));


// Eight bytes of row (lane % 16) from eight consecutive 16-byte lines of an
// interleaved cohort block: lane i of each 16-lane group addresses byte 8 i
// of the group's 128-byte window and receives row i's byte from each line.
__device__ __forceinline__ uint2 tr8(uint32_t lds_byte_addr) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  typedef __attribute__((address_space(3))) v2i lds_v2i;
  const v2i v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(size_t)lds_byte_addr);
  return make_uint2((uint32_t)v.x, (uint32_t)v.y);
}

// kIlv: W is the 16-row interleave Q4K_I[16] (superblock b of rows 16c ..
// 16c + 15 is the 2304-byte block (c * nsb + b) * 2304 whose byte 16 j + r is
// byte j of row 16c + r's record).  A stage then holds the tile's eight
// cohort blocks as they lie in memory, and each MFMA wave reads its rows'
// header and nibble bytes transposed (tr8); everything else is the same.
template <bool kGroup, bool kIlv = false, class TL = DefaultTiling>
__global__ void __launch_bounds__(TL::kThreads, 1) q4k_mfma_gemm(GemmArgs a) {
  constexpr int kMT = TL::kMT, kNT = TL::kNT, kCols = TL::kCols, kT2 = TL::kT2;
  constexpr int kMfmaWaves = TL::kMfmaWaves, kStage = TL::kStage;
  constexpr int kAQ = TL::kAQ, kAX = TL::kAX, kAQSlots = TL::kAQSlots, kAXSlots = TL::kAXSlots;
  constexpr int kSlots = TL::kSlots;
  static_assert(!kGroup || (kMT == 64 && kNT == 128), "grouped mode runs the 64 x 128 tile");
  __shared__ __align__(16) uint8_t ring[4 * kStage];  // [pair slot][parity]
  __shared__ __align__(16) uint32_t zero16[4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  if (tid < 4) zero16[tid] = 0u;
  // Tile t of the launch: m-tile fastest (dense) or expert tile fastest
  // (grouped: m0 then indexes the pair list, and the tiles are the device's
  // tile count, not the host's bound, so the schedule below spreads only real
  // tiles).  Every wave enumerates the same tiles.
  const int ntn = (a.N + kNT - 1) / kNT;
  const int ntm =
      kGroup ? min(__builtin_amdgcn_readfirstlane(*a.grp.ntiles), a.grp.tmax) : (a.M + kMT - 1) / kMT;
  auto tile_info = [&](int t, Tile& ti) -> bool {
    if constexpr (kGroup) {
      if (!group_tile(a.grp, t % ntm, ti.m0, ti.mrows, ti.w_off)) return false;
    } else {
      ti.m0 = (t % ntm) * kMT;
      ti.mrows = min(kMT, a.M - ti.m0);
      ti.w_off = 0;
    }
    ti.n0 = (t / ntm) * kNT;
    ti.m0 = __builtin_amdgcn_readfirstlane(ti.m0);
    ti.mrows = __builtin_amdgcn_readfirstlane(ti.mrows);
    ti.n0 = __builtin_amdgcn_readfirstlane(ti.n0);
    return true;
  };
  // XCD-aware persistent schedule: workgroups are dispatched round-robin over
  // the eight XCDs, so XCD x = blockIdx % 8 takes one contiguous chunk
  // [c0, c1) of the tile order (consecutive tiles share a weight block, or an
  // expert's rows, in that XCD's L2), and its P workgroups walk the chunk with
  // stride P.  With one workgroup per tile every workgroup takes exactly tile
  // c0 + blockIdx / 8.
  const int T = ntm * ntn;
  const int xcd = blockIdx.x & 7;
  const int c0 = xcd * (T >> 3) + min(xcd, T & 7);
  const int c1 = (xcd + 1) * (T >> 3) + min(xcd + 1, T & 7);
  const int P = ((int)gridDim.x - xcd + 7) >> 3;
  const int t_first = c0 + (int)(blockIdx.x >> 3);
  const int nsb = a.K >> 8;
  const int npair = (nsb + 1) >> 1;
  // LDS byte addresses as integers from one wave-uniform base (no per-lane
  // generic-to-LDS pointer casts)
  const uint32_t ring_lds = __builtin_amdgcn_readfirstlane(lds_addr(ring));

  if (wave >= kMfmaWaves) {
    // ---------------------------------------------------------- loader wave
    const int par = wave - kMfmaWaves;
    const uint32_t wrb = a.ldw;
    const uint32_t xrb = (uint32_t)nsb * kQ8_KBytes;
    const uint8_t* xbase = a.Xq;
    const uint8_t* wbase = a.W;
    uint32_t voff[kSlots];
    // bases and per-lane offsets of tile ti's loads
    auto setup = [&](const Tile& ti) {
      // grouped: rows are gathered, offsets from Xq itself (the host keeps
      // the quantized activation within 32-bit offsets)
      xbase = kGroup ? a.Xq : a.Xq + (size_t)ti.m0 * xrb;
      wbase = a.W + ti.w_off + (size_t)ti.n0 * wrb;
      // activation row of tile row r (r < mrows); grouped: lane r looks up
      // row r once and the other lanes fetch it by cross-lane permute (one
      // pair-list load and division per lane instead of one per offset)
      int lane_row = 0;
      if constexpr (kGroup) lane_row = group_act_row(a.grp, ti.m0, min(lane, ti.mrows - 1));
      auto act_row = [&](int r) -> int {
        if constexpr (kGroup)
          return __shfl(lane_row, r);
        else
          return r;
      };
#pragma unroll
      for (int k = 0; k < kSlots; ++k) {
        uint32_t o;
        if (k < kAQSlots) {
          const int q = 64 * k + lane, r = q / 17, c = min(q - 17 * r, 15);
          o = (uint32_t)act_row(min(r, ti.mrows - 1)) * xrb + 4 + 16 * c;
        } else if (k < kAQSlots + kAXSlots) {
          const int q = 64 * (k - kAQSlots) + lane, r = q / 3, e = q - 3 * r;
          o = (uint32_t)act_row(min(r, ti.mrows - 1)) * xrb + (e == 0 ? 0 : 244 + 16 * e);
        } else if constexpr (kIlv) {
          // line q of the eight 144-line cohort blocks; cohorts past N repeat
          // the last one (N is a multiple of 16)
          const int q = 64 * (k - kAQSlots - kAXSlots) + lane, i = q / 144, line = q - 144 * i;
          o = (uint32_t)(min(ti.n0 + 16 * i, a.N - 16) - ti.n0) * wrb + 16 * line;
        } else {
          const int q = 64 * (k - kAQSlots - kAXSlots) + lane, row = q / 9, part = q - 9 * row;
          o = (uint32_t)(min(ti.n0 + row, a.N - 1) - ti.n0) * wrb + 16 * part;
        }
        voff[k] = o;
      }
    };
    // superblock 2 pair + par of the current tile into ring slot `slot`
    auto issue = [&](int pair, int slot) {
      const int b = min(2 * pair + par, nsb - 1);
      const uint32_t stage = ring_lds + (uint32_t)(2 * slot + par) * kStage;
      const uint8_t* xb = xbase + (size_t)b * kQ8_KBytes;
      const uint8_t* wb = wbase + (size_t)b * (kIlv ? kCohortBlock : kQ4_KBytes);
#pragma unroll
      for (int k = 0; k < kSlots; ++k)
        lds_dma16(k < kAQSlots + kAXSlots ? xb : wb, voff[k], stage + 1024 * k);
    };
    // In place in the landed stage, token t = lane: the 16 bsums become f16
    // (min-term A operand) and the 16-byte d chunk becomes the token-scale
    // operand of the dx (x) dw outer product: bf16 pairs (h,h), (m,m), (l,l),
    // 0 with d = h + m + l to 2^-24.
    auto convert = [&](int slot) {
      if (lane >= kMT) return;  // past the tile's tokens: the region's padding
      uint8_t* ax = ring + (2 * slot + par) * kStage + kAQ + 48 * lane;
      const uint4 dch = *reinterpret_cast<const uint4*>(ax);
      const uint4 b0 = *reinterpret_cast<const uint4*>(ax + 16);
      const uint4 b1 = *reinterpret_cast<const uint4*>(ax + 32);
      const float d = __uint_as_float(dch.x);
      const uint32_t ph = pk_bf16(d, d);
      const float r1 = d - bf16_lo_to_f32(ph);
      const uint32_t pm = pk_bf16(r1, r1);
      const float r2 = r1 - bf16_lo_to_f32(pm);
      const uint32_t pl = pk_bf16(r2, r2);
      *reinterpret_cast<uint4*>(ax) = make_uint4(ph, pm, pl, 0u);
      *reinterpret_cast<uint4*>(ax + 16) =
          make_uint4(i16x2_to_f16x2(b0.x), i16x2_to_f16x2(b0.y), i16x2_to_f16x2(b0.z), i16x2_to_f16x2(b0.w));
      *reinterpret_cast<uint4*>(ax + 32) =
          make_uint4(i16x2_to_f16x2(b1.x), i16x2_to_f16x2(b1.y), i16x2_to_f16x2(b1.z), i16x2_to_f16x2(b1.w));
    };
    // The pairs of all this workgroup's tiles form one stream over the two
    // ring slots (pair g in slot g & 1): at the last pair of a tile the next
    // tile's first pair is issued, so its loads overlap this tile's last
    // pair and output stage.  Per tile: one barrier per pair, then the two
    // barriers of the output stage, as the MFMA waves.
    Tile ti;
    int t = t_first;
    while (t < c1 && !tile_info(t, ti)) t += P;
    if (t >= c1) return;  // no tile: the MFMA waves find none either
    setup(ti);
    issue(0, 0);
    int g = 0;
    for (;;) {
      Tile tn;
      int u = t + P;
      while (u < c1 && !tile_info(u, tn)) u += P;
      const bool more = u < c1;
      for (int pair = 0; pair + 1 < npair; ++pair, ++g) {
        __builtin_amdgcn_s_waitcnt(0);  // this pair's stage has landed
        convert(g & 1);
        __syncthreads();                // hand it over; the slot of pair g - 1 is free
        issue(pair + 1, (g + 1) & 1);
      }
      // the tile's last pair; the next tile's offsets are formed only here
      // (formed before the loop they would hold a second set of registers)
      __builtin_amdgcn_s_waitcnt(0);
      convert(g & 1);
      __syncthreads();
      if (more) {
        setup(tn);
        issue(0, (g + 1) & 1);
      }
      ++g;
      __syncthreads();  // the output stage's barriers
      __syncthreads();
      if (!more) return;
      t = u;
    }
  }

  // ------------------------------------------------------------ MFMA wave
  const int par = wave / kCols, wcol = wave % kCols;  // superblock parity, column group
  const int col = lane & 31, kg = lane >> 5;
  const uint32_t zaddr = lds_addr(zero16);

  v16i lo[kT2], hi[kT2];
  v16f y[kT2];
  const v16i zero = {};
  const v16f fzero = {};
  int g = 0;  // pairs consumed over this workgroup's tiles: pair g sits in ring slot g & 1
  for (int t = t_first; t < c1; t += P) {
    Tile ti;
    if (!tile_info(t, ti)) continue;
#pragma unroll
    for (int t2 = 0; t2 < kT2; ++t2)
#pragma unroll
      for (int r = 0; r < 16; ++r) y[t2][r] = 0.f;
    for (int pair = 0; pair < npair; ++pair, ++g) {
      __syncthreads();  // the loaders have staged and converted this pair
      if (2 * pair + par >= nsb) continue;  // odd nsb: the last pair has one superblock
      const uint8_t* stage = ring + (2 * (g & 1) + par) * kStage;
      const uint8_t* AQ = stage + kAQRow * col + 16 * kg;          // + 8704 t + 32 s
      const uint8_t* AX = stage + kAQ + 48 * col;                   // + 1536 t
      const uint8_t* wrow = stage + kAQ + kAX + (32 * wcol + col) * kQ4_KBytes;
      // interleaved: this lane's cohort block and the byte of its row in the
      // first line of a 16-lane group's window
      const uint32_t wtr = ring_lds + (uint32_t)(2 * (g & 1) + par) * kStage + kAQ + kAX +
                           (uint32_t)(2 * wcol + (col >> 4)) * kCohortBlock + 8 * (lane & 15);

      uint4 h;
      if constexpr (kIlv) {
        const uint2 h0 = tr8(wtr), h1 = tr8(wtr + 128);
        h = make_uint4(h0.x, h0.y, h1.x, h1.y);
      } else {
        h = *reinterpret_cast<const uint4*>(wrow);
      }
      const float dw = fp16_to_fp32(h.x & 0xffffu);
      const float dmin = fp16_to_fp32(h.x >> 16);
      const bool dz = dw == 0.f;
      const uint32_t sc03 = dz ? 0u : h.y & 0x3f3f3f3fu;
      const uint32_t sc47 = dz ? 0u : (h.w & 0x0f0f0f0fu) | (((h.y >> 6) & 0x03030303u) << 4);
      const float f = dz ? dmin : dw;
      const float nr = dz ? -1.f : -(dmin * __builtin_amdgcn_rcpf(dw));
      // per sub-block pair, the b (= sc & 7) and a (= sc >> 3) multipliers in
      // the two 16-bit halves of one register
      uint32_t cb[4], ca[4];
      {
        const uint32_t b03 = sc03 & 0x07070707u, a03 = (sc03 >> 3) & 0x07070707u;
        const uint32_t b47 = sc47 & 0x07070707u, a47 = (sc47 >> 3) & 0x07070707u;
        cb[0] = __builtin_amdgcn_perm(0u, b03, 0x0c010c00u);
        cb[1] = __builtin_amdgcn_perm(0u, b03, 0x0c030c02u);
        cb[2] = __builtin_amdgcn_perm(0u, b47, 0x0c010c00u);
        cb[3] = __builtin_amdgcn_perm(0u, b47, 0x0c030c02u);
        ca[0] = __builtin_amdgcn_perm(0u, a03, 0x0c010c00u);
        ca[1] = __builtin_amdgcn_perm(0u, a03, 0x0c030c02u);
        ca[2] = __builtin_amdgcn_perm(0u, a47, 0x0c010c00u);
        ca[3] = __builtin_amdgcn_perm(0u, a47, 0x0c030c02u);
      }

      v4i acur[kT2], anxt[kT2];
#pragma unroll
      for (int t = 0; t < kT2; ++t) acur[t] = *reinterpret_cast<const v4i*>(AQ + 32 * kAQRow * t);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        uint4 q;
        if constexpr (kIlv) {
          const uint32_t ql = wtr + 16 * (16 + 32 * g + 16 * kg);
          const uint2 q0 = tr8(ql), q1 = tr8(ql + 128);
          q = make_uint4(q0.x, q0.y, q1.x, q1.y);
        } else {
          q = *reinterpret_cast<const uint4*>(wrow + 16 + 32 * g + 16 * kg);
        }
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const int s = 2 * g + hf;
          if (s < 7) {
#pragma unroll
            for (int t = 0; t < kT2; ++t)
              anxt[t] = *reinterpret_cast<const v4i*>(AQ + 32 * kAQRow * t + 32 * (s + 1));
          }
          const uint32_t n0w = hf ? (q.x >> 4) & 0x0f0f0f0fu : q.x & 0x0f0f0f0fu;
          const uint32_t n1w = hf ? (q.y >> 4) & 0x0f0f0f0fu : q.y & 0x0f0f0f0fu;
          const uint32_t n2w = hf ? (q.z >> 4) & 0x0f0f0f0fu : q.z & 0x0f0f0f0fu;
          const uint32_t n3w = hf ? (q.w >> 4) & 0x0f0f0f0fu : q.w & 0x0f0f0f0fu;
          const v2u16 pb = __builtin_bit_cast(v2u16, cb[s >> 1]);
          const v2u16 pa = __builtin_bit_cast(v2u16, ca[s >> 1]);
          const v2u16 mb = (s & 1) ? __builtin_shufflevector(pb, pb, 1, 1) : __builtin_shufflevector(pb, pb, 0, 0);
          const v2u16 ma = (s & 1) ? __builtin_shufflevector(pa, pa, 1, 1) : __builtin_shufflevector(pa, pa, 0, 0);
          auto mul = [](uint32_t n, v2u16 m) {
            return (int)__builtin_bit_cast(uint32_t, __builtin_bit_cast(v2u16, n) * m);
          };
          const v4i b_lo = {mul(n0w, mb), mul(n1w, mb), mul(n2w, mb), mul(n3w, mb)};
          const v4i b_hi = {mul(n0w, ma), mul(n1w, ma), mul(n2w, ma), mul(n3w, ma)};
#pragma unroll
          for (int t = 0; t < kT2; ++t) {
            lo[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(acur[t], b_lo, s == 0 ? zero : lo[t], 0, 0, 0);
            hi[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(acur[t], b_hi, s == 0 ? zero : hi[t], 0, 0, 0);
          }
#pragma unroll
          for (int t = 0; t < kT2; ++t) acur[t] = anxt[t];
        }
      }

      // min term (f16: converted bsums x duplicated mins) and the dx (x) f
      // outer product (bf16: token-scale splits x f = f_h + f_l, exact)
      v16f mn[kT2], qd[kT2];
      {
        const uint32_t mn03 = h.z & 0x3f3f3f3fu;
        const uint32_t mn47 = ((h.w >> 4) & 0x0f0f0f0fu) | (((h.z >> 6) & 0x03030303u) << 4);
        const uint32_t mw = kg ? mn47 : mn03;
        const v4i bm = {(int)dup_byte_f16x2(mw, 0), (int)dup_byte_f16x2(mw, 1),
                        (int)dup_byte_f16x2(mw, 2), (int)dup_byte_f16x2(mw, 3)};
        const uint32_t pfh = pk_bf16(f, f);
        const uint32_t pf = kg ? 0u : pk_bf16(f, f - bf16_lo_to_f32(pfh));
        const v4i bq = {(int)pf, (int)pf, (int)pf, 0};
#pragma unroll
        for (int t = 0; t < kT2; ++t) {
          const v4i am = *reinterpret_cast<const v4i*>(AX + 1536 * t + 16 + 16 * kg);
          mn[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, am),
                                                        __builtin_bit_cast(v8h, bm), fzero, 0, 0, 0);
          const uint32_t qaddr = kg ? zaddr : lds_addr(AX + 1536 * t);
          const v4i aq = *(const __attribute__((address_space(3))) v4i*)(size_t)qaddr;
          qd[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, aq),
                                                         __builtin_bit_cast(v8bf, bq), fzero, 0, 0, 0);
        }
      }
      // y += (dx f) (lo + 8 hi - r Mn)
#pragma unroll
      for (int t = 0; t < kT2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float d = fmaf(mn[t][r], nr, (float)(lo[t][r] + 8 * hi[t][r]));
          y[t][r] = fmaf(d, qd[t][r], y[t][r]);
        }
    }

    // Both parities' partial sums -> two LDS planes in the slot of the tile's
    // last pair (the other slot may already be receiving the next tile) -> Y.
    // The first barrier: every wave is done reading that slot.
    __syncthreads();
    float* planes = reinterpret_cast<float*>(ring + 2 * ((g - 1) & 1) * kStage);
    tile_partials_to_lds_t<kT2, kNT>(y, wcol, lane, planes + par * (TL::kPlaneBytes / 4));
    __syncthreads();
    // grouped: lane r looks up the dst row of tile row r; the two rows this
    // lane stores are fetched by cross-lane permute here, where every lane
    // is active (inside the store's row checks some lanes are not)
    long long dst_lo = 0, dst_hi = 0;
    if constexpr (kGroup) {
      const long long own = group_dst_row(a.grp, ti.m0, min(lane, ti.mrows - 1));
      auto fetch = [&](int src) {
        return (long long)(((uint64_t)(uint32_t)__shfl((int)(own >> 32), src) << 32) |
                           (uint32_t)__shfl((int)(own & 0xffffffff), src));
      };
      dst_lo = fetch(tile_store_row(wave, lane, 0));
      dst_hi = fetch(tile_store_row(wave, lane, 1));
    }
    tile_store_from_lds_t<kMT, kNT, kMfmaWaves>(
        wave, lane, planes, planes + TL::kPlaneBytes / 4, ti.mrows, min(kNT, a.N - ti.n0),
        [&](int rr) {
          if constexpr (kGroup)
            return a.Y + (rr < 32 ? dst_lo : dst_hi) + ti.n0;
          else
            return a.Y + (size_t)(ti.m0 + rr) * a.ldy + ti.n0;
        },
        [](float e, float o) { return e + o; });
  }
}

// The GEMM over an already quantized activation.  Weight rows must be
// 4-byte aligned (dword direct-to-LDS loads) and a tile's rows (up to 128)
// must stay within 32-bit offsets.
bool gemm_q4k_ok(const uint8_t* W, size_t N, size_t K, size_t M, const RowStrides& st) {
  const size_t rb = K / 256 * kQ4_KBytes;
  const size_t ldw = N > 1 ? st.ldw : rb;
  return aligned(W, 4) && ldw % 4 == 0 && (DefaultTiling::kNT - 1) * ldw + rb < ((size_t)1 << 32) &&
         N <= (size_t)INT32_MAX && K <= (size_t)INT32_MAX && M <= (size_t)INT32_MAX &&
         ((N + 63) / 64) * ((M + 31) / 32) <= (size_t)INT32_MAX;
}

// The tiling of a dense launch.  CompileOptions.meta's bindings, when set
// on the calling thread, choose it as the reference's loop extents do
// (examples/kernels/mul_mat/q4_k_staged.py:20-24): MC activation rows per
// tile (<= 32: 32-token tiles, else 64), NC weight rows per tile (<= 64:
// 64-row tiles, else 128).  Unbound: 32-token tiles for M <= 32, 64-row
// tiles when 128-row ones would leave more than half of the CUs idle.
struct GemmShape {
  int mt, nt;
};
GemmShape gemm_q4k_shape(size_t N, size_t M) {
  const TileBindings& tb = tile_bindings();
  const int mt = tb.mc > 0 ? (tb.mc <= 32 ? 32 : 64) : (M <= 32 ? 32 : 64);
  int nt = 128;
  if (tb.nc > 0)
    nt = tb.nc <= 64 ? 64 : 128;
  else if (((N + 127) / 128) * ((M + mt - 1) / mt) * 2 < (size_t)cu_count())
    nt = 64;
  return {mt, nt};
}

template <bool kIlv, class TL>
void launch_gemm_q4k(const GemmArgs& a, size_t N, size_t M) {
  // one workgroup per CU at most (the ring takes the CU's LDS); each walks
  // its share of the tiles
  const size_t tiles = ((N + TL::kNT - 1) / TL::kNT) * ((M + TL::kMT - 1) / TL::kMT);
  const unsigned wgs = (unsigned)std::min(tiles, (size_t)cu_count());
  q4k_mfma_gemm<false, kIlv, TL><<<dim3(wgs), TL::kThreads, 0, current_stream()>>>(a);
  // the launch log names the tiling and the workgroup count
  char name[48] = "q4k_mfma_gemm";
  if (launch_log_enabled()) snprintf(name, sizeof(name), "q4k_mfma_gemm_%dx%d/%u", TL::kMT, TL::kNT, wgs);
  check_launch(name);
}

template <bool kIlv = false>
void gemm_q4k(const uint8_t* W, const uint8_t* Xq, float* Y, size_t N, size_t K, size_t M,
              const RowStrides& st) {
  const size_t rb = K / 256 * kQ4_KBytes;
  GemmArgs a{};
  a.W = W;
  a.Xq = Xq;
  a.Y = Y;
  a.N = (int)N;
  a.K = (int)K;
  a.M = (int)M;
  a.ldw = (uint32_t)(N > 1 ? st.ldw : rb);
  a.ldy = (long long)st.ldy;
  if constexpr (kIlv) {
    launch_gemm_q4k<true, DefaultTiling>(a, N, M);  // the persisted layout has no bindings
  } else {
    const GemmShape sh = gemm_q4k_shape(N, M);
    if (sh.mt == 64 && sh.nt == 128)
      launch_gemm_q4k<false, Tiling<64, 128>>(a, N, M);
    else if (sh.mt == 32 && sh.nt == 128)
      launch_gemm_q4k<false, Tiling<32, 128>>(a, N, M);
    else if (sh.mt == 64)
      launch_gemm_q4k<false, Tiling<64, 64>>(a, N, M);
    else
      launch_gemm_q4k<false, Tiling<32, 64>>(a, N, M);
  }
}

bool args_ok(const uint8_t* W, const void* Xq, const float* Y, size_t N, size_t K, size_t M,
             const RowStrides& st) {
  return K % 256 == 0 && W != nullptr && Xq != nullptr && Y != nullptr && aligned(Xq, 4) &&
         aligned(Y, 4) && strides_ok(st, K / 256 * kQ4_KBytes, 2, K, N, N, M);
}

}  // namespace

bool gemm_q4k_try(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K, size_t M,
                  const RowStrides& st) {
  if (N == 0 || M == 0 || K == 0 || X == nullptr || !args_ok(W, Xq, Y, N, K, M, st) ||
      !gemm_q4k_ok(W, N, K, M, st))
    return false;
  quantize_q8_k_rows(X, st.ldx, Xq, M, K);
  gemm_q4k(W, Xq, Y, N, K, M, st);
  return true;
}

// Prefill entry: MFMA GEMM when the shape suits it, the decode GEMV otherwise.
void mul_mat_q4k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M, const RowStrides& st) {
  if (N == 0 || M == 0 || K == 0) return;
  // the GEMV below 16 activation rows, unless its LDS cannot hold a row
  if ((M >= 16 || !q4k_gemv_fits(K)) && X != nullptr && args_ok(W, Xq, Y, N, K, M, st) &&
      gemm_q4k_ok(W, N, K, M, st)) {
    quantize_q8_k_rows(X, st.ldx, Xq, M, K);
    gemm_q4k(W, Xq, Y, N, K, M, st);
  } else {
    decode_q4k(W, X, Xq, Y, N, K, M, st);
  }
}

bool mul_mat_id_q4k_grouped_ok(const uint8_t* W, size_t xq_bytes, const float* Y, size_t N, size_t K,
                               const RowStrides& st, const PairArgs& pr, int n_pairs, const void* ws,
                               size_t ws_bytes) {
  const size_t rb = K / 256 * kQ4_KBytes;
  return N > 0 && K > 0 && n_pairs > 0 && K % 256 == 0 && pr.n_as <= kMaxExperts &&
         xq_bytes < ((size_t)1 << 32) && aligned(Y, 4) && aligned(ws, 16) &&
         ws_bytes >= moe_group_bytes(n_pairs, pr.n_as) && pr.w_es % 4 == 0 &&
         gemm_q4k_ok(W, N, K, DefaultTiling::kMT, st) && strides_ok(st, rb, 2, K, N, N, 1) &&
         (size_t)moe_tile_bound(n_pairs, pr.n_as) * ((N + 127) / 128) <= (size_t)INT32_MAX;
}

void mul_mat_id_q4k_grouped(const uint8_t* W, const uint8_t* Xq, float* Y, size_t N, size_t K,
                            const RowStrides& st, const PairArgs& pr, int n_pairs, void* ws) {
  const size_t rb = K / 256 * kQ4_KBytes;
  const MoeGroups g = moe_group(pr, n_pairs, ws);
  GemmArgs a{};
  a.W = W;
  a.Xq = Xq;
  a.Y = Y;
  a.N = (int)N;
  a.K = (int)K;
  a.M = DefaultTiling::kMT;
  a.ldw = (uint32_t)(N > 1 ? st.ldw : rb);
  a.grp = group_tiles(g, pr);
  const size_t tiles = (size_t)g.tmax * ((N + DefaultTiling::kNT - 1) / DefaultTiling::kNT);
  const size_t wgs = std::min(tiles, (size_t)cu_count());
  q4k_mfma_gemm<true><<<dim3((unsigned)wgs), DefaultTiling::kThreads, 0, current_stream()>>>(a);
  check_launch("q4k_mfma_gemm_grouped");
}

// production_mul_mat_q4_k_persistent: W is the Q4K_I[16] interleave of an
// N x K Q4_K matrix (N a multiple of 16), X is M x K, all packed.  X is
// quantized into Xq (Q8_K), then the GEMM reads the cohort blocks for M >= 16
// and the interleaved GEMV runs once per activation row below that.
void mul_mat_q4k_persistent(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t M,
                            size_t K, size_t N) {
  if (N == 0 || M == 0 || K == 0) return;
  const size_t rb = K / 256 * kQ4_KBytes, xrb = K / 256 * kQ8_KBytes;
  const RowStrides st = packed(rb, K, N);
  if (K % 256 != 0 || N % 16 != 0 || W == nullptr || X == nullptr || Xq == nullptr ||
      Y == nullptr || !aligned(W, 16) || !aligned(Xq, 4) || !aligned(Y, 4) || !aligned(X, 4) ||
      !strides_ok(st, rb, 16, K, N, N, M)) {
    set_error(hipErrorInvalidValue);
    return;
  }
  quantize_q8_k_rows(X, K, Xq, M, K);
  if ((M >= 16 || !q4k_i16_gemv_fits(N, K)) && gemm_q4k_ok(W, N, K, M, st)) {
    gemm_q4k<true>(W, Xq, Y, N, K, M, st);
  } else {
    for (size_t m = 0; m < M; ++m) q4k_i16_gemv(W, Xq + m * xrb, Y + m * N, N, K);
  }
}

void mul_mat_q4k_quantized(const uint8_t* W, const uint8_t* Xq, float* Y, size_t N, size_t K,
                           size_t M, const RowStrides& st) {
  if (N == 0 || M == 0 || K == 0) return;
  if ((M >= 16 || !q4k_gemv_fits(K)) && args_ok(W, Xq, Y, N, K, M, st) && gemm_q4k_ok(W, N, K, M, st))
    gemm_q4k(W, Xq, Y, N, K, M, st);
  else
    decode_q4k_quantized(W, Xq, Y, N, K, M, st);
}

}  // namespace weft
