// Q4_0 / MXFP4 / NVFP4 x Q8_0 and Q4_1 x Q8_1 prefill GEMMs on int8 MFMA
// (production_mul_mat_q4_0, examples/kernels/mul_mat/q4_0.py:9-30;
// production_mul_mat_mxfp4, mxfp4.py:10-35; production_mul_mat_nvfp4,
// nvfp4.py:10-43; production_mul_mat_q4_1, q4_1.py:9-10).
//
//   Y[m, n] = sum_b dx[m,b] * ws[n,b] * I[m,n,b],   I = sum_{k in b} q8[m,k] * w[n,k]
//   Q4_0:  w = q - 8,            ws = fp16 d        (ggml-cpu/quants.c:174-208)
//   MXFP4: w = codebook[q],      ws = scale[e]      (ggml-cpu/quants.c:247-276)
//   NVFP4: w = codebook[q], a UE4M3 scale per 16-element half of the block
//          (ggml-cpu/quants.c:279-313): the block's MFMA runs twice with the
//          weight operand of one half, Y += dx * (ws_lo I_lo + ws_hi I_hi)
// One v_mfma_i32_32x32x32_i8 per 32x32 tile and 32-block gives I exactly; the
// two per-block scales are applied in fp32 on VALU, which is what bounds
// these kernels.  Q4_0 / Q4_1: the factor dx ws of every output comes from
// one f16 outer-product MFMA per tile and block (both scales are fp16, the
// product exact in fp32), then convert and FMA: 2 VALU instructions per
// output and block; NVFP4 and the MXFP4 table body: 3.
//
// Activation layout.  A Q8_0 record is 34 bytes at 2-byte alignment, which
// cannot feed 16-byte operand reads.  The activation is therefore quantized
// first into Xq in a planar layout of the same size -- row m holds its K int8
// values followed by its K/32 fp16 scales (row stride 17K/16) -- and, after
// the GEMM, quantized again in GGML's record layout, so Xq ends exactly as
// q8_0_quantize writes it.  Quantization is deterministic, so both passes
// produce the same int8 values and scales.
//
// Tiling as in the Q4_K prefill: 64 tokens x 128 weight rows per workgroup,
// 8 waves (superblock parity x 4 column groups), each wave two 32x32 tiles.
// A stage is 8 blocks (256 K values).  The activation int8 tile (swizzled
// 16-byte chunks) and the raw weight rows (8 records per row) are copied to
// LDS by direct loads a stage ahead; weight operands are unpacked from the
// raw records with aligned dword reads and byte alignment.  The per-block
// token scales are loaded by one wave per parity and transposed to fp32
// [block][token] so the combine reads four tokens with one instruction.
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
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_ptr;

enum class WFmt { Q4_0, MXFP4, Q4_1, NVFP4 };

template <WFmt F>
struct WTraits;
template <>
struct WTraits<WFmt::Q4_0> {
  static constexpr int kRec = kQ4_0Bytes;  // 18
  static constexpr int kHdr = 2;           // fp16 d, then 16 nibble bytes
};
template <>
struct WTraits<WFmt::MXFP4> {
  static constexpr int kRec = kMxfp4Bytes;  // 17
  static constexpr int kHdr = 1;            // e8m0 e, then 16 nibble bytes
};
template <>
struct WTraits<WFmt::Q4_1> {
  static constexpr int kRec = kQ4_1Bytes;  // 20
  static constexpr int kHdr = 4;           // fp16 d, fp16 m, then 16 nibble bytes
};
// NVFP4: a 36-byte record covers two 32-blocks (4 UE4M3 scales, then 8 code
// bytes per 16-element sub-block); kRec is the bytes per 32 elements
template <>
struct WTraits<WFmt::NVFP4> {
  static constexpr int kRec = kNvfp4Bytes / 2;  // 18
  static constexpr int kHdr = 4;
};

// Planar activation row bytes: K int8, K/32 fp16 scales d, and for Q4_1's
// Q8_1 activation K/32 fp16 block sums s (the size of the caller's Xq row)
template <WFmt F>
constexpr size_t planar_row_bytes(size_t K) {
  return K + K / 16 + (F == WFmt::Q4_1 ? K / 16 : 0);
}

constexpr int kMT = 64;        // tokens per workgroup tile
constexpr int kNT = 128;       // weight rows per workgroup tile
constexpr int kThreads = 512;  // 8 waves: 4 column groups x 2 stage parities
constexpr int kAQ = kMT * 256;  // activation int8 per stage

struct GemmArgs {
  const uint8_t* W;
  const uint8_t* Xp;  // planar activation (rows of K int8 + K/32 fp16)
  const int8_t* codebook;
  const float* scale;
  float* Y;
  int N, K, M;
  size_t ldw;     // bytes between weight rows
  long long ldy;  // floats between output rows
  GroupTiles grp;  // grouped (MUL_MAT_ID) mode
};

// 16 bytes per lane from global straight into LDS: lane l writes
// [lds + 16 l, +16).  Inline asm keeps the compiler from making unrelated LDS
// reads wait for it; the kernel waits (s_waitcnt) itself.  Nothing else in
// this file's kernels uses M0.
__device__ __forceinline__ void lds_dma16(const uint8_t* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds), "v"(g)
               : "memory", "m0");
}
// 4 bytes per lane: lane l writes [lds + 4 l, +4)
__device__ __forceinline__ void lds_dma4(const uint8_t* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off"
               :
               : "s"(lds), "v"(g)
               : "memory", "m0");
}
// 4 bytes per lane from sbase + voff (SGPR base, 32-bit lane offset)
__device__ __forceinline__ void lds_dma4_s(const uint8_t* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2"
               :
               : "s"(lds), "v"(voff), "s"(sbase)
               : "memory", "m0");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_ptr)p;
}
__device__ __forceinline__ uint32_t ld32(const uint8_t* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}

// four nibbles (one per byte) -> the 16-entry int8 codebook c0..c3
__device__ __forceinline__ uint32_t lookup16(uint32_t n, uint32_t c0, uint32_t c1, uint32_t c2,
                                             uint32_t c3) {
  const uint32_t sel = n & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(c1, c0, sel);
  const uint32_t hi = __builtin_amdgcn_perm(c3, c2, sel);
  const uint32_t mask = ((n >> 3) & 0x01010101u) * 0xffu;
  return (hi & mask) | (lo & ~mask);
}

// LDS bytes of the int8 GEMM body: two ring slots of two stages, the token
// scales (fp32), Q4_1's token block sums (fp16), the MXFP4 / UE4M3 scale table
template <WFmt F>
constexpr bool has_table() {
  return F == WFmt::MXFP4 || F == WFmt::NVFP4;
}
// LDS bytes per weight row and stage: the row's 8 records (2 kRec dwords).
// Q4_0 / NVFP4 rows (144 bytes a stage, whole 16-byte chunks) arrive by
// 16-byte direct loads when 16-byte aligned, else by dword loads, at that
// stride (2-way bank conflicts on the operand reads).  Q4_1's 40-dword rows
// would put the 32 rows a wave reads at one record offset into 8 of the 64
// banks (4-way): its rows get one pad dword (an odd stride, 32 banks) and
// dword loads (its 16-byte loads at the unpadded stride measured 2.3 us
// slower; a padded 16-byte stride does not fit the LDS).  Padding the 36-
// and 34-dword rows measured slower: two more wave-wide loads per stage.
template <WFmt F>
constexpr int w_lds_row() {
  return 4 * (2 * WTraits<F>::kRec + ((2 * WTraits<F>::kRec) % 8 == 0 ? 1 : 0));
}
template <WFmt F>
constexpr int q80_lds_bytes() {
  return 4 * (kAQ + kNT * w_lds_row<F>()) + 2 * 2 * 8 * kMT * 4 +
         (F == WFmt::Q4_1 ? 2 * 2 * 8 * kMT * 2 : 0) + (has_table<F>() ? 256 * 4 : 0);
}

template <WFmt F, bool kGroup>
__device__ __forceinline__ void q80_gemm_body(const GemmArgs& a, uint8_t* lds) {
  using T = WTraits<F>;
  constexpr int kRB = 8 * T::kRec;           // raw weight bytes per row and stage
  constexpr int kRL = w_lds_row<F>();        // LDS bytes per weight row (Q4_1: kRB + 4)
  constexpr int kWT = kNT * kRL;             // 18432 (Q4_0) / 17408 (MXFP4) / 20992 (Q4_1)
  constexpr int kStage = kAQ + kWT;
  constexpr int kWD = kRB / 4;               // dwords per weight row and stage
  constexpr int kWDp = kRL / 4;              // the same, with the pad
  constexpr int kWSlots = kNT * kWDp / 64;   // 72 / 68 / 82 wave-wide dword loads
  constexpr int kWPerWave = (kWSlots + 3) / 4;
  constexpr int kCh = kRB / 16;              // 16-byte chunks per row and stage (9 / 10)
  constexpr int kW16 = kNT * kCh / 64;       // 18 / 20 wave-wide 16-byte loads
  constexpr int kW16PerWave = (kW16 + 3) / 4;
  static_assert(kNT * kWDp % 64 == 0 && (kRL == kRB || kRL == kRB + 4), "whole wave-wide weight loads");
  static_assert(kRB % 16 != 0 || kNT * kCh % 64 == 0, "whole wave-wide 16-byte weight loads");
  static_assert(kTilePlaneBytes <= 2 * kStage, "an output plane fits one ring half");

  // two ring slots; a slot being filled by direct loads never aliases the
  // slot being read
  uint8_t* ring0 = lds;
  uint8_t* ring1 = lds + 2 * kStage;
  float(*adt)[2][8 * kMT] = reinterpret_cast<float(*)[2][8 * kMT]>(lds + 4 * kStage);  // [slot][parity][block][token]
  // Q4_1: the tokens' fp16 block sums [slot][parity][block][token]; MXFP4: scale table
  // [slot][parity][token][block]
  uint16_t(*ast)[2][8 * kMT] = reinterpret_cast<uint16_t(*)[2][8 * kMT]>(lds + 4 * kStage + 2 * 2 * 8 * kMT * 4);
  float* scl = reinterpret_cast<float*>(lds + 4 * kStage) + 2 * 2 * 8 * kMT;
  static_assert(q80_lds_bytes<F>() == 4 * kStage + 2 * 2 * 8 * kMT * 4 +
                                          (F == WFmt::Q4_1 ? 2 * 2 * 8 * kMT * 2 : 0) +
                                          (has_table<F>() ? 256 * 4 : 0),
                "LDS carve");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int par = wave >> 2, wcol = wave & 3;
  const int col = lane & 31, kg = lane >> 5;
  const int nst = a.K >> 8;                         // stages (8 blocks each)
  const size_t xs = planar_row_bytes<F>((size_t)a.K);  // planar activation row stride
  const size_t ws_row = a.ldw;

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

  uint32_t c0 = 0, c1 = 0, c2 = 0, c3 = 0;
  if constexpr (has_table<F>()) {
    // int8[16] codebook at any alignment: four little-endian words
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)(uint8_t)a.codebook[4 * i] | (uint32_t)(uint8_t)a.codebook[4 * i + 1] << 8 |
             (uint32_t)(uint8_t)a.codebook[4 * i + 2] << 16 |
             (uint32_t)(uint8_t)a.codebook[4 * i + 3] << 24;
    c0 = w[0], c1 = w[1], c2 = w[2], c3 = w[3];
    if (tid < 256) scl[tid] = a.scale[tid];
  }

  // activation int8 tile: 16 wave-wide 16-byte loads per stage, 4 per wave
  const uint8_t* asrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = wcol + 4 * i;
    const int q = 64 * k + lane, r = q >> 4, c = (q & 15) ^ (r & 15);
    asrc[i] = a.Xp + (size_t)act_row(min(r, mrows - 1)) * xs + 16 * c;
  }
  // per-block token scales of this parity's stage: wave wcol == 0, token = lane
  const uint8_t* dsrc = a.Xp + (size_t)act_row(min(lane, mrows - 1)) * xs + a.K;

  // weight rows by 16-byte loads when a row's stage bytes are whole aligned
  // chunks (wave-uniform), at LDS stride kRB; else dword loads at kRL
  const bool w16 = kRL == kRB && kRB % 16 == 0 && ((reinterpret_cast<uintptr_t>(W) | ws_row) & 15) == 0;
  const int rl = w16 ? kRB : kRL;
  // chunk q = 64 k + lane of load k = wcol + 4 i: row q / kCh, chunk q % kCh
  // (offsets from the tile's first row: the host keeps them in 32 bits)
  const uint8_t* wtile = W + (size_t)n0 * ws_row;
  uint32_t wv16[kW16PerWave];
#pragma unroll
  for (int i = 0; i < kW16PerWave; ++i) {
    const int q = 64 * min(wcol + 4 * i, kW16 - 1) + lane, row = q / max(kCh, 1);
    wv16[i] = (uint32_t)min(row, a.N - 1 - n0) * (uint32_t)ws_row + 16 * (uint32_t)(q - kCh * row);
  }

  // LDS byte addresses as integers from one wave-uniform base: no per-use
  // generic-to-LDS pointer casts (their null checks on VALU do not compile)
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  auto issue = [&](int pair, uint8_t* ring) {
    const int st = min(2 * pair + par, nst - 1);
    const uint32_t stage = lds0 + (uint32_t)(ring - lds) + par * kStage;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      lds_dma16(asrc[i] + 256 * (size_t)st, stage + 1024 * (wcol + 4 * i));
    if (kRL == kRB && kRB % 16 == 0 && w16) {
#pragma unroll
      for (int i = 0; i < kW16PerWave; ++i)
        if (kW16 % 4 == 0 || wcol + 4 * i < kW16)  // wave-uniform
          lds_dma16(wtile + (size_t)st * kRB + wv16[i], stage + kAQ + 1024 * (wcol + 4 * i));
      return;
    }
#pragma unroll
    for (int i = 0; i < kWPerWave; ++i) {
      const int k = wcol + 4 * i;
      if (kWSlots % 4 == 0 || k < kWSlots) {  // wave-uniform
        // the pad dword repeats the row's last one
        const int q = 64 * k + lane, row = q / kWDp, part = min(q - kWDp * row, kWD - 1);
        const uint8_t* g = W + (size_t)min(n0 + row, a.N - 1) * ws_row + (size_t)st * kRB + 4 * part;
        lds_dma4(g, stage + kAQ + 256 * k);
      }
    }
  };
  uint4 dxraw = make_uint4(0, 0, 0, 0), sraw = make_uint4(0, 0, 0, 0);
  auto load_dx = [&](int pair) {
    const int st = min(2 * pair + par, nst - 1);
    dxraw = *reinterpret_cast<const uint4*>(dsrc + 16 * (size_t)st);
    if constexpr (F == WFmt::Q4_1) sraw = *reinterpret_cast<const uint4*>(dsrc + a.K / 16 + 16 * (size_t)st);
  };
  auto store_dx = [&](int slot) {
    float* d = &adt[slot][par][0];
    const uint32_t w[4] = {dxraw.x, dxraw.y, dxraw.z, dxraw.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) d[j * kMT + lane] = fp16_to_fp32((w[j >> 1] >> (16 * (j & 1))) & 0xffffu);
    if constexpr (F == WFmt::Q4_1)  // the token's eight fp16 block sums, token-major
      *reinterpret_cast<uint4*>(&ast[slot][par][8 * lane]) = sraw;
  };

  v16i I[2];
  v16f y[2];
  const v16f fzero = {};
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) y[t][r] = 0.f;
  const v16i zero = {};
  const int npair = (nst + 1) >> 1;
  const int sw = col & 15;

  // Blocks J0 .. J0 + 3 of this wave's stage of the pair in `cur`.
  auto half = [&](int pair, const uint8_t* cur, auto j0_tag) {
    constexpr int J0 = decltype(j0_tag)::value;
    const uint8_t* stage = cur + par * kStage;
    const uint8_t* AQ = stage;
    const uint8_t* wrow = stage + kAQ + (32 * wcol + col) * rl;
    const float* dxs = &adt[pair & 1][par][0];
    const uint16_t* sxs = &ast[pair & 1][par][0];
    // Q4_0: the row's 144 stage bytes as nine 16-byte LDS reads (the 36-dword
    // stride puts 16 lanes' 16-byte reads on all 64 banks); every record is
    // then taken from registers at fixed offsets
    uint32_t wq[F == WFmt::Q4_0 ? 36 : 1];
    if constexpr (F == WFmt::Q4_0) {
#pragma unroll
      for (int i = 0; i < 9; ++i) {
        // this half's records (and the dword before a record's nibbles
        // holding its scale) lie in bytes [18 J0, 18 J0 + 72)
        if (16 * i >= 18 * J0 + 72 || 16 * i + 16 <= 18 * J0) continue;
        const uint4 v = *reinterpret_cast<const uint4*>(wrow + 16 * i);
        wq[4 * i] = v.x, wq[4 * i + 1] = v.y, wq[4 * i + 2] = v.z, wq[4 * i + 3] = v.w;
      }
    }
    auto wld = [&](int byte) -> uint32_t {  // the row's aligned dword at `byte`
      if constexpr (F == WFmt::Q4_0)
        return wq[byte >> 2];
      else
        return ld32(wrow + byte);
    };
#pragma unroll
    for (int j = J0; j < J0 + 4; ++j) {
      if constexpr (F == WFmt::NVFP4) {
        // block j is half j % 2 of record j / 2: sub-blocks 2 (j % 2) + kg;
        // this lane's 16 elements are the low nibbles of its sub-block's 8
        // code bytes, then their high nibbles
        const uint8_t* rec = wrow + 36 * (j >> 1);
        const uint32_t sc4 = ld32(rec);
        const uint32_t u0 = ld32(rec + 4 + 16 * (j & 1) + 8 * kg), u1 = ld32(rec + 8 + 16 * (j & 1) + 8 * kg);
        const float wlo = scl[(sc4 >> (16 * (j & 1))) & 0xffu], whi = scl[(sc4 >> (16 * (j & 1) + 8)) & 0xffu];
        const v4i bv = {(int)lookup16(u0 & 0x0f0f0f0fu, c0, c1, c2, c3),
                        (int)lookup16(u1 & 0x0f0f0f0fu, c0, c1, c2, c3),
                        (int)lookup16((u0 >> 4) & 0x0f0f0f0fu, c0, c1, c2, c3),
                        (int)lookup16((u1 >> 4) & 0x0f0f0f0fu, c0, c1, c2, c3)};
        const v4i bz = {};
        const int chunk = (2 * j + kg) ^ sw;
        v16i I2[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const v4i av = *reinterpret_cast<const v4i*>(AQ + (32 * t + col) * 256 + 16 * chunk);
          I[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, kg ? bz : bv, zero, 0, 0, 0);
          I2[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, kg ? bv : bz, zero, 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const float4 d4 = *reinterpret_cast<const float4*>(dxs + j * kMT + 32 * t + 8 * r4 + 4 * kg);
            const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int r = 4 * r4 + q;
              y[t][r] += dv[q] * (wlo * (float)I[t][r] + whi * (float)I2[t][r]);
            }
          }
        continue;
      }
      // raw record j of this lane's weight row: header, then 16 nibble bytes
      const int off = T::kRec * j + T::kHdr;  // first nibble byte
      const int sh = off & 3, b4 = off - sh;
      uint32_t w0 = wld(b4), w1 = wld(b4 + 4), w2 = wld(b4 + 8), w3 = wld(b4 + 12);
      uint32_t q0 = w0, q1 = w1, q2 = w2, q3 = w3;
      if (sh) {
        const uint32_t w4 = wld(b4 + 16);
        q0 = __builtin_amdgcn_alignbyte(w1, w0, sh);
        q1 = __builtin_amdgcn_alignbyte(w2, w1, sh);
        q2 = __builtin_amdgcn_alignbyte(w3, w2, sh);
        q3 = __builtin_amdgcn_alignbyte(w4, w3, sh);
      }
      // header byte(s) just before the nibbles
      float wsc = 0.f;
      uint32_t wbits = 0;  // Q4_0 / Q4_1: the fp16 scale's bits
      if constexpr (F == WFmt::Q4_1) {
        const uint32_t hd = ld32(wrow + T::kRec * j);  // records are 4-byte aligned here
        wbits = hd & 0xffffu;
      } else if constexpr (F == WFmt::Q4_0) {
        wbits = sh >= 2 ? (w0 & 0xffffu) : (wld(b4 - 4) >> 16);
      } else {
        const uint32_t e = sh >= 1 ? ((w0 >> (8 * (sh - 1))) & 0xffu) : (ld32(wrow + b4 - 4) >> 24);
        wsc = scl[e];
      }
      const uint32_t shn = 4 * kg;  // kg 0: elements 0..15 (low nibbles), 1: 16..31 (high)
      uint32_t n[4] = {(q0 >> shn) & 0x0f0f0f0fu, (q1 >> shn) & 0x0f0f0f0fu,
                       (q2 >> shn) & 0x0f0f0f0fu, (q3 >> shn) & 0x0f0f0f0fu};
      v4i bv;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (F == WFmt::Q4_0)
          bv[i] = (int)(((n[i] | 0x80808080u) - 0x08080808u) ^ 0x80808080u);  // q - 8 per byte
        else if constexpr (F == WFmt::Q4_1)
          bv[i] = (int)n[i];  // q in 0..15
        else
          bv[i] = (int)lookup16(n[i], c0, c1, c2, c3);
      }
      const int chunk = (2 * j + kg) ^ sw;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const v4i av = *reinterpret_cast<const v4i*>(AQ + (32 * t + col) * 256 + 16 * chunk);
        I[t] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, zero, 0, 0, 0);
      }
      if constexpr (F == WFmt::Q4_0 || F == WFmt::Q4_1) {
        // y += (dx dw) I with the factor dx dw of every output from one f16
        // MFMA per tile as an outer product: K slot 0 holds the token's dx
        // and the row's dw (both fp16, so each product is exact in fp32,
        // as the VALU product it replaces), every other slot 0
        // (operands as raw bits: the kg half's slots are zero without a branch)
        const uint32_t kmask = kg ? 0u : 0xffffu;
        const v2u bq = {wbits & kmask, 0u};
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const _Float16 dxh = (_Float16)dxs[j * kMT + 32 * t + col];
          const v2u aq = {(uint32_t)__builtin_bit_cast(uint16_t, dxh) & kmask, 0u};
          const v16f qd = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, aq), __builtin_bit_cast(v4h, bq),
                                                              fzero, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 16; ++r) y[t][r] = fmaf(qd[r], (float)I[t][r], y[t][r]);
        }
        // keep the blocks' factor MFMAs in block order (hoisted, their
        // results would hold registers across the whole stage)
        __builtin_amdgcn_sched_barrier(0);
      } else {
        // y += (dx * ws) * I; register r of a tile holds token 8*(r/4) + 4*kg + r%4
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const float4 d4 = *reinterpret_cast<const float4*>(dxs + j * kMT + 32 * t + 8 * r4 + 4 * kg);
            const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int r = 4 * r4 + q;
              y[t][r] += (dv[q] * wsc) * (float)I[t][r];
            }
          }
      }
    }
    if constexpr (F == WFmt::Q4_1 && J0 == 4) {
      // Q4_1's min term, m s per block (ggml-cpu/quants.c:241), for the
      // stage's eight blocks at once: one f16 MFMA per tile (K = 8 blocks)
      // of the tokens' fp16 block sums against the rows' fp16 mins, added
      // into y.  Both are fp16, so every product is exact in fp32.
      const uint8_t* mrec = wrow + T::kRec * 4 * kg;  // blocks 4 kg .. 4 kg + 3 of this lane's row
      const uint32_t h0 = ld32(mrec), h1 = ld32(mrec + T::kRec), h2 = ld32(mrec + 2 * T::kRec),
                     h3 = ld32(mrec + 3 * T::kRec);
      const uint2 bm = make_uint2(__builtin_amdgcn_perm(h1, h0, 0x07060302u), __builtin_amdgcn_perm(h3, h2, 0x07060302u));
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint2 am = *reinterpret_cast<const uint2*>(sxs + 8 * (32 * t + col) + 4 * kg);
        y[t] = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, am), __builtin_bit_cast(v4h, bm), y[t],
                                                   0, 0, 0);
      }
    }
  };
  // A pair: the stage's first four blocks, then this wave's share of the
  // next pair's direct loads, then the last four.  Issued right after the
  // barrier, every wave's first block waited behind the workgroup's queued
  // loads (the MXFP4 GEMM measured 39.5 -> 37.8 us per call for the move).
  auto step = [&](int pair, const uint8_t* cur, uint8_t* nxt) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of this pair have landed
    __syncthreads();                // everyone's; the previous pair is consumed
    const bool refill = pair + 1 < npair;
    if (refill && wcol == 0) load_dx(pair + 1);
    const bool active = 2 * pair + par < nst;
    if (active) half(pair, cur, std::integral_constant<int, 0>{});
    if (refill) issue(pair + 1, nxt);
    if (active) half(pair, cur, std::integral_constant<int, 4>{});
    if (refill && wcol == 0) store_dx((pair + 1) & 1);  // slot last read a pair ago
  };

  issue(0, ring0);
  if (wcol == 0) {
    load_dx(0);
    store_dx(0);
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
      [](float e, float o) { return e + o; });
}

template <WFmt F, bool kGroup>
__global__ void __launch_bounds__(kThreads, 1) q80_mfma_gemm(GemmArgs a) {
  __shared__ __align__(16) uint8_t lds[q80_lds_bytes<F>()];
  q80_gemm_body<F, kGroup>(a, lds);
}

__device__ __forceinline__ float4 ldx4(const float* p, bool a16) {
  if (a16) return *reinterpret_cast<const float4*>(p);
  return make_float4(p[0], p[1], p[2], p[3]);
}

// GGML's MXFP4 tables: kvalues_mxfp4 (ggml-common.h:1116-1118) and
// ggml_e8m0_to_fp32_half (ggml-impl.h:477-495): 2^(e-128), e < 2 as fp32
// subnormals.  Thread i checks entry i; a workgroup of at least 256 threads
// covers both tables.
__device__ __forceinline__ bool ggml_mxfp4_entry(const int8_t* codebook, const float* scale, int i) {
  bool ok = true;
  if (i < 256) {
    const uint32_t bits = i < 2 ? 0x00200000u << i : (uint32_t)(i - 1) << 23;
    ok = __float_as_uint(scale[i]) == bits;
  }
  if (i < 16) {
    const int u = i & 7, kv = u < 5 ? u : u == 5 ? 6 : u == 6 ? 8 : 12;
    ok = ok && codebook[i] == ((i & 8) ? -kv : kv);
  }
  return ok;
}

// Q8_0 quantization of X (M x K) into the planar layout: row m at m * 17K/16,
// K int8 values then K/32 fp16 scales.  Same arithmetic as q8_0_quantize
// (ggml-quants.c:238-261), so the values equal the record layout's.
//
// For the MXFP4 block-scaled GEMM (kMx, and the caller passed GGML's tables)
// the int8 values are stored as sign and magnitude and in that GEMM's K
// order: byte 2i of a block holds element i, byte 2i + 1 element i + 16.
//
// kS (Q4_1's Q8_1 activation): the block sums s = fp16(sum(q) * d) follow
// the scales, K/32 fp16 more per row.
template <bool kMx, bool kS = false>
__global__ void __launch_bounds__(256) q80_planar_kernel(const float* __restrict__ X, long long ldx,
                                                         bool a16, uint8_t* __restrict__ Xp,
                                                         long long nb, int bpr, long long xs,
                                                         const int8_t* codebook, const float* scale) {
  bool kord = false;
  if constexpr (kMx) kord = __syncthreads_and(ggml_mxfp4_entry(codebook, scale, threadIdx.x)) != 0;
  const int lane = threadIdx.x & (kWave - 1);
  const long long wave = ((long long)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const long long nwaves = (long long)gridDim.x * blockDim.x / kWave;
  const long long steps = (nb + 7) / 8;
  for (long long s = wave; s < steps; s += nwaves) {
    const long long b = 8 * s + lane / 8;
    const bool live = b < nb;
    const long long row = b / bpr, blk = b - row * bpr;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) x = ldx4(X + row * ldx + 32 * blk + 4 * (lane & 7), a16);
    const Q8_0Lane r = q80_quantize_8lanes(x);
    uint32_t sh = 0;
    if constexpr (kS) sh = q81_sum_half(r);
    uint32_t word = (uint32_t)pack4_i8(r.q);
    int at = 4 * (lane & 7);
    if (kord) {
      // lane g holds elements 4g..4g+3; lanes g and g ^ 4 (elements 16
      // apart) interleave into bytes 8(g % 4) .. 8(g % 4) + 7
      uint32_t sm = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) sm |= (uint32_t)(r.q[k] < 0 ? 0x80 | -r.q[k] : r.q[k]) << (8 * k);
      const uint32_t other = (uint32_t)__shfl_xor((int)sm, 4);
      const bool upper = (lane & 4) != 0;
      word = upper ? __builtin_amdgcn_perm(sm, other, 0x07030602u) : __builtin_amdgcn_perm(other, sm, 0x05010400u);
      at = 8 * (lane & 3) + (upper ? 4 : 0);
    }
    if (!live) continue;
    uint8_t* rp = Xp + row * xs;
    *reinterpret_cast<uint32_t*>(rp + 32 * blk + at) = word;
    if ((lane & 7) == 0) *reinterpret_cast<uint16_t*>(rp + (long long)bpr * 32 + 2 * blk) = (uint16_t)r.dh;
    if (kS && (lane & 7) == 0) *reinterpret_cast<uint16_t*>(rp + (long long)bpr * 34 + 2 * blk) = (uint16_t)sh;
  }
}

// ---------------------------------------------------------------------------
// MXFP4 x Q8_0 prefill on the gfx950 block-scaled f8f6f4 MFMA.
//
// GGML's MXFP4 record is OCP MXFP4: 16 bytes of E2M1 nibbles (kvalues_mxfp4
// is twice E2M1) and an E8M0 exponent whose GGML scale is 2^(e-128).  So
// v_mfma_scale_f32_32x32x64_f8f6f4 takes the weight bytes unchanged as its
// fp4 A operand and e as the A block scale: a block contributes
// 2^(e-127) * sum E2M1(q) * x = ws * I exactly.  The activation side must be
// an 8-bit float, and a Q8_0 value (int8, |x| <= 127) is not exact in E4M3,
// so each value is split by magnitude: |x| = 16 mh + ml with mh in 0..7 and
// ml in 0..15, both planes carrying the sign of x.  With a block scale of
// 2^9 the E4M3 codes 0x00..0x0f are exactly the integers 0..15 (subnormals,
// then the first binade), so a plane's code is its magnitude with x's sign
// bit; the hi plane's block scale is 2^13 (x16).  The planar pre-pass stores
// x as a sign-and-magnitude byte (s | mh << 4 | ml), so the codes are
// lo = b & 0x8f and hi = b & 0x80 | (b >> 4) & 7: four VALU operations per
// four values.  One MFMA (K = 64) takes a 32-value weight block, twice,
// against the hi and lo planes of the matching activation block and returns
// ws * I for a 32x32 tile; the fp16 token scale is applied by one FMA per
// output and block.
//
// Operand layout (measured on the device): the weights are the fp4 A
// operand and the activation the fp8 B operand, so a lane owns one token and
// its scale is one value per block.  The fp4 operand of lane (row i, half h)
// holds K values [32h, 32h + 32) as 32 nibbles, low nibble first: both
// halves carry the same weight record.  The fp8 operand of lane (col j,
// half h) holds K values [16h, 16h + 16) of each 32-value half in dwords 0-3
// (hi plane) and 4-7 (lo plane).  Block b's scales come from lanes i + 32b /
// j + 32b.  The MFMA's K order within a block therefore pairs nibble k with
// GGML element k/2 + 16 (k%2), the order the pre-pass writes.
//
// Tiling: 64 tokens x 128 weight rows per workgroup, 8 waves = 2 column
// halves x 4 K phases.  The K loop walks pairs of stages (16 blocks, 512 K
// values); phase p takes the pair's blocks 4p .. 4p + 3 (phases 0-1 the
// first stage, 2-3 the second) and computes all four 32x32 tiles of its
// 64 x 64 quarter, so each weight operand and each split activation operand
// feeds two MFMAs.  The four phases' partial sums are added through LDS at
// the end, in phase order.  Every global byte arrives by direct
// global->LDS 16-byte loads into two pair slots, one pair ahead:
// activation rows with their 16 chunks of 16 bytes XOR-swizzled by token
// (conflict-free operand reads), the token scales block-major, and each
// weight row's 272 bytes of the pair (16 records) as four 68-byte phase
// segments at 16-byte aligned LDS offsets 80 p of a 336-byte row (five
// chunks each, the fifth ending at the segment's end; a 16-byte load needs
// only a 4-byte aligned source).  A phase then reads its four records of a
// row with four 16-byte LDS reads and one dword, at a row stride (84
// dwords) that puts 16 lanes' 16-byte reads on all 64 banks.  One barrier
// per pair.
namespace mx {

constexpr int kMT = 64;
constexpr int kNT = 128;
constexpr int kAct = kMT * 256;            // 16384: one stage's activation tile
constexpr int kRowW = 336;                 // LDS bytes per weight row and pair: 4 segments, 1 pad chunk
constexpr int kSeg = 80;                   // LDS bytes per phase segment (68 used)
constexpr int kSD = 2 * kAct;              // token scales, fp16 [stage][block pair][token][2]
constexpr int kSW = kSD + 2 * kMT * 16;    // 34816: weight rows
constexpr int kSlot = kSW + kNT * kRowW;   // 77824
constexpr int kLds = 2 * kSlot;            // 155648
constexpr int kWChunks = kRowW / 16;       // 21 chunks per LDS row
constexpr int kWLoads = kNT * kWChunks / 64;  // 42 wave-wide 16-byte loads of weights
static_assert(kNT * kWChunks % 64 == 0 && 4 * kSeg <= kRowW, "whole wave-wide weight loads");

// Exponents whose block terms the scaled MFMA reproduces.  GGML forms
// d = fp16(dx) * 2^(e-128), then sumf + d * I, each step rounded
// (ggml-cpu/quants.c:265-273); the MFMA forms 2^(e-128) * I exactly and one
// FMA adds it times dx.  With |dx| in [2^-24, 65504] and
// |I| <= 32 * 12 * 127 < 2^15.6:
//   * e >= 26 keeps d and 2^(e-128) I normal, so both sides round the same
//     real product once;
//   * e <= 224 keeps |2^(e-128) I dx| < 2^128, so no finite product
//     overflows (the FMA does not round its product: an overflow that GGML
//     turns into inf before the add would be lost against an inf already in
//     the sum).  An inf dx gives inf, or NaN for I = 0, on both sides.
// Other exponents (e = 255, whose 2^127 has no E8M0 block-scale encoding,
// included) take GGML's order.
constexpr uint32_t kSafeLo = 26, kSafeHi = 224;
static_assert(8 * 4 * 16 * 64 * 4 <= kLds, "partial sums fit the ring");

// 16 bytes per lane from sbase + voff into [lds + 16 lane, +16)
__device__ __forceinline__ void dma16_s(const uint8_t* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(lds), "v"(voff), "s"(sbase)
               : "memory", "m0");
}

// LDS-only barrier: outstanding direct loads stay in flight
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

typedef int v8i __attribute__((ext_vector_type(8)));

// y += dx * d for a tile whose MFMA applied the block scales
__device__ __forceinline__ v16f fma_block(v16f y, v16f d, float dx) {
#pragma unroll
  for (int r = 0; r < 16; ++r) y[r] = fmaf(d[r], dx, y[r]);
  return y;
}

// A tile computed at unit block scale (d = I / 2 exactly), combined in
// GGML's order: register r holds weight row 8 (r / 4) + 4 h + r % 4 of the
// tile, whose exponent byte sits at LDS address e0 + kRowW (8 (r / 4) + r % 4)
// (e0: the exponent of row 4 h).
__device__ __forceinline__ v16f ggml_block_terms(v16f y, v16f d, float dx, uint32_t e0) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const uint32_t er =
        *(const __attribute__((address_space(3))) uint8_t*)(size_t)(e0 + kRowW * (8 * (r >> 2) + (r & 3)));
    y[r] = ggml_scaled_term(y[r], dx, e8m0_half(er), 2.f * d[r]);
  }
  return y;
}

template <bool kGroup>
__device__ void scaled_body(const GemmArgs& a, uint8_t* lds) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int cp = wave & 1, ph = wave >> 1;  // column half, K phase
  const int col = lane & 31, h = lane >> 5;
  const int nst = a.K >> 8;
  const uint32_t xs = (uint32_t)a.K + (uint32_t)a.K / 16;  // planar activation row stride
  const uint32_t ws_row = (uint32_t)a.ldw;  // the host keeps a tile's rows in 32-bit offsets

  int m0, n0, mrows;
  const uint8_t* W = a.W;
  {
    const int ntm = kGroup ? a.grp.tmax : (a.M + kMT - 1) / kMT;
    const int Tn = ntm * ((a.N + kNT - 1) / kNT);
    const int L = blockIdx.x, x = L & 7, j = L >> 3;
    const int t = x * (Tn >> 3) + min(x, Tn & 7) + j;
    n0 = __builtin_amdgcn_readfirstlane((t / ntm) * kNT);
    if constexpr (kGroup) {
      long long w_off;
      if (!group_tile(a.grp, t % ntm, m0, mrows, w_off)) return;  // no barrier yet
      W += w_off;
    } else {
      m0 = __builtin_amdgcn_readfirstlane((t % ntm) * kMT);
      mrows = min(kMT, a.M - m0);
    }
  }
  // grouped: rows are gathered, offsets from Xp itself (the host keeps the
  // planar activation within 32-bit offsets)
  const uint8_t* xbase = kGroup ? a.Xp : a.Xp + (size_t)m0 * xs;
  const uint8_t* wbase = W + (size_t)n0 * ws_row;
  const int mlast = mrows - 1, nlast = a.N - 1 - n0;
  auto act_row = [&](int r) -> uint32_t {
    if constexpr (kGroup)
      return (uint32_t)group_act_row(a.grp, m0, r);
    else
      return (uint32_t)r;
  };

  // Load plan per pair: 2 x 16 activation loads (1 KB = 4 tokens each), 8
  // dword loads of the token scales (stage w / 4, block pair w % 4 of 64
  // tokens: wave w), then the weight rows.  Rows past M / N repeat the last
  // row.
  auto act_off = [&](int c) {
    const int q = 64 * c + lane, t = q >> 4, s = q & 15;
    return act_row(min(t, mlast)) * xs + 16 * (uint32_t)(s ^ (t & 15));
  };
  const uint32_t va0 = act_off(wave), va1 = act_off(wave + 8);
  const uint32_t vsc = act_row(min(lane, mlast)) * xs + (uint32_t)a.K + 4 * (uint32_t)(wave & 3);
  // weight chunks: load k = wave + 8 i (< 42) covers LDS chunks q = 64 k + lane:
  // row q / 21, chunk c = q % 21 = 5 s + j of segment s (c = 20: the pad,
  // a copy of s = 3, j = 4); chunk j < 4 holds segment bytes 16 j .. +15,
  // chunk 4 bytes 52 .. 67.  A single last stage has only segments 0-1:
  // segments 2-3 then copy them (in the row; no phase reads them).
  auto w_off = [&](int k, bool tail) {
    const int q = 64 * min(k, kWLoads - 1) + lane, row = q / kWChunks, c = q - kWChunks * row;
    const int sg = min(c / 5, 3), j = c - 5 * sg;
    return (uint32_t)min(row, nlast) * ws_row + 68 * (uint32_t)(tail ? sg & 1 : sg) + (j < 4 ? 16 * j : 52);
  };
  uint32_t vw[6];
#pragma unroll
  for (int i = 0; i < 6; ++i) vw[i] = w_off(wave + 8 * i, false);

  // LDS byte addresses as integers from one wave-uniform base: no per-use
  // generic-to-LDS pointer casts (their null checks on VALU do not compile)
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  // a pair with both stages (every pair but an odd K's last): the loads
  // without the tail offsets
  auto issue_pair = [&](int p) {
    const uint32_t slot = lds0 + (uint32_t)(p & 1) * kSlot;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const uint8_t* xb = xbase + 256 * (size_t)(2 * p + s);
      dma16_s(xb, va0, slot + kAct * s + 1024 * wave);
      dma16_s(xb, va1, slot + kAct * s + 1024 * (wave + 8));
    }
    lds_dma4_s(xbase + 16 * (size_t)(2 * p + (wave >> 2)), vsc, slot + kSD + 256 * wave);
    const uint8_t* wb = wbase + 272 * (size_t)p;
#pragma unroll
    for (int i = 0; i < 6; ++i)
      if (wave + 8 * i < kWLoads) dma16_s(wb, vw[i], slot + kSW + 1024 * (wave + 8 * i));
  };
  auto issue = [&](int p) {
    const uint32_t slot = lds0 + (uint32_t)(p & 1) * kSlot;
    const bool both = 2 * p + 1 < nst;  // the pair's second stage exists
#pragma unroll
    for (int s = 0; s < 2; ++s)
      if (s == 0 || both) {
        const uint8_t* xb = xbase + 256 * (size_t)(2 * p + s);
        dma16_s(xb, va0, slot + kAct * s + 1024 * wave);
        dma16_s(xb, va1, slot + kAct * s + 1024 * (wave + 8));
      }
    if (wave < 4 || both) lds_dma4_s(xbase + 16 * (size_t)(2 * p + (wave >> 2)), vsc, slot + kSD + 256 * wave);
    const uint8_t* wb = wbase + 272 * (size_t)p;
#pragma unroll
    for (int i = 0; i < 6; ++i)
      if (wave + 8 * i < kWLoads)
        dma16_s(wb, both ? vw[i] : w_off(wave + 8 * i, true), slot + kSW + 1024 * (wave + 8 * i));
  };

  v16f y[4];  // tile 2 * token half + column tile
#pragma unroll
  for (int q = 0; q < 4; ++q) y[q] = v16f{};
  const v16f fzero = {};
  const int x_scale = h ? 127 + 9 : 127 + 13;  // B block 0: hi plane (x16), block 1: lo plane
  const int sp = ph >> 1;                      // the phase's stage within a pair

  // Blocks J0, J0 + 1 of the phase's four blocks of pair p.  kExact false:
  // every tile takes its exponent e as the hardware block scale, and `out`
  // collects whether any e lies outside [kSafeLo, kSafeHi] (the results are
  // then discarded).  kExact true: a column tile whose 32 rows all have
  // exponents in range does the same; otherwise (wave-uniform) its MFMA runs
  // at unit scale and the block is combined in GGML's order.
  auto phase_blocks = [&](int p, auto exact_tag, bool& out, auto j0_tag) {
    constexpr bool kExact = decltype(exact_tag)::value;
    constexpr int J0 = decltype(j0_tag)::value;
    const uint8_t* slot = lds + (p & 1) * kSlot;
    const uint32_t slot_lds = lds0 + (uint32_t)(p & 1) * kSlot;
    // of the 17 dwords holding records 4 ph .. 4 ph + 3 of rows
    // 64 cp + 32 ct + col (four 16-byte reads and the segment's last dword,
    // at byte 76 of its copy), those of records J0 and J0 + 1: bytes
    // [17 J0, 17 J0 + 34)
    uint32_t wd[2][17];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const uint8_t* wr = slot + kSW + kRowW * (64 * cp + 32 * ct + col) + kSeg * ph;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (16 * i + 16 <= 17 * J0 || 16 * i >= 17 * J0 + 34) continue;
        const uint4 v = *reinterpret_cast<const uint4*>(wr + 16 * i);
        wd[ct][4 * i] = v.x, wd[ct][4 * i + 1] = v.y, wd[ct][4 * i + 2] = v.z, wd[ct][4 * i + 3] = v.w;
      }
      if (J0 == 2) wd[ct][16] = ld32(wr + 76);
    }
#pragma unroll
    for (int j = J0; j < J0 + 2; ++j) {
      const int bs = 4 * (ph & 1) + j;  // block within stage sp
      // record j: e at byte 17 j, then 16 nibble bytes
      constexpr int kE[4] = {0, 17, 34, 51};
      const int n0b = kE[j] + 1, dw0 = n0b >> 2, sh = n0b & 3;
      v8i wv[2];
      int wsc[2];
      bool exact[2] = {false, false};
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        const uint32_t e = (wd[ct][kE[j] >> 2] >> (8 * (kE[j] & 3))) & 0xffu;
        const bool unsafe = e - kSafeLo > kSafeHi - kSafeLo;  // unsigned
        if constexpr (kExact)
          exact[ct] = __builtin_amdgcn_ballot_w64(unsafe) != 0;
        else
          out |= unsafe;
        wsc[ct] = exact[ct] ? 127 : (int)e;
        const uint32_t* w = &wd[ct][dw0];
        wv[ct] = sh ? v8i{(int)__builtin_amdgcn_alignbyte(w[1], w[0], sh), (int)__builtin_amdgcn_alignbyte(w[2], w[1], sh),
                          (int)__builtin_amdgcn_alignbyte(w[3], w[2], sh), (int)__builtin_amdgcn_alignbyte(w[4], w[3], sh),
                          0, 0, 0, 0}
                    : v8i{(int)w[0], (int)w[1], (int)w[2], (int)w[3], 0, 0, 0, 0};
      }
      v8i xv[2];
      float dx[2];
#pragma unroll
      for (int th = 0; th < 2; ++th) {
        const int t = 32 * th + col;
        const uint4 raw =
            *reinterpret_cast<const uint4*>(slot + kAct * sp + 256 * t + 16 * ((2 * bs + h) ^ (col & 15)));
        const uint32_t rw[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          xv[th][k] = (int)(((rw[k] >> 4) & 0x07070707u) | (rw[k] & 0x80808080u));
          xv[th][4 + k] = (int)(rw[k] & 0x8f8f8f8fu);
        }
        dx[th] = (float)*reinterpret_cast<const _Float16*>(slot + kSD + 1024 * sp + 4 * (64 * (bs >> 1) + t) +
                                                            2 * (bs & 1));
      }
      // four independent MFMAs in flight, then y += dx * (ws * I)
      v16f d[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        d[q] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wv[q & 1], xv[q >> 1], fzero, 4, 0, 0, wsc[q & 1], 0,
                                                               x_scale);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int ct = q & 1;
        if (kExact && exact[ct])  // wave-uniform
          y[q] = ggml_block_terms(y[q], d[q], dx[q >> 1],
                                  slot_lds + kSW + kRowW * (64 * cp + 32 * ct + 4 * h) + kSeg * ph + kE[j]);
        else
          y[q] = fma_block(y[q], d[q], dx[q >> 1]);
      }
    }
  };

  // The K loop.  The direct loads of the next pair go into the slot the
  // previous pair used (free after the barrier), and each wave waits for all
  // of its own loads (vmcnt 0) at the top of a pair.  A wave issues its share
  // between its phase's second and third blocks: issued right after the
  // barrier, every wave's first block waited behind the workgroup's ~80
  // queued loads (39.5 -> 37.8 us per call at 512 x 4096 x 4096); issued
  // after the third block or spread over the blocks they land too late for
  // the next barrier.  An odd K's last pair (one stage) is issued at the top.
  const int npair = (nst + 1) >> 1;
  auto kloop = [&](auto exact_tag, bool& out) {
    issue(0);
    for (int p = 0; p < npair; ++p) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      lds_barrier();  // the pair is in for every wave; the previous pair's slot is free
      const bool next = p + 1 < npair, full = 2 * (p + 1) + 1 < nst;
      if (next && !full) issue(p + 1);
      const bool active = 2 * p + sp < nst;
      if (active) phase_blocks(p, exact_tag, out, std::integral_constant<int, 0>{});
      if (next && full) issue_pair(p + 1);
      if (active) phase_blocks(p, exact_tag, out, std::integral_constant<int, 2>{});
    }
  };
  // Weights quantized by GGML keep every exponent in range, and the loop
  // without per-tile branches runs once.  A workgroup that met an exponent
  // out of range runs the K loop again with GGML's order for those tiles.
  bool out = false;
  kloop(std::integral_constant<bool, false>{}, out);
  if (__syncthreads_or(out)) {  // also: every wave is done with the ring
#pragma unroll
    for (int q = 0; q < 4; ++q) y[q] = v16f{};
    kloop(std::integral_constant<bool, true>{}, out);
  }

  // partial sums of the four K phases -> LDS; wave (cp, p) finishes tile p
  __syncthreads();
  float4* red = reinterpret_cast<float4*>(lds);
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
      red[((wave * 4 + q) * 4 + r4) * 64 + lane] =
          make_float4(y[q][4 * r4], y[q][4 * r4 + 1], y[q][4 * r4 + 2], y[q][4 * r4 + 3]);
  __syncthreads();
  const int q = ph, th = q >> 1, ct = q & 1;
  const int rr = 32 * th + col;
  const bool v4 = (kGroup ? ((a.grp.y_s1 | a.grp.y_s2) & 3) == 0 : (a.ldy & 3) == 0) &&
                  (reinterpret_cast<uintptr_t>(a.Y) & 15) == 0;
#pragma unroll
  for (int r4 = 0; r4 < 4; ++r4) {
    float4 v = red[(((cp + 0) * 4 + q) * 4 + r4) * 64 + lane];
#pragma unroll
    for (int p2 = 1; p2 < 4; ++p2) {
      const float4 u = red[(((cp + 2 * p2) * 4 + q) * 4 + r4) * 64 + lane];
      v.x += u.x;
      v.y += u.y;
      v.z += u.z;
      v.w += u.w;
    }
    // register r holds weight row 8*(r/4) + 4*h + r%4 of the tile
    const int gn = n0 + 64 * cp + 32 * ct + 8 * r4 + 4 * h;
    if (rr < mrows) {
      float* yr = a.Y + (kGroup ? group_dst_row(a.grp, m0, rr) : (long long)(m0 + rr) * a.ldy);
      if (v4 && gn + 3 < a.N) {
        *reinterpret_cast<float4*>(yr + gn) = v;
      } else {
        const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (gn + k < a.N) yr[gn + k] = vv[k];
      }
    }
  }
}

}  // namespace mx

constexpr int kMxLds = mx::kLds > q80_lds_bytes<WFmt::MXFP4>() ? mx::kLds : q80_lds_bytes<WFmt::MXFP4>();

// The block-scaled MFMA computes with GGML's tables; with any other tables
// the workgroup runs the int8 body, which looks every value up.
template <bool kGroup>
__global__ void __launch_bounds__(kThreads, 1) mxfp4_gemm(GemmArgs a) {
  __shared__ __align__(16) uint8_t lds[kMxLds];
  if (__syncthreads_and(ggml_mxfp4_entry(a.codebook, a.scale, threadIdx.x)))
    mx::scaled_body<kGroup>(a, lds);
  else
    q80_gemm_body<WFmt::MXFP4, kGroup>(a, lds);
}

// Q8_0 quantization of M rows of X (ldx floats apart) into the planar layout
template <WFmt F>
void planar_pass(const float* X, size_t ldx, uint8_t* Xp, size_t M, size_t K, const int8_t* codebook,
                 const float* scale) {
  const long long nb = (long long)(M * K / 32);
  const long long xs = (long long)planar_row_bytes<F>(K);
  const long long waves = (nb + 7) / 8;
  const int grid = (int)std::max<long long>(1, std::min<long long>((long long)cu_count() * 8, (waves + 3) / 4));
  const bool a16 = aligned(X, 16) && ldx % 4 == 0;
  q80_planar_kernel<F == WFmt::MXFP4, F == WFmt::Q4_1><<<grid, 256, 0, current_stream()>>>(
      X, (long long)ldx, a16, Xp, nb, (int)(K / 32), xs, codebook, scale);
  check_launch("q80_planar_kernel");
}

template <WFmt F>
bool prefill_q80(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                 const float* scale, float* Y, size_t N, size_t K, size_t M, const RowStrides& st) {
  using T = WTraits<F>;
  const size_t rb = K / 32 * T::kRec;
  const size_t ldw = N > 1 ? st.ldw : rb;
  // MFMA path preconditions; otherwise the caller runs the GEMV kernels.
  // Weight rows feed dword direct-to-LDS loads (4-byte aligned) and a tile's
  // rows must stay within 32-bit offsets.
  // Below 16 activation rows the GEMV kernels run, unless their LDS cannot
  // hold a row of K values.
  constexpr int kGemvFmt = F == WFmt::Q4_0 ? 0 : F == WFmt::MXFP4 ? 1 : F == WFmt::Q4_1 ? 6 : 5;
  if ((M < 16 && staged_gemv_fits(kGemvFmt, K)) || K % 256 || !aligned(W, 4) || ldw % 4 != 0 ||
      (kNT - 1) * ldw + rb >= ((size_t)1 << 32) || !aligned(Xq, 16) || !aligned(Y, 4) || !aligned(X, 4) ||
      N > (size_t)INT32_MAX || K > (size_t)INT32_MAX || M > (size_t)INT32_MAX ||
      !strides_ok(st, rb, 1, K, N, N, M) ||
      ((N + kNT - 1) / kNT) * ((M + kMT - 1) / kMT) > (size_t)INT32_MAX)
    return false;
  if (has_table<F>() && (codebook == nullptr || scale == nullptr)) return false;
  const size_t ldx = M > 1 ? st.ldx : K;
  planar_pass<F>(X, ldx, Xq, M, K, codebook, scale);
  const size_t tiles = ((N + kNT - 1) / kNT) * ((M + kMT - 1) / kMT);
  GemmArgs ga{W, Xq, codebook, scale, Y, (int)N, (int)K, (int)M, ldw, (long long)st.ldy, GroupTiles{}};
  if constexpr (F == WFmt::MXFP4) {
    mxfp4_gemm<false><<<dim3((unsigned)tiles), kThreads, 0, current_stream()>>>(ga);
  } else {
    q80_mfma_gemm<F, false><<<dim3((unsigned)tiles), kThreads, 0, current_stream()>>>(ga);
  }
  check_launch(F == WFmt::MXFP4 ? "mxfp4_gemm" : F == WFmt::NVFP4 ? "nvfp4_mfma_gemm" : "q80_mfma_gemm");
  // Xq ends in GGML's record layout
  if constexpr (F == WFmt::Q4_1)
    quantize_q8_1_rows(X, ldx, Xq, M, K);
  else
    quantize_q8_0_rows(X, ldx, Xq, M, K);
  return true;
}

}  // namespace

// MUL_MAT_ID on the grouped GEMMs (Q4_0: fmt 0, MXFP4: fmt 1, NVFP4: fmt 2,
// Q4_1: fmt 3, whose activation is Q8_1).  X rows
// (token t, row j) at t * x_s2 + j * x_s1 floats are quantized into Xq
// planar, then in GGML's records after the GEMM, as the dense path does.
bool mul_mat_id_q80_grouped_ok(int fmt, const uint8_t* W, const float* X, const uint8_t* Xq, const float* Y,
                               size_t N, size_t K, const RowStrides& st, const PairArgs& pr, int n_pairs,
                               int n_tok, const void* ws, size_t ws_bytes, const int8_t* codebook,
                               const float* scale) {
  const size_t rb = K / 32 * (fmt == 0 ? kQ4_0Bytes : fmt == 1 ? kMxfp4Bytes : fmt == 2 ? kNvfp4Bytes / 2 : kQ4_1Bytes);
  const size_t ldw = N > 1 ? st.ldw : rb;
  const size_t xq_bytes = (size_t)n_tok * pr.ne11 * (K / 32) * (fmt == 3 ? kQ8_1Bytes : kQ8_0Bytes);
  return N > 0 && K > 0 && n_pairs > 0 && K % 256 == 0 && X != nullptr && aligned(X, 4) &&
         aligned(W, 4) && ldw % 4 == 0 && (kNT - 1) * ldw + rb < ((size_t)1 << 32) &&
         aligned(Xq, 16) && xq_bytes < ((size_t)1 << 32) && aligned(Y, 4) && aligned(ws, 16) &&
         ws_bytes >= moe_group_bytes(n_pairs, pr.n_as) && pr.w_es % 4 == 0 &&
         pr.n_as <= kMaxExperts && N <= (size_t)INT32_MAX && K <= (size_t)INT32_MAX &&
         strides_ok(st, rb, 1, K, N, N, 1) && (fmt == 0 || fmt == 3 || (codebook != nullptr && scale != nullptr)) &&
         (size_t)moe_tile_bound(n_pairs, pr.n_as) * ((N + kNT - 1) / kNT) <= (size_t)INT32_MAX;
}

void mul_mat_id_q80_grouped(int fmt, const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N,
                            size_t K, const RowStrides& st, const PairArgs& pr, int n_pairs, int n_tok,
                            void* ws, const int8_t* codebook, const float* scale) {
  const size_t rb = K / 32 * (fmt == 0 ? kQ4_0Bytes : fmt == 1 ? kMxfp4Bytes : fmt == 2 ? kNvfp4Bytes / 2 : kQ4_1Bytes);
  const size_t rows = (size_t)n_tok * pr.ne11;
  const size_t xs = fmt == 3 ? planar_row_bytes<WFmt::Q4_1>(K) : planar_row_bytes<WFmt::Q4_0>(K);
  // rows (t, j) of X at t * x_s2 + j * x_s1: one pass when they are evenly
  // spaced, else one per token
  auto each_plane = [&](auto&& pass, size_t row_bytes) {
    if (pr.ne11 == 1) return pass(X, n_tok > 1 ? (size_t)pr.x_s2 : K, Xq, (size_t)n_tok);
    if (n_tok == 1 || pr.x_s2 == (long long)pr.ne11 * pr.x_s1) return pass(X, (size_t)pr.x_s1, Xq, rows);
    for (int t = 0; t < n_tok; ++t)
      pass(X + (size_t)t * pr.x_s2, (size_t)pr.x_s1, Xq + (size_t)t * pr.ne11 * row_bytes, (size_t)pr.ne11);
  };
  each_plane([&](const float* x, size_t l, uint8_t* xp, size_t m) {
    if (fmt == 1)
      planar_pass<WFmt::MXFP4>(x, l, xp, m, K, codebook, scale);
    else if (fmt == 3)
      planar_pass<WFmt::Q4_1>(x, l, xp, m, K, nullptr, nullptr);
    else
      planar_pass<WFmt::Q4_0>(x, l, xp, m, K, nullptr, nullptr);  // the plain int8 planar layout
  }, xs);
  const MoeGroups g = moe_group(pr, n_pairs, ws);
  GemmArgs ga{W, Xq, codebook, scale, Y, (int)N, (int)K, kMT, N > 1 ? st.ldw : rb, 0, group_tiles(g, pr)};
  const size_t wgs = (size_t)g.tmax * ((N + kNT - 1) / kNT);
  if (fmt == 0)
    q80_mfma_gemm<WFmt::Q4_0, true><<<dim3((unsigned)wgs), kThreads, 0, current_stream()>>>(ga);
  else if (fmt == 1)
    mxfp4_gemm<true><<<dim3((unsigned)wgs), kThreads, 0, current_stream()>>>(ga);
  else if (fmt == 2)
    q80_mfma_gemm<WFmt::NVFP4, true><<<dim3((unsigned)wgs), kThreads, 0, current_stream()>>>(ga);
  else
    q80_mfma_gemm<WFmt::Q4_1, true><<<dim3((unsigned)wgs), kThreads, 0, current_stream()>>>(ga);
  check_launch(fmt == 1 ? "mxfp4_gemm" : fmt == 2 ? "nvfp4_mfma_gemm" : "q80_mfma_gemm");
  // Xq ends in GGML's record layout
  if (fmt == 3)
    each_plane([&](const float* x, size_t l, uint8_t* xq, size_t m) { quantize_q8_1_rows(x, l, xq, m, K); },
               (K / 32) * kQ8_1Bytes);
  else
    each_plane([&](const float* x, size_t l, uint8_t* xq, size_t m) { quantize_q8_0_rows(x, l, xq, m, K); },
               (K / 32) * kQ8_0Bytes);
}

bool gemm_q80_try(int fmt, const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                  const float* scale, float* Y, size_t N, size_t K, size_t M, const RowStrides& st) {
  if (N == 0 || M == 0 || K == 0 || W == nullptr || X == nullptr || Xq == nullptr || Y == nullptr) return false;
  switch (fmt) {
    case 0: return prefill_q80<WFmt::Q4_0>(W, X, Xq, nullptr, nullptr, Y, N, K, M, st);
    case 1: return prefill_q80<WFmt::MXFP4>(W, X, Xq, codebook, scale, Y, N, K, M, st);
    case 5: return prefill_q80<WFmt::NVFP4>(W, X, Xq, codebook, scale, Y, N, K, M, st);
    case 6: return prefill_q80<WFmt::Q4_1>(W, X, Xq, nullptr, nullptr, Y, N, K, M, st);
    default: return false;
  }
}

void mul_mat_q4_0(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                  size_t M, const RowStrides& st) {
  if (N == 0 || M == 0 || K == 0) return decode_q4_0(W, X, Xq, Y, N, K, M, st);
  if (W == nullptr || X == nullptr || Xq == nullptr || Y == nullptr ||
      !prefill_q80<WFmt::Q4_0>(W, X, Xq, nullptr, nullptr, Y, N, K, M, st))
    decode_q4_0(W, X, Xq, Y, N, K, M, st);
}

void mul_mat_q4_1(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                  size_t M, const RowStrides& st) {
  if (N == 0 || M == 0 || K == 0) return decode_q4_1(W, X, Xq, Y, N, K, M, st);
  if (W == nullptr || X == nullptr || Xq == nullptr || Y == nullptr ||
      !prefill_q80<WFmt::Q4_1>(W, X, Xq, nullptr, nullptr, Y, N, K, M, st))
    decode_q4_1(W, X, Xq, Y, N, K, M, st);
}

void mul_mat_nvfp4(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                   const float* ue4m3, float* Y, size_t N, size_t K, size_t M, const RowStrides& st) {
  if (N == 0 || M == 0 || K == 0) return decode_nvfp4(W, X, Xq, codebook, ue4m3, Y, N, K, M, st);
  if (W == nullptr || X == nullptr || Xq == nullptr || Y == nullptr ||
      !prefill_q80<WFmt::NVFP4>(W, X, Xq, codebook, ue4m3, Y, N, K, M, st))
    decode_nvfp4(W, X, Xq, codebook, ue4m3, Y, N, K, M, st);
}

void mul_mat_mxfp4(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                   const float* scale, float* Y, size_t N, size_t K, size_t M, const RowStrides& st) {
  if (N == 0 || M == 0 || K == 0) return decode_mxfp4(W, X, Xq, codebook, scale, Y, N, K, M, st);
  if (W == nullptr || X == nullptr || Xq == nullptr || Y == nullptr ||
      !prefill_q80<WFmt::MXFP4>(W, X, Xq, codebook, scale, Y, N, K, M, st))
    decode_mxfp4(W, X, Xq, codebook, scale, Y, N, K, M, st);
}

}  // namespace weft
