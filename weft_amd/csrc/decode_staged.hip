// Decode GEMV for the formats whose records are not 16-byte multiples:
// Q4_0 x Q8_0 (18 B / 32), MXFP4 x Q8_0 (17 B / 32), IQ2_XXS x Q8_K
// (66 B / 256), Q6_K x Q8_K (210 B / 256), Q5_K x Q8_K (176 B / 256),
// NVFP4 x Q8_0 (36 B / 64), Q4_1 x Q8_1 (20 B / 32), IQ2_XS x Q8_K
// (74 B / 256); plus their single-output vec_dots.
//
// Semantics (GGML generic vec_dots, ggml-cpu/quants.c):
//   Q4_0    :174-208  y = sum_b dw_b * dx_b * sum_32 (q-8) * x
//   MXFP4   :247-276  y = sum_b dx_b * e8m0_half(e_b) * sum_32 kv[q] * x
//   IQ2_XXS :855-895  y = 0.125 * sum_B dw * dx * sum_g (2 s_g + 1) *
//                         sum_32 grid[idx] * sign * x
//   Q6_K    :800-853  y = sum_B dw * dx * sum_g sc_g * sum_16 (q - 32) * x
//   NVFP4   ggml-cpu/quants.c:279-313  y = sum_B sum_s dx * ue4m3(d_s) * sum_16 kv[q] * x
//   Q5_K    :720-798  y = sum_B dx * (dw * sum_s sc_s * sum_32 q * x
//                                    - dmin * sum_s m_s * bsum_s)
//   Q4_1    :211-245  y = sum_b (dw_b dx_b) sum_32 q x + m_b s_b
//   IQ2_XS  :897-946  y = 0.125 * sum_B dw * dx * sum_h (2 s_h + 1) *
//                         sum_16 grid[idx] * sign * x   (h: 16-element halves)
// and the Weft kernels examples/kernels/mul_mat/{q4_0_decode,mxfp4_decode,
// iq2_xxs_decode}.py (quantize X into Xq, then one vec_dot per output).
//
// gfx950 mapping.  Records straddle 16-byte boundaries, so a wave streams
// its rows segment by segment (up to ~2.3 KB) through a private LDS window:
// coalesced 16-byte loads into registers, one segment ahead of the one being
// computed, then into the window, where lanes pick their record out at any
// byte offset with two aligned ds_read_b32 + v_alignbyte per word.  One
// lane owns one 32-element block (Q4_0, MXFP4) or one 32-element group of an
// IQ2_XXS superblock; its int8 products run on v_dot4_i32_i8 against the
// quantized activation in LDS.  MXFP4's 16-entry codebook is looked up four
// nibbles at a time with two v_perm_b32; the IQ2_XXS grid and sign tables
// live in LDS.  The activation is quantized inside every workgroup, and
// workgroup 0 writes Xq, exactly as in the Q4_K decode kernel.
#include <algorithm>

#include "activation.h"
#include "kernels.h"
#include "pairs.h"
#include "runtime.h"
#include "weft_hip.h"

namespace weft {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxRowsPerPass = 4;
// per-wave LDS window (bytes), with slack.  A wave keeps one segment in
// flight while it computes the previous one, so the window sets the bytes in
// flight per CU (16 waves x ~4.5 KB): with ~2 us of loaded HBM latency,
// 2.3 KB windows held Q5_K / Q6_K near 2.3-2.7 TB/s.
constexpr int kWindow = 4608 + 32;

enum class Fmt { Q4_0, MXFP4, IQ2_XXS, Q6_K, Q5_K, NVFP4, Q4_1, IQ2_XS };

template <Fmt F>
struct Traits;
template <>
struct Traits<Fmt::Q4_0> {
  static constexpr int kElems = 32, kBytes = 18, kSegRecords = 256, kItemsPerRecord = 1;
  static constexpr bool kQ8K = false;
};
template <>
struct Traits<Fmt::MXFP4> {
  static constexpr int kElems = 32, kBytes = 17, kSegRecords = 256, kItemsPerRecord = 1;
  static constexpr bool kQ8K = false;
};
template <>
struct Traits<Fmt::IQ2_XXS> {
  static constexpr int kElems = 256, kBytes = 66, kSegRecords = 64, kItemsPerRecord = 8;
  static constexpr bool kQ8K = true;
};
template <>
struct Traits<Fmt::Q6_K> {
  static constexpr int kElems = 256, kBytes = 210, kSegRecords = 16, kItemsPerRecord = 4;
  static constexpr bool kQ8K = true;
};
template <>
struct Traits<Fmt::NVFP4> {
  static constexpr int kElems = 64, kBytes = 36, kSegRecords = 128, kItemsPerRecord = 1;
  static constexpr bool kQ8K = false;
};
template <>
struct Traits<Fmt::Q5_K> {
  static constexpr int kElems = 256, kBytes = 176, kSegRecords = 16, kItemsPerRecord = 4;
  static constexpr bool kQ8K = true;
};

template <>
struct Traits<Fmt::Q4_1> {
  static constexpr int kElems = 32, kBytes = 20, kSegRecords = 224, kItemsPerRecord = 1;
  static constexpr bool kQ8K = false;
};
template <>
struct Traits<Fmt::IQ2_XS> {
  static constexpr int kElems = 256, kBytes = 74, kSegRecords = 56, kItemsPerRecord = 8;
  static constexpr bool kQ8K = true;
};

// Q4_1 pairs with the Q8_1 activation (block sums s), every other 32-element
// format with Q8_0
template <Fmt F>
constexpr bool act_q81() {
  return F == Fmt::Q4_1;
}
// LDS for lookup tables: IQ2_XS's 512 x 8 grid and 128 x 8 signs, else 3 KB
template <Fmt F>
constexpr int table_bytes() {
  return F == Fmt::IQ2_XS ? 6144 : F == Fmt::IQ2_XXS ? 4096 : 3072;
}

struct Args {
  const uint8_t* W;
  const float* X;
  const uint8_t* xq_in;
  uint8_t* xq_out;
  const int8_t* tab0;  // grid (IQ2_XXS) or codebook (MXFP4)
  const void* tab1;    // signs (IQ2_XXS) or fp32 scale table (MXFP4)
  float* Y;
  int N, K;
  int m0, mb;
  int rows_per_wg;
  long long y_stride;
  size_t ldw;  // bytes between weight rows
  size_t ldx;  // elements between activation rows
  PairArgs pair;  // MUL_MAT_ID pairs (pair.ids null: none)
  int accumulate;  // K chunk after the first: add to Y instead of storing
};

// 4 bytes starting at any LDS byte offset o (o+7 must be inside the buffer)
__device__ __forceinline__ uint32_t lds_u32(const char* base, int o) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(base + (o & ~3));
  return __builtin_amdgcn_alignbyte(w[1], w[0], (uint32_t)(o & 3));
}

// n consecutive 4-byte values from LDS byte offset o (any alignment): n + 1
// aligned word reads and n byte-aligns (o + 4n + 3 inside the buffer)
template <int n>
__device__ __forceinline__ void lds_run(const char* base, int o, uint32_t (&v)[n]) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(base + (o & ~3));
  const uint32_t sh = (uint32_t)(o & 3);
  uint32_t t[n + 1];
#pragma unroll
  for (int i = 0; i <= n; ++i) t[i] = w[i];
#pragma unroll
  for (int i = 0; i < n; ++i) v[i] = __builtin_amdgcn_alignbyte(t[i + 1], t[i], sh);
}

// One segment of a row staged through registers, so the next segment's loads
// are in flight while the current one is computed from LDS: fetch() issues
// the 16-byte loads of bytes [p0, p1) (chunks reaching outside [lo, hi) are
// read byte by byte, inside only), put() writes them into the wave's window
// and returns the offset of p0 inside it.
constexpr int kChunksPerLane = (kWindow / 16 + kWave - 1) / kWave;

struct SegmentFetch {
  uint4 c[kChunksPerLane];
  int nchunks, off;

  __device__ __forceinline__ void fetch(const uint8_t* p0, const uint8_t* p1, const uint8_t* lo,
                                        const uint8_t* hi, int lane) {
    const uint8_t* a0 = reinterpret_cast<const uint8_t*>(reinterpret_cast<uintptr_t>(p0) & ~(uintptr_t)15);
    nchunks = (int)((p1 - a0 + 15) >> 4);
    off = (int)(p0 - a0);
#pragma unroll
    for (int j = 0; j < kChunksPerLane; ++j) {
      const int ch = lane + kWave * j;
      const uint8_t* src = a0 + 16 * ch;
      if (ch >= nchunks) {
        c[j] = make_uint4(0, 0, 0, 0);
      } else if (src >= lo && src + 16 <= hi) {
        c[j] = *reinterpret_cast<const uint4*>(src);
      } else {
        uint32_t w[4] = {0, 0, 0, 0};
        for (int i = 0; i < 16; ++i)
          if (src + i >= lo && src + i < hi) w[i >> 2] |= (uint32_t)src[i] << (8 * (i & 3));
        c[j] = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
  }

  __device__ __forceinline__ int put(char* win, int lane) const {
#pragma unroll
    for (int j = 0; j < kChunksPerLane; ++j) {
      const int ch = lane + kWave * j;
      if (ch < nchunks) *reinterpret_cast<uint4*>(win + 16 * ch) = c[j];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    return off;
  }
};

__device__ __forceinline__ void window_release() {
  // all lanes are done reading the window before it is overwritten
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// bytewise (a - 8) for nibbles a in [0, 15], no borrow between bytes
__device__ __forceinline__ int sub8(uint32_t a) {
  return (int)(((a | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
}

// four nibbles n (one per byte, 0..15) -> codebook bytes
__device__ __forceinline__ int lookup16(uint32_t n, uint32_t c0, uint32_t c1, uint32_t c2,
                                        uint32_t c3) {
  const uint32_t sel = n & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(c1, c0, sel);
  const uint32_t hi = __builtin_amdgcn_perm(c3, c2, sel);
  const uint32_t mask = ((n >> 3) & 0x01010101u) * 0xffu;
  return (int)((hi & mask) | (lo & ~mask));
}

// four +-1 sign bytes -> byte masks (0xff where -1), as the sign table is
// staged in LDS
__device__ __forceinline__ uint32_t sign_mask4(uint32_t s) { return ((s >> 7) & 0x01010101u) * 0xffu; }

// negate the bytes of g where the mask byte is 0xff: for a byte b != 0,
// (b ^ 0xff) + 1 never carries into the next byte (tables with a 0 grid
// byte or a sign other than +-1 take mul8x4, weft_common.h)
__device__ __forceinline__ int apply_signs(uint32_t g, uint32_t m) {
  return (int)((g ^ m) + (m & 0x01010101u));
}

template <Fmt F>
__global__ void __launch_bounds__(kThreads) staged_gemv_kernel(Args a) {
  using T = Traits<F>;
  static_assert(T::kSegRecords * T::kBytes + 16 <= kWindow, "a segment fits the window");
  if (a.pair.ids != nullptr && !resolve_pair(a)) return;
  extern __shared__ __align__(16) char lds[];
  char* windows = lds;                             // kWaves * kWindow
  char* tables = windows + kWaves * kWindow;       // lookup tables
  char* act = tables + table_bytes<F>();           // activation rows
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int nwaves = blockDim.x / kWave;
  const int K = a.K;

  // IQ2: the grid, then the sign rows as byte masks, then as given; `bad`
  // marks a table word outside the masks' precondition (weft_common.h)
  __shared__ uint32_t tflag[kWaves];
  bool bad = false;
  if constexpr (F == Fmt::IQ2_XXS || F == Fmt::IQ2_XS) {
    constexpr int kGridWords = F == Fmt::IQ2_XS ? 1024 : 512;
    for (int i = threadIdx.x; i < kGridWords; i += blockDim.x) {
      const uint32_t g = reinterpret_cast<const uint32_t*>(a.tab0)[i];
      reinterpret_cast<uint32_t*>(tables)[i] = g;
      bad |= !iq2_grid_word_ok(g);
    }
    for (int i = threadIdx.x; i < 256; i += blockDim.x) {
      const uint32_t sg = reinterpret_cast<const uint32_t*>(a.tab1)[i];
      reinterpret_cast<uint32_t*>(tables + 4 * kGridWords)[i] = sign_mask4(sg);
      reinterpret_cast<uint32_t*>(tables + 4 * kGridWords + 1024)[i] = sg;
      bad |= !iq2_sign_word_ok(sg);
    }
    iq2_flag_wave(tflag, bad);
  } else if constexpr (F == Fmt::MXFP4 || F == Fmt::NVFP4) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x)
      reinterpret_cast<float*>(tables)[i] = reinterpret_cast<const float*>(a.tab1)[i];
  }
  char* win = windows + wave * kWindow;
  const int nrec = K / T::kElems;
  const size_t rb = a.ldw;
  const uint8_t* wlo = a.W;
  // end of the last row: staging windows are clamped to [wlo, whi)
  const uint8_t* whi = a.W + (size_t)(a.N - 1) * rb + (size_t)nrec * T::kBytes;
  const int row0 = blockIdx.x * a.rows_per_wg;
  const int row1 = min(a.N, row0 + a.rows_per_wg);

  // this wave's (row, segment) sequence, one segment fetched ahead
  const int nseg = (nrec + T::kSegRecords - 1) / T::kSegRecords;
  const int my_rows = row0 + wave < row1 ? (row1 - row0 - wave + nwaves - 1) / nwaves : 0;
  const int total = my_rows * nseg;
  auto seg_span = [&](int si, const uint8_t*& p0, const uint8_t*& p1) {
    const int ri = si / nseg, r0 = (si - ri * nseg) * T::kSegRecords;
    const uint8_t* wr = a.W + (size_t)(row0 + wave + nwaves * ri) * rb;
    p0 = wr + (size_t)r0 * T::kBytes;
    p1 = wr + (size_t)min(r0 + T::kSegRecords, nrec) * T::kBytes;
  };
  // the first segment's loads are issued before the activation is staged,
  // so its HBM latency overlaps the quantization
  SegmentFetch pf;
  if (total > 0) {
    const uint8_t *p0, *p1;
    seg_span(0, p0, p1);
    pf.fetch(p0, p1, wlo, whi, lane);
  }
  if constexpr (T::kQ8K) {
    if (a.X != nullptr)
      stage_q8k_quantize(a.X, a.ldx, blockIdx.x == 0 ? a.xq_out : nullptr, K, a.m0, a.mb, act);
    else
      stage_q8k_load(a.xq_in, K, a.m0, a.mb, act);
  } else if constexpr (act_q81<F>()) {
    if (a.X != nullptr)
      stage_q81_quantize(a.X, a.ldx, blockIdx.x == 0 ? a.xq_out : nullptr, K, a.m0, a.mb, act);
    else
      stage_q81_load(a.xq_in, K, a.m0, a.mb, act);
  } else {
    if (a.X != nullptr)
      stage_q80_quantize(a.X, a.ldx, blockIdx.x == 0 ? a.xq_out : nullptr, K, a.m0, a.mb, act);
    else
      stage_q80_load(a.xq_in, K, a.m0, a.mb, act);
  }
  __syncthreads();
  // IQ2 tables within the masks' precondition (the same in every workgroup)
  bool canon = true;
  if constexpr (F == Fmt::IQ2_XXS || F == Fmt::IQ2_XS) canon = iq2_flags_clear(tflag, nwaves);

  uint32_t c0 = 0, c1 = 0, c2 = 0, c3 = 0;
  if constexpr (F == Fmt::MXFP4 || F == Fmt::NVFP4) {
    // int8[16] codebook, any alignment: four little-endian words
    const uint8_t* cb = reinterpret_cast<const uint8_t*>(a.tab0);
    c0 = ld_u32_a1(cb);
    c1 = ld_u32_a1(cb + 4);
    c2 = ld_u32_a1(cb + 8);
    c3 = ld_u32_a1(cb + 12);
  }

  float acc[kMaxRowsPerPass];
  for (int si = 0; si < total; ++si) {
    const int ri = si / nseg, seg = si - ri * nseg;
    const int row = row0 + wave + nwaves * ri;
    const int r0 = seg * T::kSegRecords;
    if (seg == 0) {
#pragma unroll
      for (int m = 0; m < kMaxRowsPerPass; ++m) acc[m] = 0.f;
    }
    {
      const int nr = min(T::kSegRecords, nrec - r0);
      const int off0 = pf.put(win, lane);
      if (si + 1 < total) {
        const uint8_t *p0, *p1;
        seg_span(si + 1, p0, p1);
        pf.fetch(p0, p1, wlo, whi, lane);
      }
      const int items = nr * T::kItemsPerRecord;
      // wave-uniform trip count: the IQ2_XXS branch reduces across lanes
      for (int it0 = 0; it0 < items; it0 += kWave) {
        const int it = it0 + lane;
        const bool valid = it < items;
        if constexpr (F == Fmt::Q4_0 || F == Fmt::MXFP4) {
          if (!valid) continue;
          const int b = it;             // block within segment
          const int gb = r0 + b;        // block within row
          const int o = off0 + T::kBytes * b;
          const int qo = o + (F == Fmt::Q4_0 ? 2 : 1);
          const uint32_t w0 = lds_u32(win, qo), w1 = lds_u32(win, qo + 4);
          const uint32_t w2 = lds_u32(win, qo + 8), w3 = lds_u32(win, qo + 12);
          int lo0, lo1, lo2, lo3, hi0, hi1, hi2, hi3;
          float wscale;
          if constexpr (F == Fmt::Q4_0) {
            wscale = fp16_to_fp32(lds_u32(win, o) & 0xffffu);
            lo0 = sub8(w0 & 0x0f0f0f0fu); lo1 = sub8(w1 & 0x0f0f0f0fu);
            lo2 = sub8(w2 & 0x0f0f0f0fu); lo3 = sub8(w3 & 0x0f0f0f0fu);
            hi0 = sub8((w0 >> 4) & 0x0f0f0f0fu); hi1 = sub8((w1 >> 4) & 0x0f0f0f0fu);
            hi2 = sub8((w2 >> 4) & 0x0f0f0f0fu); hi3 = sub8((w3 >> 4) & 0x0f0f0f0fu);
          } else {
            wscale = reinterpret_cast<const float*>(tables)[lds_u32(win, o) & 0xffu];
            lo0 = lookup16(w0, c0, c1, c2, c3); lo1 = lookup16(w1, c0, c1, c2, c3);
            lo2 = lookup16(w2, c0, c1, c2, c3); lo3 = lookup16(w3, c0, c1, c2, c3);
            hi0 = lookup16(w0 >> 4, c0, c1, c2, c3); hi1 = lookup16(w1 >> 4, c0, c1, c2, c3);
            hi2 = lookup16(w2 >> 4, c0, c1, c2, c3); hi3 = lookup16(w3 >> 4, c0, c1, c2, c3);
          }
#pragma unroll
          for (int m = 0; m < kMaxRowsPerPass; ++m) {
            if (m >= a.mb) break;
            const Q80View v = q80_view(act, K, m);
            const int4 xl = *reinterpret_cast<const int4*>(v.qs + 32 * gb);
            const int4 xh = *reinterpret_cast<const int4*>(v.qs + 32 * gb + 16);
            int s = dot4(lo0, xl.x, 0);
            s = dot4(lo1, xl.y, s);
            s = dot4(lo2, xl.z, s);
            s = dot4(lo3, xl.w, s);
            s = dot4(hi0, xh.x, s);
            s = dot4(hi1, xh.y, s);
            s = dot4(hi2, xh.z, s);
            s = dot4(hi3, xh.w, s);
            if constexpr (F == Fmt::MXFP4)
              acc[m] = ggml_scaled_term(acc[m], v.d[gb], wscale, (float)s);  // GGML's order
            else
              acc[m] += (float)s * wscale * v.d[gb];
          }
        } else if constexpr (F == Fmt::Q4_1) {
          if (!valid) continue;
          // one 32-element block per lane: unsigned nibbles against Q8_1,
          // GGML's (dw dx) sumi + m s per block (ggml-cpu/quants.c:211-245)
          const int gb = r0 + it;
          const int o = off0 + T::kBytes * it;
          const uint32_t hd = lds_u32(win, o);
          const float dw = fp16_to_fp32(hd & 0xffffu), mw = fp16_to_fp32(hd >> 16);
          uint32_t q[4];
          lds_run(win, o + 4, q);
          const int lo0 = (int)(q[0] & 0x0f0f0f0fu), lo1 = (int)(q[1] & 0x0f0f0f0fu);
          const int lo2 = (int)(q[2] & 0x0f0f0f0fu), lo3 = (int)(q[3] & 0x0f0f0f0fu);
          const int hi0 = (int)((q[0] >> 4) & 0x0f0f0f0fu), hi1 = (int)((q[1] >> 4) & 0x0f0f0f0fu);
          const int hi2 = (int)((q[2] >> 4) & 0x0f0f0f0fu), hi3 = (int)((q[3] >> 4) & 0x0f0f0f0fu);
#pragma unroll
          for (int m = 0; m < kMaxRowsPerPass; ++m) {
            if (m >= a.mb) break;
            const Q81View v = q81_view(act, K, m);
            const int4 xl = *reinterpret_cast<const int4*>(v.qs + 32 * gb);
            const int4 xh = *reinterpret_cast<const int4*>(v.qs + 32 * gb + 16);
            int p = dot4(lo0, xl.x, 0);
            p = dot4(lo1, xl.y, p);
            p = dot4(lo2, xl.z, p);
            p = dot4(lo3, xl.w, p);
            p = dot4(hi0, xh.x, p);
            p = dot4(hi1, xh.y, p);
            p = dot4(hi2, xh.z, p);
            p = dot4(hi3, xh.w, p);
            acc[m] += (dw * v.d[gb]) * (float)p + mw * v.s[gb];
          }
        } else if constexpr (F == Fmt::IQ2_XS) {
          // item = (superblock, 32-group g); 8 lanes per superblock.  Entry
          // l's u16 word: grid row bits 0-8, sign row bits 9-15; entries 0-1
          // take scale nibble low, 2-3 high (ggml-cpu/quants.c:897-946)
          const int sb = valid ? it >> 3 : 0, g = it & 7;
          const int gsb = r0 + sb;
          const int o = off0 + T::kBytes * sb;
          const float dw = fp16_to_fp32(lds_u32(win, o) & 0xffffu);
          uint32_t q[2];
          lds_run(win, o + 2 + 8 * g, q);
          const uint32_t sc = lds_u32(win, o + 66 + g) & 0xffu;
          const uint2* grid = reinterpret_cast<const uint2*>(tables);
          const uint2* sgn = reinterpret_cast<const uint2*>(tables + (canon ? 4096 : 5120));
          int wv[8];
#pragma unroll
          for (int l = 0; l < 4; ++l) {
            const uint32_t word = (q[l >> 1] >> (16 * (l & 1))) & 0xffffu;
            const uint2 gv = grid[word & 511u];
            const uint2 sv = sgn[word >> 9];
            wv[2 * l] = canon ? apply_signs(gv.x, sv.x) : (int)mul8x4(gv.x, sv.x);
            wv[2 * l + 1] = canon ? apply_signs(gv.y, sv.y) : (int)mul8x4(gv.y, sv.y);
          }
          const int ls1 = 2 * (int)(sc & 15u) + 1, ls2 = 2 * (int)(sc >> 4) + 1;
#pragma unroll
          for (int m = 0; m < kMaxRowsPerPass; ++m) {
            if (m >= a.mb) break;
            const Q8KView v = q8k_view(act, K, m);
            const int4 x0 = *reinterpret_cast<const int4*>(v.qs + 256 * gsb + 32 * g);
            const int4 x1 = *reinterpret_cast<const int4*>(v.qs + 256 * gsb + 32 * g + 16);
            int s0 = dot4(wv[0], x0.x, 0);
            s0 = dot4(wv[1], x0.y, s0);
            s0 = dot4(wv[2], x0.z, s0);
            s0 = dot4(wv[3], x0.w, s0);
            int s1 = dot4(wv[4], x1.x, 0);
            s1 = dot4(wv[5], x1.y, s1);
            s1 = dot4(wv[6], x1.z, s1);
            s1 = dot4(wv[7], x1.w, s1);
            // the superblock's integer sum over its 8 groups, then one fp32 term
            const int bsum = sum8_of_sum4(sum4(valid ? s0 * ls1 + s1 * ls2 : 0));
            if (valid && g == 0) acc[m] += (dw * v.d[gsb]) * (float)bsum;
          }
        } else if constexpr (F == Fmt::NVFP4) {
          if (!valid) continue;
          // item = one 64-element record: sub-block s (16 elements) is the low
          // then high nibbles of qs words 2 s, 2 s + 1 and meets half s % 2 of
          // Q8_0 block 2 gb + s / 2
          const int gb = r0 + it;
          const int o = off0 + T::kBytes * it;
          // one sub-block at a time: its two words decoded, then every row
          // (decoding all eight words up front spilled at 128 VGPRs)
          const uint32_t sw = lds_u32(win, o);
          const float* tab = reinterpret_cast<const float*>(tables);
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            uint32_t q[2];
            lds_run(win, o + 4 + 8 * s, q);
            const int lo0 = lookup16(q[0], c0, c1, c2, c3), lo1 = lookup16(q[1], c0, c1, c2, c3);
            const int hi0 = lookup16(q[0] >> 4, c0, c1, c2, c3), hi1 = lookup16(q[1] >> 4, c0, c1, c2, c3);
            const float ws = tab[(sw >> (8 * s)) & 0xffu];
            const int xb = 2 * gb + s / 2;
#pragma unroll
            for (int m = 0; m < kMaxRowsPerPass; ++m) {
              if (m >= a.mb) break;
              const Q80View v = q80_view(act, K, m);
              const int4 x = *reinterpret_cast<const int4*>(v.qs + 32 * xb + 16 * (s % 2));
              int p = dot4(lo0, x.x, 0);
              p = dot4(lo1, x.y, p);
              p = dot4(hi0, x.z, p);
              p = dot4(hi1, x.w, p);
              acc[m] += v.d[xb] * ws * (float)p;
            }
          }
        } else if constexpr (F == Fmt::Q5_K) {
          // item = (superblock, 64-element group g): qs bytes 48 + 32 g + l
          // hold sub-block 2 g in their low and 2 g + 1 in their high
          // nibbles, bits 2 g and 2 g + 1 of qh bytes 16 + l the fifth bits;
          // one header decode and one 4-lane reduction per two sub-blocks
          const int sb = valid ? it >> 2 : 0, g = it & 3;
          const int gsb = r0 + sb;
          const int o = off0 + T::kBytes * sb;
          uint32_t hd[4], qs[8], qh[8];
          lds_run(win, o, hd);
          lds_run(win, o + 48 + 32 * g, qs);
          lds_run(win, o + 16, qh);
          int sc0, mn0, sc1, mn1;
          q4k_scale_min(2 * g, hd[1], hd[2], hd[3], sc0, mn0);
          q4k_scale_min(2 * g + 1, hd[1], hd[2], hd[3], sc1, mn1);
          const float dw = fp16_to_fp32(hd[0] & 0xffffu), dmin = fp16_to_fp32(hd[0] >> 16);
          // bit 2 g (2 g + 1) of each byte to bit 4
          const uint32_t rot0 = (uint32_t)(2 * g + 28) & 31u, rot1 = (uint32_t)(2 * g + 29) & 31u;
          int wl[8], wh[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            wl[j] = (int)((qs[j] & 0x0f0f0f0fu) | (__builtin_amdgcn_alignbit(qh[j], qh[j], rot0) & 0x10101010u));
            wh[j] = (int)(((qs[j] >> 4) & 0x0f0f0f0fu) |
                          (__builtin_amdgcn_alignbit(qh[j], qh[j], rot1) & 0x10101010u));
          }
#pragma unroll
          for (int m = 0; m < kMaxRowsPerPass; ++m) {
            if (m >= a.mb) break;
            const Q8KView v = q8k_view(act, K, m);
            const int4* xv = reinterpret_cast<const int4*>(v.qs + 256 * gsb + 64 * g);
            const int4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
            int p0 = dot4(wl[0], x0.x, 0);
            p0 = dot4(wl[1], x0.y, p0);
            p0 = dot4(wl[2], x0.z, p0);
            p0 = dot4(wl[3], x0.w, p0);
            p0 = dot4(wl[4], x1.x, p0);
            p0 = dot4(wl[5], x1.y, p0);
            p0 = dot4(wl[6], x1.z, p0);
            p0 = dot4(wl[7], x1.w, p0);
            int p1 = dot4(wh[0], x2.x, 0);
            p1 = dot4(wh[1], x2.y, p1);
            p1 = dot4(wh[2], x2.z, p1);
            p1 = dot4(wh[3], x2.w, p1);
            p1 = dot4(wh[4], x3.x, p1);
            p1 = dot4(wh[5], x3.y, p1);
            p1 = dot4(wh[6], x3.z, p1);
            p1 = dot4(wh[7], x3.w, p1);
            const int2 bp = *reinterpret_cast<const int2*>(v.bp + 8 * gsb + 2 * g);
            // exact int32 S and Mn of the superblock over its 4 groups
            // (|S| <= 256 * 31 * 127 * 63), then one fp32 term
            const int S = sum4(valid ? sc0 * p0 + sc1 * p1 : 0);
            const int Mn = sum4(valid ? mn0 * bp.x + mn1 * bp.y : 0);
            if (valid && g == 0) acc[m] += v.d[gsb] * (dw * (float)S - dmin * (float)Mn);
          }
        } else if constexpr (F == Fmt::Q6_K) {
          // item = (superblock, 64 elements): chunks g0 = 4 h + c and
          // g1 = g0 + 2 of half h (c = 0, 1) share ql bytes 64 h + 32 c + l
          // (low / high nibble) and qh bytes 128 + 32 h + l (bits 2 c /
          // 2 c + 4); chunk g's two 16-groups scale by sc[2 g], sc[2 g + 1]
          const int sb = valid ? it >> 2 : 0, G = it & 3;
          const int gsb = r0 + sb;
          const int o = off0 + T::kBytes * sb;
          const int h = G >> 1, c = G & 1;
          const int g0 = 4 * h + c, g1 = g0 + 2;
          uint32_t lq[8], hq[8];
          lds_run(win, o + 64 * h + 32 * c, lq);
          lds_run(win, o + 128 + 32 * h, hq);
          const uint32_t sw0 = lds_u32(win, o + 192 + 2 * g0), sw1 = lds_u32(win, o + 192 + 2 * g1);
          const int sc00 = (int)(int8_t)(sw0 & 0xffu), sc01 = (int)(int8_t)((sw0 >> 8) & 0xffu);
          const int sc10 = (int)(int8_t)(sw1 & 0xffu), sc11 = (int)(int8_t)((sw1 >> 8) & 0xffu);
          const float dw = fp16_to_fp32(lds_u32(win, o + 208) & 0xffffu);
          const int hs0 = 2 * c, hs1 = 2 * c + 4;
          int w0[8], w1[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const uint32_t q0 = (lq[j] & 0x0f0f0f0fu) | (((hq[j] >> hs0) & 0x03030303u) << 4);
            const uint32_t q1 = ((lq[j] >> 4) & 0x0f0f0f0fu) | (((hq[j] >> hs1) & 0x03030303u) << 4);
            w0[j] = (int)(((q0 | 0x80808080u) - 0x20202020u) ^ 0x80808080u);  // bytewise q - 32
            w1[j] = (int)(((q1 | 0x80808080u) - 0x20202020u) ^ 0x80808080u);
          }
#pragma unroll
          for (int m = 0; m < kMaxRowsPerPass; ++m) {
            if (m >= a.mb) break;
            const Q8KView v = q8k_view(act, K, m);
            const int4* xa = reinterpret_cast<const int4*>(v.qs + 256 * gsb + 32 * g0);
            const int4* xb = reinterpret_cast<const int4*>(v.qs + 256 * gsb + 32 * g1);
            const int4 x0 = xa[0], x1 = xa[1], y0 = xb[0], y1 = xb[1];
            int s00 = dot4(w0[0], x0.x, 0);
            s00 = dot4(w0[1], x0.y, s00);
            s00 = dot4(w0[2], x0.z, s00);
            s00 = dot4(w0[3], x0.w, s00);
            int s01 = dot4(w0[4], x1.x, 0);
            s01 = dot4(w0[5], x1.y, s01);
            s01 = dot4(w0[6], x1.z, s01);
            s01 = dot4(w0[7], x1.w, s01);
            int s10 = dot4(w1[0], y0.x, 0);
            s10 = dot4(w1[1], y0.y, s10);
            s10 = dot4(w1[2], y0.z, s10);
            s10 = dot4(w1[3], y0.w, s10);
            int s11 = dot4(w1[4], y1.x, 0);
            s11 = dot4(w1[5], y1.y, s11);
            s11 = dot4(w1[6], y1.z, s11);
            s11 = dot4(w1[7], y1.w, s11);
            // the superblock's exact int32 sum over its 4 items, then one
            // fp32 term (|sum| <= 256 * 32 * 127 * 128 < 2^31)
            const int bsum = sum4(valid ? sc00 * s00 + sc01 * s01 + sc10 * s10 + sc11 * s11 : 0);
            if (valid && G == 0) acc[m] += (dw * v.d[gsb]) * (float)bsum;
          }
        } else {  // IQ2_XXS: item = (superblock, 32-group); 8 lanes per superblock
          const int sb = valid ? it >> 3 : 0, g = it & 7;
          const int gsb = r0 + sb;
          const int o = off0 + T::kBytes * sb;
          const float dw = fp16_to_fp32(lds_u32(win, o) & 0xffffu);
          const uint32_t idx = lds_u32(win, o + 2 + 8 * g);
          const uint32_t meta = lds_u32(win, o + 6 + 8 * g);
          const uint2* grid = reinterpret_cast<const uint2*>(tables);
          const uint2* sgn = reinterpret_cast<const uint2*>(tables + (canon ? 2048 : 3072));
          int wv[8];
#pragma unroll
          for (int l = 0; l < 4; ++l) {
            const uint2 gv = grid[(idx >> (8 * l)) & 0xffu];
            const uint2 sv = sgn[(meta >> (7 * l)) & 127u];
            wv[2 * l] = canon ? apply_signs(gv.x, sv.x) : (int)mul8x4(gv.x, sv.x);
            wv[2 * l + 1] = canon ? apply_signs(gv.y, sv.y) : (int)mul8x4(gv.y, sv.y);
          }
          const int ls = 2 * (int)(meta >> 28) + 1;
#pragma unroll
          for (int m = 0; m < kMaxRowsPerPass; ++m) {
            if (m >= a.mb) break;
            const Q8KView v = q8k_view(act, K, m);
            const int4 x0 = *reinterpret_cast<const int4*>(v.qs + 256 * gsb + 32 * g);
            const int4 x1 = *reinterpret_cast<const int4*>(v.qs + 256 * gsb + 32 * g + 16);
            int s = dot4(wv[0], x0.x, 0);
            s = dot4(wv[1], x0.y, s);
            s = dot4(wv[2], x0.z, s);
            s = dot4(wv[3], x0.w, s);
            s = dot4(wv[4], x1.x, s);
            s = dot4(wv[5], x1.y, s);
            s = dot4(wv[6], x1.z, s);
            s = dot4(wv[7], x1.w, s);
            // the superblock's integer sum over its 8 groups (8 aligned lanes),
            // then one fp32 term, as ggml_vec_dot_iq2_xxs_q8_K_generic
            const int bsum = sum8_of_sum4(sum4(valid ? s * ls : 0));
            if (valid && g == 0) acc[m] += (dw * v.d[gsb]) * (float)bsum;
          }
        }
      }
      window_release();
    }
    if (seg == nseg - 1) {
#pragma unroll
      for (int m = 0; m < kMaxRowsPerPass; ++m) {
        if (m >= a.mb) break;
        float tot = wave_sum_f(acc[m]);
        if constexpr (F == Fmt::IQ2_XXS || F == Fmt::IQ2_XS) tot *= 0.125f;
        if (lane == 0) {
          float* yp = a.Y + (size_t)(a.m0 + m) * a.y_stride + row;
          *yp = a.accumulate ? *yp + tot : tot;
        }
      }
    }
  }
}

// A row whose quantized activation does not fit the LDS beside the windows:
// one launch per activation row and K chunk (a multiple of 1024 values that
// fits), each staging and quantizing its chunk of the row (block 0 writes
// that chunk's Xq records, which fall on whole Q8 blocks) and adding its
// partial dot products to Y, which the first chunk stores.  Launches are
// ordered on the stream.
template <Fmt F>
void launch_chunked(const uint8_t* W, const float* X, const uint8_t* xq_in, uint8_t* xq_out,
                    const int8_t* tab0, const void* tab1, float* Y, size_t N, size_t K, size_t M,
                    const RowStrides& st) {
  using T = Traits<F>;
  auto row_lds = [](size_t k) {
    return T::kQ8K ? q8k_lds_row_bytes((int)k) : act_q81<F>() ? q81_lds_row_bytes((int)k) : q80_lds_row_bytes((int)k);
  };
  const size_t fixed = (size_t)kWaves * kWindow + table_bytes<F>();
  const size_t cap = max_lds_per_block();
  size_t kc = 0;
  while (fixed + row_lds(kc + 1024) <= cap) kc += 1024;
  if (kc == 0) {
    set_error(hipErrorInvalidValue);
    return;
  }
  const size_t act_elems = T::kQ8K ? 256 : 32;
  const size_t act_rec = T::kQ8K ? kQ8_KBytes : act_q81<F>() ? kQ8_1Bytes : kQ8_0Bytes;
  const size_t xrow = K / act_elems * act_rec;  // bytes of one quantized activation row
  const int cus = cu_count();
  const TileBindings& tb = tile_bindings();
  const int rows_per_wg = tb.nc > 0 ? (int)std::min<size_t>(N, (size_t)tb.nc) : (int)((N + cus - 1) / cus);
  const int grid = (int)((N + rows_per_wg - 1) / rows_per_wg);
  for (size_t m = 0; m < M; ++m) {
    for (size_t k0 = 0; k0 < K; k0 += kc) {
      const size_t k = std::min(kc, K - k0);
      const size_t xo = m * xrow + k0 / act_elems * act_rec;
      Args a;
      a.W = W + k0 / T::kElems * T::kBytes;
      a.X = X != nullptr ? X + m * st.ldx + k0 : nullptr;
      a.xq_in = xq_in != nullptr ? xq_in + xo : nullptr;
      a.xq_out = xq_out != nullptr ? xq_out + xo : nullptr;
      a.tab0 = tab0;
      a.tab1 = tab1;
      a.Y = Y + m * st.ldy;
      a.N = (int)N;
      a.K = (int)k;
      a.m0 = 0;
      a.mb = 1;
      a.rows_per_wg = rows_per_wg;
      a.y_stride = (long long)st.ldy;
      a.ldw = st.ldw;
      a.ldx = st.ldx;
      a.pair = PairArgs{};
      a.accumulate = k0 > 0;
      staged_gemv_kernel<F><<<grid, kThreads, fixed + row_lds(k), current_stream()>>>(a);
      check_launch("staged_gemv_kernel");
    }
  }
}

template <Fmt F>
void launch(const uint8_t* W, const float* X, const uint8_t* xq_in, uint8_t* xq_out,
            const int8_t* tab0, const void* tab1, float* Y, size_t N, size_t K, size_t M,
            const RowStrides& st, const PairArgs* pr = nullptr, int n_pairs = 0) {
  using T = Traits<F>;
  if (pr != nullptr) M = 1;  // one activation row per pair
  if (N == 0 || M == 0 || K == 0 || (pr != nullptr && n_pairs <= 0)) return;
  const size_t act_align = T::kQ8K ? 4 : 2;
  const size_t w_align = F == Fmt::MXFP4 || F == Fmt::Q6_K || F == Fmt::NVFP4 ? 1 : 2;
  constexpr bool kGrid = F == Fmt::IQ2_XXS || F == Fmt::IQ2_XS;
  if (K % T::kElems != 0 || W == nullptr || Y == nullptr || (X == nullptr && xq_in == nullptr) ||
      N > (size_t)INT32_MAX || K > (size_t)INT32_MAX || M > (size_t)INT32_MAX ||
      !aligned(W, w_align) || !aligned(Y, 4) || (X && !aligned(X, 4)) ||
      (xq_in && !aligned(xq_in, act_align)) || (xq_out && !aligned(xq_out, act_align)) ||
      ((F == Fmt::MXFP4 || F == Fmt::NVFP4 || kGrid) && (tab0 == nullptr || tab1 == nullptr)) ||
      (kGrid && (!aligned(tab0, 4) || !aligned(tab1, 4))) ||
      ((F == Fmt::MXFP4 || F == Fmt::NVFP4) && !aligned(tab1, 4)) ||
      !strides_ok(st, K / T::kElems * T::kBytes, w_align, K, N, N, M) ||
      (pr != nullptr && pr->w_es % (long long)w_align != 0)) {
    set_error(hipErrorInvalidValue);
    return;
  }
  if constexpr (F == Fmt::Q4_0 || F == Fmt::MXFP4 || F == Fmt::NVFP4 || F == Fmt::Q4_1) {
    // batch 1: the register-resident kernel of decode_rec.hip when it applies
    constexpr int kRecFmt = F == Fmt::MXFP4 ? 1 : F == Fmt::NVFP4 ? 5 : F == Fmt::Q4_1 ? 6 : 0;
    if (pr == nullptr && M == 1 && X != nullptr &&
        decode_rec_m1(kRecFmt, W, X, xq_out, tab0, static_cast<const float*>(tab1), Y, N, K, st))
      return;
  }
  if constexpr (F == Fmt::Q5_K) {
    // batch 1: the register-resident kernel of decode_q5k.hip when it applies
    if (pr == nullptr && M == 1 && X != nullptr && decode_q5k_m1(W, X, xq_out, Y, N, K, st)) return;
  }
  if constexpr (F == Fmt::Q6_K) {
    // batch 1: the register-resident kernel of decode_q6k.hip when it applies
    if (pr == nullptr && M == 1 && X != nullptr && decode_q6k_m1(W, X, xq_out, Y, N, K, st)) return;
  }
  if constexpr (kGrid) {
    // batch 1: the register-resident kernel of decode_iq2.hip when it applies
    if (pr == nullptr && M == 1 && X != nullptr &&
        decode_iq2_m1(F == Fmt::IQ2_XS, W, X, xq_out, tab0, static_cast<const int8_t*>(tab1), Y, N, K, st))
      return;
  }
  const size_t row_lds = T::kQ8K ? q8k_lds_row_bytes((int)K)
                         : act_q81<F>() ? q81_lds_row_bytes((int)K)
                                        : q80_lds_row_bytes((int)K);
  const size_t fixed = (size_t)kWaves * kWindow + table_bytes<F>();
  const size_t cap = max_lds_per_block();
  if (fixed + row_lds > cap) {
    if (pr == nullptr) return launch_chunked<F>(W, X, xq_in, xq_out, tab0, tab1, Y, N, K, M, st);
    set_error(hipErrorInvalidValue);
    return;
  }
  const TileBindings& tb = tile_bindings();
  int mb_max = (int)std::min<size_t>(kMaxRowsPerPass, (cap - fixed) / row_lds);
  if (tb.mr > 0) mb_max = std::min(mb_max, tb.mr);
  const int cus = cu_count();
  const int rows_per_wg = tb.nc > 0 ? (int)std::min<size_t>(N, (size_t)tb.nc) : (int)((N + cus - 1) / cus);
  const int grid = (int)((N + rows_per_wg - 1) / rows_per_wg);
  for (size_t m0 = 0; m0 < M; m0 += mb_max) {
    Args a;
    a.W = W;
    a.X = X;
    a.xq_in = xq_in;
    a.xq_out = xq_out;
    a.tab0 = tab0;
    a.tab1 = tab1;
    a.Y = Y;
    a.N = (int)N;
    a.K = (int)K;
    a.m0 = (int)m0;
    a.mb = (int)std::min<size_t>(mb_max, M - m0);
    a.rows_per_wg = rows_per_wg;
    a.y_stride = (long long)st.ldy;
    a.ldw = st.ldw;
    a.ldx = st.ldx;
    a.pair = PairArgs{};
    a.accumulate = 0;
    if (pr == nullptr) {
      staged_gemv_kernel<F><<<grid, kThreads, fixed + row_lds * a.mb, current_stream()>>>(a);
      check_launch("staged_gemv_kernel");
      continue;
    }
    for (int p0 = 0; p0 < n_pairs; p0 += kMaxGridY) {
      a.pair = *pr;
      a.pair.pair0 = p0;
      const dim3 g((unsigned)grid, (unsigned)std::min(kMaxGridY, n_pairs - p0));
      staged_gemv_kernel<F><<<g, kThreads, fixed + row_lds, current_stream()>>>(a);
      check_launch("staged_gemv_kernel");
    }
  }
}

}  // namespace

// Decode entry points shared with the prefill file for small M.  A row the
// GEMV's LDS cannot hold goes to the format's GEMM when it takes the call.
void decode_q4_0(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M, const RowStrides& st) {
  if (!staged_gemv_fits(0, K) && gemm_q80_try(0, W, X, Xq, nullptr, nullptr, Y, N, K, M, st)) return;
  launch<Fmt::Q4_0>(W, X, nullptr, Xq, nullptr, nullptr, Y, N, K, M, st);
}
void decode_mxfp4(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                  const float* scale, float* Y, size_t N, size_t K, size_t M, const RowStrides& st) {
  if (!staged_gemv_fits(1, K) && gemm_q80_try(1, W, X, Xq, codebook, scale, Y, N, K, M, st)) return;
  launch<Fmt::MXFP4>(W, X, nullptr, Xq, codebook, scale, Y, N, K, M, st);
}
void decode_iq2_xxs(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid,
                    const int8_t* signs, float* Y, size_t N, size_t K, size_t M,
                    const RowStrides& st) {
  if (!staged_gemv_fits(2, K) && gemm_iq2_try(false, W, X, Xq, grid, signs, Y, N, K, M, st)) return;
  launch<Fmt::IQ2_XXS>(W, X, nullptr, Xq, grid, signs, Y, N, K, M, st);
}

void decode_pairs(int fmt, const uint8_t* W, const float* X, const uint8_t* xq_in, uint8_t* xq_out,
                  const int8_t* tab0, const void* tab1, float* Y, size_t N, size_t K,
                  const RowStrides& st, const PairArgs& pr, int n_pairs) {
  switch (fmt) {
    case 0: return launch<Fmt::Q4_0>(W, X, xq_in, xq_out, nullptr, nullptr, Y, N, K, 1, st, &pr, n_pairs);
    case 1: return launch<Fmt::MXFP4>(W, X, xq_in, xq_out, tab0, tab1, Y, N, K, 1, st, &pr, n_pairs);
    case 3: return launch<Fmt::Q6_K>(W, X, xq_in, xq_out, nullptr, nullptr, Y, N, K, 1, st, &pr, n_pairs);
    case 4: return launch<Fmt::Q5_K>(W, X, xq_in, xq_out, nullptr, nullptr, Y, N, K, 1, st, &pr, n_pairs);
    case 5: return launch<Fmt::NVFP4>(W, X, xq_in, xq_out, tab0, tab1, Y, N, K, 1, st, &pr, n_pairs);
    case 6: return launch<Fmt::Q4_1>(W, X, xq_in, xq_out, nullptr, nullptr, Y, N, K, 1, st, &pr, n_pairs);
    case 7: return launch<Fmt::IQ2_XS>(W, X, xq_in, xq_out, tab0, tab1, Y, N, K, 1, st, &pr, n_pairs);
    default: return launch<Fmt::IQ2_XXS>(W, X, xq_in, xq_out, tab0, tab1, Y, N, K, 1, st, &pr, n_pairs);
  }
}

void decode_q4_1(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M, const RowStrides& st) {
  if (!staged_gemv_fits(6, K) && gemm_q80_try(6, W, X, Xq, nullptr, nullptr, Y, N, K, M, st)) return;
  launch<Fmt::Q4_1>(W, X, nullptr, Xq, nullptr, nullptr, Y, N, K, M, st);
}

void decode_iq2_xs(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid,
                   const int8_t* signs, float* Y, size_t N, size_t K, size_t M, const RowStrides& st) {
  if (!staged_gemv_fits(7, K) && gemm_iq2_try(true, W, X, Xq, grid, signs, Y, N, K, M, st)) return;
  launch<Fmt::IQ2_XS>(W, X, nullptr, Xq, grid, signs, Y, N, K, M, st);
}

void decode_q6_k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M, const RowStrides& st) {
  if (!staged_gemv_fits(3, K) && gemm_kq_try(true, W, X, Xq, Y, N, K, M, st)) return;
  launch<Fmt::Q6_K>(W, X, nullptr, Xq, nullptr, nullptr, Y, N, K, M, st);
}

void decode_q5_k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                 size_t M, const RowStrides& st) {
  if (!staged_gemv_fits(4, K) && gemm_kq_try(false, W, X, Xq, Y, N, K, M, st)) return;
  launch<Fmt::Q5_K>(W, X, nullptr, Xq, nullptr, nullptr, Y, N, K, M, st);
}

void decode_nvfp4(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                  const float* scale, float* Y, size_t N, size_t K, size_t M, const RowStrides& st) {
  if (!staged_gemv_fits(5, K) && gemm_q80_try(5, W, X, Xq, codebook, scale, Y, N, K, M, st)) return;
  launch<Fmt::NVFP4>(W, X, nullptr, Xq, codebook, scale, Y, N, K, M, st);
}

namespace {
template <Fmt F>
bool staged_fits(size_t K) {
  using T = Traits<F>;
  if (K == 0 || K > (size_t)INT32_MAX) return true;  // refused elsewhere, not for its LDS
  const size_t row_lds = T::kQ8K ? q8k_lds_row_bytes((int)K)
                         : act_q81<F>() ? q81_lds_row_bytes((int)K)
                                        : q80_lds_row_bytes((int)K);
  return (size_t)kWaves * kWindow + table_bytes<F>() + row_lds <= max_lds_per_block();
}
}  // namespace

// Whether the staged GEMV's LDS holds one activation row of K values (the
// same test as launch<F>'s): a longer row goes to the prefill GEMM.
bool staged_gemv_fits(int fmt, size_t K) {
  switch (fmt) {
    case 0: return staged_fits<Fmt::Q4_0>(K);
    case 1: return staged_fits<Fmt::MXFP4>(K);
    case 3: return staged_fits<Fmt::Q6_K>(K);
    case 4: return staged_fits<Fmt::Q5_K>(K);
    case 5: return staged_fits<Fmt::NVFP4>(K);
    case 6: return staged_fits<Fmt::Q4_1>(K);
    case 7: return staged_fits<Fmt::IQ2_XS>(K);
    default: return staged_fits<Fmt::IQ2_XXS>(K);
  }
}

void decode_quantized(int fmt, const uint8_t* W, const uint8_t* Xq, const int8_t* tab0,
                      const void* tab1, float* Y, size_t N, size_t K, size_t M,
                      const RowStrides& st) {
  switch (fmt) {
    case 0: return launch<Fmt::Q4_0>(W, nullptr, Xq, nullptr, nullptr, nullptr, Y, N, K, M, st);
    case 1: return launch<Fmt::MXFP4>(W, nullptr, Xq, nullptr, tab0, tab1, Y, N, K, M, st);
    case 3: return launch<Fmt::Q6_K>(W, nullptr, Xq, nullptr, nullptr, nullptr, Y, N, K, M, st);
    case 4: return launch<Fmt::Q5_K>(W, nullptr, Xq, nullptr, nullptr, nullptr, Y, N, K, M, st);
    case 5: return launch<Fmt::NVFP4>(W, nullptr, Xq, nullptr, tab0, tab1, Y, N, K, M, st);
    case 6: return launch<Fmt::Q4_1>(W, nullptr, Xq, nullptr, nullptr, nullptr, Y, N, K, M, st);
    case 7: return launch<Fmt::IQ2_XS>(W, nullptr, Xq, nullptr, tab0, tab1, Y, N, K, M, st);
    default: return launch<Fmt::IQ2_XXS>(W, nullptr, Xq, nullptr, tab0, tab1, Y, N, K, M, st);
  }
}

}  // namespace weft

extern "C" {

void production_mul_mat_q4_0_decode(const uint8_t* W, const float* X, uint8_t* Xq, float* Y,
                                    size_t N, size_t K, size_t M) {
  if (X == nullptr || Xq == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::decode_q4_0(W, X, Xq, Y, N, K, M, weft::packed(K / 32 * weft::kQ4_0Bytes, K, N));
}

void production_mul_mat_mxfp4_decode(const uint8_t* W, const float* X, uint8_t* Xq,
                                     const int8_t* codebook, const float* scale, float* Y,
                                     size_t N, size_t K, size_t M) {
  if (X == nullptr || Xq == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::decode_mxfp4(W, X, Xq, codebook, scale, Y, N, K, M, weft::packed(K / 32 * weft::kMxfp4Bytes, K, N));
}

void production_mul_mat_iq2_xxs_decode(const uint8_t* W, const float* X, uint8_t* Xq,
                                       const int8_t* grid, const int8_t* signs, float* Y, size_t N,
                                       size_t K, size_t M) {
  if (X == nullptr || Xq == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::decode_iq2_xxs(W, X, Xq, grid, signs, Y, N, K, M,
                       weft::packed(K / 256 * weft::kIq2xxsBytes, K, N));
}

void quantized_vec_dot_q4_0_q8_0(const uint8_t* W, const uint8_t* X, float* Y, size_t K) {
  if (X == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::launch<weft::Fmt::Q4_0>(W, nullptr, X, nullptr, nullptr, nullptr, Y, 1, K, 1, weft::packed(0, K, 1));
}

void quantized_vec_dot_mxfp4_q8_0(const uint8_t* W, const uint8_t* X, const int8_t* codebook,
                                  const float* scale, float* Y, size_t K) {
  if (X == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::launch<weft::Fmt::MXFP4>(W, nullptr, X, nullptr, codebook, scale, Y, 1, K, 1, weft::packed(0, K, 1));
}

void production_mul_mat_q6_k_decode(const uint8_t* W, const float* X, uint8_t* Xq, float* Y,
                                    size_t N, size_t K, size_t M) {
  if (X == nullptr || Xq == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::decode_q6_k(W, X, Xq, Y, N, K, M, weft::packed(K / 256 * weft::kQ6_KBytes, K, N));
}

// Q6_K mul_mat: the int8-MFMA GEMM for prefill shapes, the GEMV otherwise
void production_mul_mat_q6_k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N,
                             size_t K, size_t M) {
  if (X == nullptr || Xq == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::mul_mat_q6k(W, X, Xq, Y, N, K, M, weft::packed(K / 256 * weft::kQ6_KBytes, K, N));
}

void production_mul_mat_nvfp4_decode(const uint8_t* W, const float* X, uint8_t* Xq,
                                     const int8_t* codebook, const float* scale, float* Y, size_t N,
                                     size_t K, size_t M) {
  if (X == nullptr || Xq == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::decode_nvfp4(W, X, Xq, codebook, scale, Y, N, K, M,
                     weft::packed(K / 64 * weft::kNvfp4Bytes, K, N));
}

// NVFP4 mul_mat: the int8-MFMA GEMM for prefill shapes, the GEMV otherwise
void production_mul_mat_nvfp4(const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                              const float* scale, float* Y, size_t N, size_t K, size_t M) {
  if (X == nullptr || Xq == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::mul_mat_nvfp4(W, X, Xq, codebook, scale, Y, N, K, M, weft::packed(K / 64 * weft::kNvfp4Bytes, K, N));
}

void quantized_vec_dot_nvfp4_q8_0(const uint8_t* W, const uint8_t* X, const int8_t* codebook,
                                  const float* scale, float* Y, size_t K) {
  if (X == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::launch<weft::Fmt::NVFP4>(W, nullptr, X, nullptr, codebook, scale, Y, 1, K, 1,
                                 weft::packed(0, K, 1));
}

void production_mul_mat_q5_k_decode(const uint8_t* W, const float* X, uint8_t* Xq, float* Y,
                                    size_t N, size_t K, size_t M) {
  if (X == nullptr || Xq == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::decode_q5_k(W, X, Xq, Y, N, K, M, weft::packed(K / 256 * weft::kQ5_KBytes, K, N));
}

// Q5_K mul_mat: the int8-MFMA GEMM for prefill shapes, the GEMV otherwise
void production_mul_mat_q5_k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N,
                             size_t K, size_t M) {
  if (X == nullptr || Xq == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::mul_mat_q5k(W, X, Xq, Y, N, K, M, weft::packed(K / 256 * weft::kQ5_KBytes, K, N));
}

void quantized_vec_dot_q5_k_q8_k(const uint8_t* W, const uint8_t* X, float* Y, size_t K) {
  if (X == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::launch<weft::Fmt::Q5_K>(W, nullptr, X, nullptr, nullptr, nullptr, Y, 1, K, 1, weft::packed(0, K, 1));
}

void quantized_vec_dot_q6_k_q8_k(const uint8_t* W, const uint8_t* X, float* Y, size_t K) {
  if (X == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::launch<weft::Fmt::Q6_K>(W, nullptr, X, nullptr, nullptr, nullptr, Y, 1, K, 1, weft::packed(0, K, 1));
}

void production_mul_mat_q4_1_decode(const uint8_t* W, const float* X, uint8_t* Xq, float* Y,
                                    size_t N, size_t K, size_t M) {
  if (X == nullptr || Xq == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::decode_q4_1(W, X, Xq, Y, N, K, M, weft::packed(K / 32 * weft::kQ4_1Bytes, K, N));
}

void quantized_vec_dot_q4_1_q8_1(const uint8_t* W, const uint8_t* X, float* Y, size_t K) {
  if (X == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::launch<weft::Fmt::Q4_1>(W, nullptr, X, nullptr, nullptr, nullptr, Y, 1, K, 1, weft::packed(0, K, 1));
}

void quantized_vec_dot_iq2_xs_q8_k(const uint8_t* W, const uint8_t* X, const int8_t* grid,
                                   const int8_t* signs, float* Y, size_t K) {
  if (X == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::launch<weft::Fmt::IQ2_XS>(W, nullptr, X, nullptr, grid, signs, Y, 1, K, 1, weft::packed(0, K, 1));
}

void quantized_vec_dot_iq2_xxs_q8_k(const uint8_t* W, const uint8_t* X, const int8_t* grid,
                                    const int8_t* signs, float* Y, size_t K) {
  if (X == nullptr) return weft::set_error(hipErrorInvalidValue);
  weft::launch<weft::Fmt::IQ2_XXS>(W, nullptr, X, nullptr, grid, signs, Y, 1, K, 1, weft::packed(0, K, 1));
}

}  // extern "C"
