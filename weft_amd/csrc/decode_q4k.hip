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
// Lane t of a 64-item step owns (superblock s = t/8, 16-byte qs chunk
// j = t%8): one 16-byte load of its qs chunk and one of the superblock's
// 16-byte header (the 8 lanes of a superblock share its cache line), so a
// step reads 8 consecutive superblocks (1152 B).  The 32 nibbles of a chunk
// are 16-element halves of sub-blocks 2g and 2g+1 (g = j/2); each half is
// dotted with the Q8_K activation in LDS by four v_dot4_i32_i8, scaled by its
// 6-bit sub-block scale (unpacked in VGPRs with GGML's 32-bit mask trick) and
// folded into one fp32 FMA chain per lane.  Rows are summed with DPP.
//
// Chunk c of a wave's work is step (c % iters) of its row (c / iters).  A
// wave works in rounds of kDepth chunks whose loads are all issued before any
// is consumed.  The activation's loads go out first, then the first round of
// weight loads, then the activation is quantized into LDS (one wave per Q8_K
// superblock, bit-exact with quantize_row_q8_K_ref) while the weights stream
// in.  Workgroup 0 also stores the quantized records into Xq, so the whole
// mul_mat is a single launch.
#include <algorithm>

#include "activation.h"
#include "kernels.h"
#include "pairs.h"
#include "runtime.h"
#include "weft_hip.h"

namespace weft {

constexpr int kQ4KDepth = 6;  // 64-item steps in flight per wave

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
  size_t ldw;            // bytes between weight rows
  size_t ldx;            // elements between activation rows
  PairArgs pair;         // MUL_MAT_ID pairs (pair.ids null: none)
  int accumulate = 0;    // K chunk after the first (q4k_gemv_kernel): add to Y
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

// MB: compile-time bound on the activation rows of one launch (a.mb <= MB).
template <bool A16, int MB, int NT>
__global__ void __launch_bounds__(NT) q4k_gemv_kernel(Q4KArgs a) {
  if (a.pair.ids != nullptr && !resolve_pair(a)) return;
  extern __shared__ __align__(16) char lds[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  constexpr int nwaves = NT / kWave;
  const int K = a.K;
  const int nsb = K >> 8;
  const int items = nsb * 8;
  const int iters = (items + kWave - 1) / kWave;
  const size_t rb = a.ldw;
  const int row0 = blockIdx.x * a.rows_per_wg + wave;
  const int row_end = min(a.N, blockIdx.x * a.rows_per_wg + a.rows_per_wg);
  const int my_rows = row0 < row_end ? (row_end - row0 + nwaves - 1) / nwaves : 0;
  const int nchunks = my_rows * iters;

  uint4 hb[kQ4KDepth], qb[kQ4KDepth];
  // lanes past the row's last item re-read its last item (same cache lines)
  auto issue = [&](int c, uint4& h, uint4& q) {
    const int r = c / iters, it = c - r * iters;
    const int t = min(it * kWave + lane, items - 1);
    const int row = min(row0 + r * nwaves, a.N - 1);  // a wave without rows re-reads a valid row
    const uint8_t* sb = a.W + (size_t)row * rb + (size_t)(t >> 3) * kQ4_KBytes;
    h = load16<A16>(sb);
    q = load16<A16>(sb + 16 + 16 * (t & 7));
  };

  Q8KStager stager;
  if (a.X != nullptr) stager.prefetch(a.X, a.ldx, K, a.m0, a.mb);
  __builtin_amdgcn_sched_barrier(0);
  // The first round's loads are unconditional (straight-line code keeps the
  // in-order wait counts exact): past its last chunk a lane re-requests a
  // chunk it already holds (an L1/L2 hit, never extra HBM traffic).
#pragma unroll
  for (int d = 0; d < kQ4KDepth; ++d) issue(min(d, max(nchunks, 1) - 1), hb[d], qb[d]);
  __builtin_amdgcn_sched_barrier(0);

  if (a.X != nullptr)
    stager.finish(a.X, a.ldx, blockIdx.x == 0 ? a.xq_out : nullptr, K, a.m0, a.mb, lds);
  else
    stage_q8k_load(a.xq_in, K, a.m0, a.mb, lds);
  __syncthreads();

  float acc[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) acc[m] = 0.f;

  for (int base = 0; base < nchunks; base += kQ4KDepth) {
#pragma unroll
    for (int d = 0; d < kQ4KDepth; ++d) {
      const int c = base + d;
      if (c < nchunks) {
        const int r = c / iters, it = c - r * iters;
        const int t = it * kWave + lane;
        const bool live = t < items;
        const int tt = live ? t : items - 1;
        const int s = tt >> 3, j = tt & 7, g = j >> 1, half = j & 1;
        // 6-bit scales and mins of the 8 sub-blocks as bytes of four words
        // (the utmp unpack of ggml-cpu/quants.c:676-681)
        const uint32_t u0 = hb[d].y, u1 = hb[d].z, u2 = hb[d].w;
        const uint32_t sc03 = u0 & 0x3f3f3f3fu;
        const uint32_t sc47 = (u2 & 0x0f0f0f0fu) | (((u0 >> 6) & 0x03030303u) << 4);
        const uint32_t mn03 = u1 & 0x3f3f3f3fu;
        const uint32_t mn47 = ((u2 >> 4) & 0x0f0f0f0fu) | (((u1 >> 6) & 0x03030303u) << 4);
        const uint32_t scw = g < 2 ? sc03 : sc47;
        const uint32_t mnw = g < 2 ? mn03 : mn47;
        const int sh = 16 * (g & 1);
        const int sc_lo = (scw >> sh) & 0xff, sc_hi = (scw >> (sh + 8)) & 0xff;
        const int m_lo = (mnw >> sh) & 0xff, m_hi = (mnw >> (sh + 8)) & 0xff;
        const float dw = fp16_to_fp32(hb[d].x & 0xffffu);
        const float dmin = fp16_to_fp32(hb[d].x >> 16);
        const uint32_t q0 = qb[d].x, q1 = qb[d].y, q2 = qb[d].z, q3 = qb[d].w;
        const int l0 = (int)(q0 & 0x0f0f0f0fu), l1 = (int)(q1 & 0x0f0f0f0fu);
        const int l2 = (int)(q2 & 0x0f0f0f0fu), l3 = (int)(q3 & 0x0f0f0f0fu);
        const int h0 = (int)((q0 >> 4) & 0x0f0f0f0fu), h1 = (int)((q1 >> 4) & 0x0f0f0f0fu);
        const int h2 = (int)((q2 >> 4) & 0x0f0f0f0fu), h3 = (int)((q3 >> 4) & 0x0f0f0f0fu);
#pragma unroll
        for (int m = 0; m < MB; ++m) {
          if (m >= a.mb) break;
          const Q8KView v = q8k_view(lds, K, m);
          const int8_t* xb = v.qs + 256 * s + 64 * g + 16 * half;
          const int4 xl = *reinterpret_cast<const int4*>(xb);
          const int4 xh = *reinterpret_cast<const int4*>(xb + 32);
          int pl = dot4(l0, xl.x, 0);
          pl = dot4(l1, xl.y, pl);
          pl = dot4(l2, xl.z, pl);
          pl = dot4(l3, xl.w, pl);
          int ph = dot4(h0, xh.x, 0);
          ph = dot4(h1, xh.y, ph);
          ph = dot4(h2, xh.z, ph);
          ph = dot4(h3, xh.w, ph);
          // |pl|, |ph| <= 16*15*127 and scales <= 63: 24-bit multiplies are exact
          const int S = __mul24(sc_lo, pl) + __mul24(sc_hi, ph);
          const int2 bp = *reinterpret_cast<const int2*>(v.bp + 8 * s + 2 * g);
          const int Mn = half ? 0 : __mul24(m_lo, bp.x) + __mul24(m_hi, bp.y);
          const float dx = v.d[s];
          const float val = dx * (dw * (float)S - dmin * (float)Mn);
          acc[m] += live ? val : 0.f;
        }
        if (it == iters - 1) {
          const int row = row0 + r * nwaves;
#pragma unroll
          for (int m = 0; m < MB; ++m) {
            if (m >= a.mb) break;
            const float tot = wave_sum_f(acc[m]);
            if (lane == 0) {
              float* yp = a.Y + (size_t)(a.m0 + m) * a.y_stride + row;
              *yp = a.accumulate ? *yp + tot : tot;
            }
            acc[m] = 0.f;
          }
        }
      }
    }
    if (base + kQ4KDepth < nchunks) {
#pragma unroll
      for (int d = 0; d < kQ4KDepth; ++d)
        issue(min(base + kQ4KDepth + d, nchunks - 1), hb[d], qb[d]);
    }
  }
}

// ---------------------------------------------------------------------------
// Batch-1 kernel.  The arithmetic per weight byte decides this kernel on
// CDNA4: a wave64 VALU op occupies a SIMD16 for 4 cycles, so a CU retires
// about one wave-instruction per cycle, and the decode of 1 KB of Q4_K costs
// tens of them.  This variant cuts VALU work per byte:
//   * lane l of a step owns superblock l/4 of the step and its 64-element
//     group g = l%4: 32 B of qs (two 16-byte loads) and the 16-byte header,
//     so one header decode serves 64 weights and a step is 16 consecutive
//     superblocks (2304 B);
//   * that lane meets the same 64 activation values in every row, so they
//     are read from LDS into VGPRs once, after quantization;
//   * load addresses are a wave-uniform row base (SGPRs) plus a lane-constant
//     offset, so the weight stream needs no per-load VALU address math.
// STEPS = steps per row (K <= 4096 * STEPS).  A wave walks its rows
// row_first + k * nwaves with one row of lookahead (ping-pong register
// buffers): the next row's loads are in flight while the current row is
// computed, so every CU keeps ~16 rows in flight and computes as its data
// streams in, instead of bursting all its requests up front and computing
// after the last one lands.
// RB = row buffers: 2 for the ping-pong walk above, 1 when the launch gives
// every wave at most one row.  The library launches <1, 1024, 2> (K <= 4096);
// longer rows go to q4k_gemv_ks_kernel, which splits a row's steps over
// waves instead of holding every step's activation slice in one wave.
template <int STEPS, int NT, int RB>
__global__ void __launch_bounds__(NT) q4k_gemv_m1_kernel(Q4KArgs a) {
  static_assert(RB == 1 || RB == 2, "one or two row buffers");
  if (a.pair.ids != nullptr && !resolve_pair(a)) return;
  extern __shared__ __align__(16) char lds[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  constexpr int nwaves = NT / kWave;
  const int K = a.K;
  const int nsb = K >> 8;
  const size_t rb = a.ldw;
  const int lsb = lane >> 2, g = lane & 3;
  // lane-constant byte offsets of step st (clamped to the row's last superblock)
  int off[STEPS];
  bool live[STEPS];
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    const int sb = 16 * st + lsb;
    live[st] = sb < nsb;
    off[st] = min(sb, nsb - 1) * kQ4_KBytes;
  }
  const int row_first = blockIdx.x * a.rows_per_wg + wave;
  const int row_end = min(a.N, blockIdx.x * a.rows_per_wg + a.rows_per_wg);
  const int nrows = row_first < row_end ? (row_end - row_first + nwaves - 1) / nwaves : 0;

  // 16 lanes per superblock, four superblocks per wave pass: P passes cover
  // the 16 STEPS superblocks of the longest row
  Q8KStager16<(4 * STEPS + nwaves - 1) / nwaves> stager;
  stager.prefetch(a.X, a.ldx, K, a.m0, 1);
  // keep the activation loads ahead of the weight loads: waits are in issue
  // order, so the quantization then waits for X only
  __builtin_amdgcn_sched_barrier(0);

  struct RowBuf {
    uint4 h[STEPS], qa[STEPS], qc[STEPS];
  };
  auto issue = [&](RowBuf& buf, int k) {
    const int row = min(row_first + k * nwaves, a.N - 1);  // clamped: always a valid row
    const uint8_t* wr = a.W + (size_t)row * rb;
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
      const uint8_t* sb = wr + off[st];
      buf.h[st] = *reinterpret_cast<const uint4*>(sb);
      buf.qa[st] = *reinterpret_cast<const uint4*>(sb + 16 + 32 * g);
      buf.qc[st] = *reinterpret_cast<const uint4*>(sb + 32 + 32 * g);
    }
  };
  RowBuf bufA, bufB;
  issue(bufA, 0);  // bufB is only used (and allocated) when RB == 2
  __builtin_amdgcn_sched_barrier(0);

  stager.finish(a.X, a.ldx, blockIdx.x == 0 ? a.xq_out : nullptr, K, a.m0, 1, lds);
  __syncthreads();

  // this lane's activation slice of every step
  int4 xl0[STEPS], xl1[STEPS], xh0[STEPS], xh1[STEPS];
  float dx[STEPS];
  int bp0[STEPS], bp1[STEPS];
  {
    const Q8KView v = q8k_view(lds, K, 0);
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
      const int sb = min(16 * st + lsb, nsb - 1);
      const int8_t* xb = v.qs + 256 * sb + 64 * g;
      xl0[st] = *reinterpret_cast<const int4*>(xb);
      xl1[st] = *reinterpret_cast<const int4*>(xb + 16);
      xh0[st] = *reinterpret_cast<const int4*>(xb + 32);
      xh1[st] = *reinterpret_cast<const int4*>(xb + 48);
      dx[st] = v.d[sb];
      const int2 bp = *reinterpret_cast<const int2*>(v.bp + 8 * sb + 2 * g);
      bp0[st] = bp.x;
      bp1[st] = bp.y;
    }
  }

  auto compute = [&](const RowBuf& buf, int k) {
    float acc = 0.f;
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
      const uint4 h = buf.h[st];
      // 6-bit scale / min of sub-blocks 2g and 2g+1 (the utmp unpack of
      // ggml-cpu/quants.c:676-681, one word picked per lane)
      const uint32_t scw = g < 2 ? (h.y & 0x3f3f3f3fu)
                                 : ((h.w & 0x0f0f0f0fu) | (((h.y >> 6) & 0x03030303u) << 4));
      const uint32_t mnw = g < 2 ? (h.z & 0x3f3f3f3fu)
                                 : (((h.w >> 4) & 0x0f0f0f0fu) | (((h.z >> 6) & 0x03030303u) << 4));
      const int sh = 16 * (g & 1);
      const int sc_lo = (scw >> sh) & 0xff, sc_hi = (scw >> (sh + 8)) & 0xff;
      const int m_lo = (mnw >> sh) & 0xff, m_hi = (mnw >> (sh + 8)) & 0xff;
      const uint4 qa4 = buf.qa[st], qc4 = buf.qc[st];
      int pl = dot4((int)(qa4.x & 0x0f0f0f0fu), xl0[st].x, 0);
      pl = dot4((int)(qa4.y & 0x0f0f0f0fu), xl0[st].y, pl);
      pl = dot4((int)(qa4.z & 0x0f0f0f0fu), xl0[st].z, pl);
      pl = dot4((int)(qa4.w & 0x0f0f0f0fu), xl0[st].w, pl);
      pl = dot4((int)(qc4.x & 0x0f0f0f0fu), xl1[st].x, pl);
      pl = dot4((int)(qc4.y & 0x0f0f0f0fu), xl1[st].y, pl);
      pl = dot4((int)(qc4.z & 0x0f0f0f0fu), xl1[st].z, pl);
      pl = dot4((int)(qc4.w & 0x0f0f0f0fu), xl1[st].w, pl);
      int ph = dot4((int)((qa4.x >> 4) & 0x0f0f0f0fu), xh0[st].x, 0);
      ph = dot4((int)((qa4.y >> 4) & 0x0f0f0f0fu), xh0[st].y, ph);
      ph = dot4((int)((qa4.z >> 4) & 0x0f0f0f0fu), xh0[st].z, ph);
      ph = dot4((int)((qa4.w >> 4) & 0x0f0f0f0fu), xh0[st].w, ph);
      ph = dot4((int)((qc4.x >> 4) & 0x0f0f0f0fu), xh1[st].x, ph);
      ph = dot4((int)((qc4.y >> 4) & 0x0f0f0f0fu), xh1[st].y, ph);
      ph = dot4((int)((qc4.z >> 4) & 0x0f0f0f0fu), xh1[st].z, ph);
      ph = dot4((int)((qc4.w >> 4) & 0x0f0f0f0fu), xh1[st].w, ph);
      // |pl|, |ph| <= 32*15*127 and scales <= 63: 24-bit multiplies are exact
      const int S = __mul24(sc_lo, pl) + __mul24(sc_hi, ph);
      const int Mn = __mul24(m_lo, bp0[st]) + __mul24(m_hi, bp1[st]);
      const float dw = fp16_to_fp32(h.x & 0xffffu);
      const float dmin = fp16_to_fp32(h.x >> 16);
      // lanes past the row's last superblock duplicate it: they add exactly 0
      const float t = dx[st] * (dw * (float)S - dmin * (float)Mn);
      acc += live[st] ? t : 0.f;
    }
    const float tot = wave_sum_f(acc);
    if (lane == 0) a.Y[row_first + k * nwaves] = tot;
  };

  if constexpr (RB == 1) {
    if (nrows > 0) compute(bufA, 0);
    return;
  }
  // Issues inside the loop are unconditional so the in-order wait counts stay
  // exact (a conditional issue forces a full wait on the other path).
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

// ---------------------------------------------------------------------------
// Batch-1 kernel for rows longer than one step (4096 < K <= 4096 * KS), e.g.
// config 3's W_down (K = 11008: 43 superblocks in 3 steps).  The waves of a
// workgroup form groups of KS: wave w computes step w % KS of the rows of
// group w / KS, so each wave keeps one step's activation slice in VGPRs and
// walks its rows with the ping-pong lookahead of q4k_gemv_m1_kernel (rows
// row_first + k * ngroups).  The KS partial sums of a row meet in LDS and
// are added in step order once every wave is done.  Waves past the last
// whole group quantize and wait at the barriers only.
template <int KS, int NT>
__global__ void __launch_bounds__(NT) q4k_gemv_ks_kernel(Q4KArgs a) {
  if (a.pair.ids != nullptr && !resolve_pair(a)) return;
  extern __shared__ __align__(16) char lds[];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  constexpr int nwaves = NT / kWave;
  constexpr int ngroups = nwaves / KS;
  const int K = a.K;
  const int nsb = K >> 8;
  const size_t rb = a.ldw;
  const int st = wave % KS, grp = wave / KS;
  const int lsb = lane >> 2, g = lane & 3;
  // steps take ceil(nsb / KS) <= 16 consecutive superblocks each, so the
  // last step is not left with a short tail (43 = 15 + 15 + 13)
  const int spb = (nsb + KS - 1) / KS;
  const int sb = st * spb + lsb;
  const bool live = lsb < spb && sb < nsb;
  const int off = min(sb, nsb - 1) * kQ4_KBytes;
  const int row_base = blockIdx.x * a.rows_per_wg;
  const int row_end = min(a.N, row_base + a.rows_per_wg);
  const int row_first = row_base + grp;
  const int nrows = grp < ngroups && row_first < row_end ? (row_end - row_first + ngroups - 1) / ngroups : 0;
  // partial sums [row - row_base][step], after the activation row
  float* part = reinterpret_cast<float*>(lds + q8k_lds_row_bytes(K));

  Q8KStager16<(4 * KS + nwaves - 1) / nwaves> stager;
  stager.prefetch(a.X, a.ldx, K, a.m0, 1);
  __builtin_amdgcn_sched_barrier(0);

  struct RowBuf {
    uint4 h, qa, qc;
  };
  auto issue = [&](RowBuf& buf, int k) {
    const int row = min(row_first + k * ngroups, a.N - 1);  // clamped: always a valid row
    const uint8_t* sbp = a.W + (size_t)row * rb + off;
    buf.h = *reinterpret_cast<const uint4*>(sbp);
    buf.qa = *reinterpret_cast<const uint4*>(sbp + 16 + 32 * g);
    buf.qc = *reinterpret_cast<const uint4*>(sbp + 32 + 32 * g);
  };
  RowBuf bufA, bufB;
  issue(bufA, 0);
  __builtin_amdgcn_sched_barrier(0);

  stager.finish(a.X, a.ldx, blockIdx.x == 0 ? a.xq_out : nullptr, K, a.m0, 1, lds);
  __syncthreads();

  int4 xl0, xl1, xh0, xh1;
  float dx;
  int bp0, bp1;
  {
    const Q8KView v = q8k_view(lds, K, 0);
    const int sbc = min(sb, nsb - 1);
    const int8_t* xb = v.qs + 256 * sbc + 64 * g;
    xl0 = *reinterpret_cast<const int4*>(xb);
    xl1 = *reinterpret_cast<const int4*>(xb + 16);
    xh0 = *reinterpret_cast<const int4*>(xb + 32);
    xh1 = *reinterpret_cast<const int4*>(xb + 48);
    dx = v.d[sbc];
    const int2 bp = *reinterpret_cast<const int2*>(v.bp + 8 * sbc + 2 * g);
    bp0 = bp.x;
    bp1 = bp.y;
  }

  auto compute = [&](const RowBuf& buf, int k) {
    const uint4 h = buf.h;
    const uint32_t scw = g < 2 ? (h.y & 0x3f3f3f3fu)
                               : ((h.w & 0x0f0f0f0fu) | (((h.y >> 6) & 0x03030303u) << 4));
    const uint32_t mnw = g < 2 ? (h.z & 0x3f3f3f3fu)
                               : (((h.w >> 4) & 0x0f0f0f0fu) | (((h.z >> 6) & 0x03030303u) << 4));
    const int sh = 16 * (g & 1);
    const int sc_lo = (scw >> sh) & 0xff, sc_hi = (scw >> (sh + 8)) & 0xff;
    const int m_lo = (mnw >> sh) & 0xff, m_hi = (mnw >> (sh + 8)) & 0xff;
    const uint4 qa4 = buf.qa, qc4 = buf.qc;
    int pl = dot4((int)(qa4.x & 0x0f0f0f0fu), xl0.x, 0);
    pl = dot4((int)(qa4.y & 0x0f0f0f0fu), xl0.y, pl);
    pl = dot4((int)(qa4.z & 0x0f0f0f0fu), xl0.z, pl);
    pl = dot4((int)(qa4.w & 0x0f0f0f0fu), xl0.w, pl);
    pl = dot4((int)(qc4.x & 0x0f0f0f0fu), xl1.x, pl);
    pl = dot4((int)(qc4.y & 0x0f0f0f0fu), xl1.y, pl);
    pl = dot4((int)(qc4.z & 0x0f0f0f0fu), xl1.z, pl);
    pl = dot4((int)(qc4.w & 0x0f0f0f0fu), xl1.w, pl);
    int ph = dot4((int)((qa4.x >> 4) & 0x0f0f0f0fu), xh0.x, 0);
    ph = dot4((int)((qa4.y >> 4) & 0x0f0f0f0fu), xh0.y, ph);
    ph = dot4((int)((qa4.z >> 4) & 0x0f0f0f0fu), xh0.z, ph);
    ph = dot4((int)((qa4.w >> 4) & 0x0f0f0f0fu), xh0.w, ph);
    ph = dot4((int)((qc4.x >> 4) & 0x0f0f0f0fu), xh1.x, ph);
    ph = dot4((int)((qc4.y >> 4) & 0x0f0f0f0fu), xh1.y, ph);
    ph = dot4((int)((qc4.z >> 4) & 0x0f0f0f0fu), xh1.z, ph);
    ph = dot4((int)((qc4.w >> 4) & 0x0f0f0f0fu), xh1.w, ph);
    const int S = __mul24(sc_lo, pl) + __mul24(sc_hi, ph);
    const int Mn = __mul24(m_lo, bp0) + __mul24(m_hi, bp1);
    const float dw = fp16_to_fp32(h.x & 0xffffu);
    const float dmin = fp16_to_fp32(h.x >> 16);
    const float t = dx * (dw * (float)S - dmin * (float)Mn);
    const float tot = wave_sum_f(live ? t : 0.f);  // dead lanes duplicate a live superblock
    if (lane == 0) part[(row_first + k * ngroups - row_base) * KS + st] = tot;
  };

  // one row of lookahead, as in q4k_gemv_m1_kernel (deeper prefetch measured
  // slower: the requests queue behind each other)
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
  __syncthreads();
  for (int r = threadIdx.x; r < row_end - row_base; r += NT) {
    float y = part[r * KS];
#pragma unroll
    for (int s = 1; s < KS; ++s) y += part[r * KS + s];
    a.Y[row_base + r] = y;
  }
}

namespace {

constexpr int kMaxRowsPerPass = 4;

template <int MB, int NT>
void launch_one(bool a16, dim3 grid, size_t lds, const Q4KArgs& a) {
  if (a16)
    q4k_gemv_kernel<true, MB, NT><<<grid, NT, lds, current_stream()>>>(a);
  else
    q4k_gemv_kernel<false, MB, NT><<<grid, NT, lds, current_stream()>>>(a);
}

}  // namespace

bool q4k_gemv_fits(size_t K) {
  return K == 0 || K > (size_t)INT32_MAX || q8k_lds_row_bytes((int)K) <= max_lds_per_block();
}

namespace {

// X != null -> quantize (and write Xq), else read xq_in.  pr: MUL_MAT_ID
// pairs (one activation row each, blockIdx.y = pair).
void launch_q4k(const uint8_t* W, const float* X, const uint8_t* xq_in, uint8_t* xq_out, float* Y,
                size_t N, size_t K, size_t M, const RowStrides& st, const PairArgs* pr = nullptr,
                int n_pairs = 0) {
  if (pr != nullptr) M = 1;
  if (N == 0 || M == 0 || K == 0 || (pr != nullptr && n_pairs <= 0)) return;
  if (K % 256 != 0 || W == nullptr || Y == nullptr || (X == nullptr && xq_in == nullptr) ||
      N > (size_t)INT32_MAX || K > (size_t)INT32_MAX || M > (size_t)INT32_MAX ||
      !aligned(W, 2) || !aligned(Y, 4) || (xq_in && !aligned(xq_in, 4)) ||
      (xq_out && !aligned(xq_out, 4)) || (X && !aligned(X, 4)) ||
      !strides_ok(st, K / 256 * kQ4_KBytes, 2, K, N, N, M) || (pr != nullptr && pr->w_es % 2 != 0)) {
    set_error(hipErrorInvalidValue);
    return;
  }
  const size_t row_lds = q8k_lds_row_bytes((int)K);
  const size_t lds_cap = max_lds_per_block();
  if (row_lds > lds_cap) {
    if (pr != nullptr) {
      set_error(hipErrorInvalidValue);  // activation row does not fit in LDS
      return;
    }
    // one launch per activation row and K chunk (a multiple of 1024 values
    // whose Q8_K row fits), staging and quantizing that chunk (workgroup 0
    // writes its Xq records, whole superblocks) and adding its partial dot
    // products to Y, which the first chunk stores; ordered on the stream
    constexpr int NT = 1024;
    size_t kc = 0;
    while (q8k_lds_row_bytes((int)(kc + 1024)) <= lds_cap) kc += 1024;
    const int cus = cu_count();
    const TileBindings& tb = tile_bindings();
    const int rows_per_wg = tb.nc > 0 ? (int)std::min<size_t>(N, (size_t)tb.nc) : (int)((N + cus - 1) / cus);
    const dim3 grid((unsigned)((N + rows_per_wg - 1) / rows_per_wg));
    const size_t xrow = K / 256 * kQ8_KBytes;
    for (size_t m = 0; m < M; ++m) {
      for (size_t k0 = 0; k0 < K; k0 += kc) {
        const size_t k = std::min(kc, K - k0);
        Q4KArgs a;
        a.W = W + k0 / 256 * kQ4_KBytes;
        a.X = X != nullptr ? X + m * st.ldx + k0 : nullptr;
        a.xq_in = xq_in != nullptr ? xq_in + m * xrow + k0 / 256 * kQ8_KBytes : nullptr;
        a.xq_out = xq_out != nullptr ? xq_out + m * xrow + k0 / 256 * kQ8_KBytes : nullptr;
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
        const bool a16 = aligned(a.W, 16) && (N == 1 || st.ldw % 16 == 0);
        launch_one<1, NT>(a16, grid, q8k_lds_row_bytes((int)k), a);
        check_launch("q4k_gemv_kernel");
      }
    }
    return;
  }
  constexpr int NT = 1024;
  const TileBindings& tb = tile_bindings();
  int mb_max = (int)std::min<size_t>(kMaxRowsPerPass, lds_cap / row_lds);
  if (tb.mr > 0) mb_max = std::min(mb_max, tb.mr);
  const int cus = cu_count();
  const int rows_per_wg = tb.nc > 0 ? (int)std::min<size_t>(N, (size_t)tb.nc) : (int)((N + cus - 1) / cus);
  const int grid = (int)((N + rows_per_wg - 1) / rows_per_wg);
  const bool a16 = aligned(W, 16) && (N == 1 || st.ldw % 16 == 0) && (pr == nullptr || pr->w_es % 16 == 0);
  const bool x16 = aligned(X, 16) && (pr == nullptr || (pr->x_s1 % 4 == 0 && pr->x_s2 % 4 == 0));
  // launch over the pairs (or once), gridDim.y pairs at a time
  auto each = [&](Q4KArgs a, int g, auto&& go) {
    if (pr == nullptr) {
      a.pair = PairArgs{};
      go(a, dim3((unsigned)g));
      return;
    }
    for (int p0 = 0; p0 < n_pairs; p0 += kMaxGridY) {
      a.pair = *pr;
      a.pair.pair0 = p0;
      go(a, dim3((unsigned)g, (unsigned)std::min(kMaxGridY, n_pairs - p0)));
    }
  };
  if (M == 1 && X != nullptr && a16 && x16 && K <= 3 * 4096) {
    // batch 1: the register-resident kernels.  One step per row (K <= 4096)
    // runs 1024-thread workgroups, two per CU (62 VGPRs); longer rows split
    // each row's steps over a group of waves (q4k_gemv_ks_kernel).
    const int steps = (int)((K + 4095) / 4096);
    Q4KArgs a;
    a.W = W;
    a.X = X;
    a.xq_in = nullptr;
    a.xq_out = xq_out;
    a.Y = Y;
    a.N = (int)N;
    a.K = (int)K;
    a.m0 = 0;
    a.mb = 1;
    a.y_stride = (long long)st.ldy;
    a.ldw = st.ldw;
    a.ldx = st.ldx;
    if (steps == 1) {
      const int wgs = 2 * cus;
      a.rows_per_wg = tb.nc > 0 ? rows_per_wg : (int)((N + wgs - 1) / wgs);
      const int g1 = (int)((N + a.rows_per_wg - 1) / a.rows_per_wg);
      each(a, g1, [&](const Q4KArgs& b, dim3 g) {
        q4k_gemv_m1_kernel<1, 1024, 2><<<g, 1024, row_lds, current_stream()>>>(b);
        check_launch("q4k_gemv_m1_kernel");
      });
      return;
    }
    // one workgroup per CU: every workgroup quantizes the whole activation,
    // so more (smaller) workgroups only add that prologue (measured: 7.8 us
    // at 768 threads x 256 for config 3's W_down, 9.6 us at 2 per CU)
    const int wgs = cus;
    a.rows_per_wg = tb.nc > 0 ? rows_per_wg : (int)((N + wgs - 1) / wgs);
    const int g1 = (int)((N + a.rows_per_wg - 1) / a.rows_per_wg);
    const size_t lds = row_lds + (size_t)a.rows_per_wg * steps * sizeof(float);
    if (lds <= lds_cap) {  // else the general kernel below
      each(a, g1, [&](const Q4KArgs& b, dim3 g) {
        if (steps == 2)
          q4k_gemv_ks_kernel<2, 1024><<<g, 1024, lds, current_stream()>>>(b);
        else
          q4k_gemv_ks_kernel<3, 768><<<g, 768, lds, current_stream()>>>(b);
        check_launch("q4k_gemv_ks_kernel");
      });
      return;
    }
  }
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
    a.y_stride = (long long)st.ldy;
    a.ldw = st.ldw;
    a.ldx = st.ldx;
    const size_t lds = row_lds * a.mb;
    each(a, grid, [&](const Q4KArgs& b, dim3 g) {
      if (b.mb == 1)
        launch_one<1, NT>(a16, g, lds, b);
      else
        launch_one<kMaxRowsPerPass, NT>(a16, g, lds, b);
      check_launch("q4k_gemv_kernel");
    });
  }
}

}  // namespace

void decode_q4k(const uint8_t* W, const float* X, uint8_t* Xq, float* Y, size_t N, size_t K,
                size_t M, const RowStrides& st) {
  // a row the GEMV's LDS cannot hold goes to the GEMM when it takes the call
  if (!q4k_gemv_fits(K) && gemm_q4k_try(W, X, Xq, Y, N, K, M, st)) return;
  launch_q4k(W, X, nullptr, Xq, Y, N, K, M, st);
}

void decode_q4k_quantized(const uint8_t* W, const uint8_t* Xq, float* Y, size_t N, size_t K,
                          size_t M, const RowStrides& st) {
  launch_q4k(W, nullptr, Xq, nullptr, Y, N, K, M, st);
}

void decode_q4k_pairs(const uint8_t* W, const float* X, const uint8_t* xq_in, uint8_t* xq_out,
                      float* Y, size_t N, size_t K, const RowStrides& st, const PairArgs& pr,
                      int n_pairs) {
  launch_q4k(W, X, xq_in, xq_out, Y, N, K, 1, st, &pr, n_pairs);
}

}  // namespace weft

extern "C" {

void production_mul_mat_q4_k_decode(const uint8_t* W, const float* X, uint8_t* Xq, float* Y,
                                    size_t N, size_t K, size_t M) {
  if (X == nullptr || Xq == nullptr) {
    weft::set_error(hipErrorInvalidValue);
    return;
  }
  weft::decode_q4k(W, X, Xq, Y, N, K, M, weft::packed(K / 256 * weft::kQ4_KBytes, K, N));
}

void quantized_vec_dot_q4_k_q8_k(const uint8_t* W, const uint8_t* X, float* Y, size_t K) {
  if (X == nullptr) {
    weft::set_error(hipErrorInvalidValue);
    return;
  }
  const weft::RowStrides st = weft::packed(K / 256 * weft::kQ4_KBytes, K, 1);
  // a row the GEMV's LDS cannot hold: the GEMM on the quantized row
  if (!weft::q4k_gemv_fits(K)) return weft::mul_mat_q4k_quantized(W, X, Y, 1, K, 1, st);
  weft::launch_q4k(W, nullptr, X, nullptr, Y, 1, K, 1, st);
}

}  // extern "C"
