// Batch-1 decode GEMV for the 32- and 64-element formats: Q4_0 x Q8_0
// (18-byte records), MXFP4 x Q8_0 (17), Q4_1 x Q8_1 (20) and NVFP4 x Q8_0
// (36 bytes per 64 values): production_mul_mat_{q4_0,mxfp4,q4_1,nvfp4}_decode
// at M = 1 (examples/kernels/mul_mat/q4_0_decode.py:10-20,
// mxfp4_decode.py:10-23, q4_1_decode.py:10-11, nvfp4_decode.py), rows of up
// to 4096 values.
//
// Semantics (GGML generic vec_dots, ggml-cpu/quants.c):
//   Q4_0  :174-208  y = sum_b (I_b * dw_b) * dx_b,   I_b = sum_32 (q - 8) * x
//   MXFP4 :247-276  y = sum_b (dx_b * e8m0_half(e_b)) * I_b,  I_b = sum_32 kv[q] * x
//   Q4_1  :210-245  y = sum_b (dw_b dx_b) * I_b + m_b * s_b,  I_b = sum_32 q * x
//   NVFP4 :279-313  y = sum_sub (dx * ue4m3(d_sub)) * I_sub over 16-value sub-blocks
//
// gfx950 mapping, as the Q4_K batch-1 kernel: lane j of a row owns 64 values
// (records 2j and 2j + 1, or NVFP4 record j), loaded straight into VGPRs --
// 36, 34, 40 or 36 bytes at a 4-byte aligned base (MXFP4 lanes start at
// byte 0 or 2 of a dword), so a wave reads one row as a contiguous stream
// without any LDS staging.  Its 64 activation values (the same for every
// row), their two fp16 scales (and, for Q4_0, their sums, which turn
// sum (q - 8) x into sum q x - 8 sum x; for Q4_1 the blocks' s) are read
// from LDS into VGPRs once.  Nibbles meet the activation in v_dot4_i32_i8;
// the MXFP4 / NVFP4 caller codebook is looked up four nibbles at a time with
// v_perm_b32 and the scale table is staged in LDS.  A wave walks its rows
// with one row of lookahead (ping-pong registers), rows are summed with DPP.
// The activation is quantized in every workgroup (8 lanes per block,
// bit-exact with quantize_row_q8_0_ref / _q8_1_ref); workgroup 0 writes Xq,
// so the mul_mat is one launch.
#include <algorithm>

#include "activation.h"
#include "kernels.h"
#include "runtime.h"
#include "weft_hip.h"

namespace weft {
namespace {

constexpr int kRecThreads = 1024;
constexpr int kRecWaves = kRecThreads / kWave;

struct RecArgs {
  const uint8_t* W;
  const float* X;
  uint8_t* xq_out;
  const int8_t* codebook;  // MXFP4: int8[16]
  const float* scale;      // MXFP4: fp32[256]
  float* Y;
  int N, K;
  int rows_per_wg;
  size_t ldw;
};

// four nibbles n (one per byte, 0..15) -> bytes of the 16-entry table c0..c3
__device__ __forceinline__ int rec_lookup16(uint32_t n, uint32_t c0, uint32_t c1, uint32_t c2,
                                            uint32_t c3) {
  const uint32_t sel = n & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm(c1, c0, sel);
  const uint32_t hi = __builtin_amdgcn_perm(c3, c2, sel);
  const uint32_t mask = ((n >> 3) & 0x01010101u) * 0xffu;
  return (int)((hi & mask) | (lo & ~mask));
}

enum class RF { Q4_0, MXFP4, Q4_1, NVFP4 };

template <RF F>
__global__ void __launch_bounds__(kRecThreads) rec_gemv_m1_kernel(RecArgs a) {
  constexpr bool kMx = F == RF::MXFP4;
  constexpr bool kNv = F == RF::NVFP4;
  constexpr bool kQ1 = F == RF::Q4_1;
  constexpr bool kTab = kMx || kNv;
  constexpr int kW = kQ1 ? 10 : 9;  // dwords per lane and row
  extern __shared__ __align__(16) char lds[];
  float* tab = reinterpret_cast<float*>(lds);  // MXFP4 / NVFP4 scale table (1 KB)
  char* act = lds + 1024;                      // Q8_0 / Q8_1 activation row
  // bytes per 32 values
  constexpr int kB = kMx ? kMxfp4Bytes : kQ1 ? kQ4_1Bytes : kNv ? kNvfp4Bytes / 2 : kQ4_0Bytes;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int K = a.K;
  const int nrec = K >> 5;     // 32-value blocks: even, <= 128
  const int nlanes = nrec >> 1;
  const bool live = lane < nlanes;
  const int j = min(lane, nlanes - 1);
  const uint32_t boff = (uint32_t)(2 * kB * j);  // the lane's first byte in its row
  const uint32_t a0 = boff & ~3u, sh = boff & 3u;  // sh = 0 but for MXFP4 (0 or 2)
  const uint32_t row_bytes = (uint32_t)(nrec * kB);
  // MXFP4 lanes at sh = 0 need bytes a0 .. a0 + 33: the ninth dword reaches
  // two bytes past them, which the row's last lane may not read
  const bool short9 = a0 + 36 > row_bytes;
  const size_t rb = a.ldw;
  const int row_first = blockIdx.x * a.rows_per_wg + wave;
  const int row_end = min(a.N, blockIdx.x * a.rows_per_wg + a.rows_per_wg);
  const int nrows = row_first < row_end ? (row_end - row_first + kRecWaves - 1) / kRecWaves : 0;

  // activation loads first (8 lanes per Q8_0 block, one 8-block step per
  // wave): waiting for them does not wait for the weight loads issued next
  const int nb = nrec;
  const int b_act = 8 * wave + (lane >> 3);
  float4 xv = make_float4(0.f, 0.f, 0.f, 0.f);
  if (b_act < nb) xv = *reinterpret_cast<const float4*>(a.X + 32 * b_act + 4 * (lane & 7));
  __builtin_amdgcn_sched_barrier(0);

  struct RowBuf {
    uint32_t w[kW];
  };
  auto issue = [&](RowBuf& buf, int k) {
    const int row = min(row_first + k * kRecWaves, a.N - 1);  // clamped: always a valid row
    const uint8_t* p = a.W + (size_t)row * rb + a0;
    const uint4 v0 = *reinterpret_cast<const uint4*>(p);
    const uint4 v1 = *reinterpret_cast<const uint4*>(p + 16);
    buf.w[0] = v0.x, buf.w[1] = v0.y, buf.w[2] = v0.z, buf.w[3] = v0.w;
    buf.w[4] = v1.x, buf.w[5] = v1.y, buf.w[6] = v1.z, buf.w[7] = v1.w;
    if constexpr (kQ1) {
      const uint2 v2 = *reinterpret_cast<const uint2*>(p + 32);
      buf.w[8] = v2.x, buf.w[9] = v2.y;
    } else if (kMx && short9) {
      buf.w[8] = ld_u16(p + 32);
    } else {
      buf.w[8] = *reinterpret_cast<const uint32_t*>(p + 32);
    }
  };
  // the scale table next (one entry per thread): it is needed with the
  // activation, so it does not queue behind the weight rows
  float tsc = 0.f;
  if constexpr (kTab)
    if (threadIdx.x < 256) tsc = a.scale[threadIdx.x];
  __builtin_amdgcn_sched_barrier(0);

  RowBuf bufA, bufB;
  issue(bufA, 0);
  __builtin_amdgcn_sched_barrier(0);

  if constexpr (kTab)
    if (threadIdx.x < 256) tab[threadIdx.x] = tsc;
  {
    const Q8_0Lane r = q80_quantize_8lanes(xv);
    uint32_t sh16 = 0;
    if constexpr (kQ1) sh16 = q81_sum_half(r);  // every lane: a shuffle inside
    if (b_act < nb) {
      const int packed = pack4_i8(r.q);
      if constexpr (kQ1) {
        const Q81View v = q81_view(act, K, 0);
        reinterpret_cast<int*>(v.qs + 32 * b_act)[lane & 7] = packed;
        if ((lane & 7) == 0) {
          v.d[b_act] = fp16_to_fp32(r.dh);
          v.s[b_act] = fp16_to_fp32(sh16);
        }
      } else {
        const Q80View v = q80_view(act, K, 0);
        reinterpret_cast<int*>(v.qs + 32 * b_act)[lane & 7] = packed;
        if ((lane & 7) == 0) v.d[b_act] = fp16_to_fp32(r.dh);
      }
      if (blockIdx.x == 0) {
        constexpr int kXB = kQ1 ? kQ8_1Bytes : kQ8_0Bytes, kXH = kQ1 ? 4 : 2;
        uint8_t* rec = a.xq_out + (size_t)b_act * kXB;
        uint16_t* q16 = reinterpret_cast<uint16_t*>(rec + kXH + 4 * (lane & 7));
        q16[0] = (uint16_t)((uint32_t)packed & 0xffffu);
        q16[1] = (uint16_t)((uint32_t)packed >> 16);
        if ((lane & 7) == 0) {
          reinterpret_cast<uint16_t*>(rec)[0] = (uint16_t)r.dh;
          if constexpr (kQ1) reinterpret_cast<uint16_t*>(rec)[1] = (uint16_t)sh16;
        }
      }
    }
  }
  __syncthreads();

  // this lane's two blocks: low halves (elements 0-15) and high halves (16-31)
  int4 xl[2], xh[2];
  float dx[2], sx[2] = {0.f, 0.f};
  int s8[2];  // -8 * sum x (Q4_0)
  {
    const Q80View v = q80_view(act, K, 0);  // Q8_1's qs and d lie as Q8_0's
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int b = 2 * j + r;
      xl[r] = *reinterpret_cast<const int4*>(v.qs + 32 * b);
      xh[r] = *reinterpret_cast<const int4*>(v.qs + 32 * b + 16);
      dx[r] = v.d[b];
      if constexpr (kQ1) sx[r] = q81_view(act, K, 0).s[b];
      int s = dot4(0x01010101, xl[r].x, 0);
      s = dot4(0x01010101, xl[r].y, s);
      s = dot4(0x01010101, xl[r].z, s);
      s = dot4(0x01010101, xl[r].w, s);
      s = dot4(0x01010101, xh[r].x, s);
      s = dot4(0x01010101, xh[r].y, s);
      s = dot4(0x01010101, xh[r].z, s);
      s = dot4(0x01010101, xh[r].w, s);
      s8[r] = -8 * s;
    }
  }
  uint32_t c0 = 0, c1 = 0, c2 = 0, c3 = 0;
  if constexpr (kTab) {
    const uint8_t* cb = reinterpret_cast<const uint8_t*>(a.codebook);
    c0 = ld_u32_a1(cb);
    c1 = ld_u32_a1(cb + 4);
    c2 = ld_u32_a1(cb + 8);
    c3 = ld_u32_a1(cb + 12);
  }

  auto compute = [&](const RowBuf& buf, int k) {
    const uint32_t* w = buf.w;
    float acc = 0.f;
    if constexpr (kNv) {
      // record j: four UE4M3 sub-block scales, then 8 code bytes per
      // sub-block s (its values 0-7 in the low nibbles, 8-15 in the high);
      // sub-block s meets half s % 2 of activation block 2 j + s / 2
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t u0 = w[1 + 2 * s], u1 = w[2 + 2 * s];
        const int4 x = (s & 1) ? xh[s >> 1] : xl[s >> 1];
        int I = dot4(rec_lookup16(u0 & 0x0f0f0f0fu, c0, c1, c2, c3), x.x, 0);
        I = dot4(rec_lookup16(u1 & 0x0f0f0f0fu, c0, c1, c2, c3), x.y, I);
        I = dot4(rec_lookup16((u0 >> 4) & 0x0f0f0f0fu, c0, c1, c2, c3), x.z, I);
        I = dot4(rec_lookup16((u1 >> 4) & 0x0f0f0f0fu, c0, c1, c2, c3), x.w, I);
        acc += (dx[s >> 1] * tab[(w[0] >> (8 * s)) & 0xffu]) * (float)I;
      }
      const float tot = wave_sum_f(live ? acc : 0.f);
      if (lane == 0) a.Y[row_first + k * kRecWaves] = tot;
      return;
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      uint32_t q[4];
      float ws;
      uint32_t e = 0;
      if constexpr (kMx) {
        // record r at byte sh + 17 r: e, then 16 nibble bytes
        if (r == 0) {
          e = __builtin_amdgcn_alignbyte(w[1], w[0], sh) & 0xffu;
#pragma unroll
          for (int i = 0; i < 4; ++i) q[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh + 1);
        } else {
          // sh = 0: e at byte 17, nibbles at 18; sh = 2: e at 19, nibbles at 20
          e = (w[4] >> (8 * (sh + 1))) & 0xffu;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            q[i] = sh ? w[5 + i] : __builtin_amdgcn_alignbyte(w[5 + i], w[4 + i], 2);
        }
        ws = tab[e];
      } else if constexpr (kQ1) {
        // record r at byte 20 r: fp16 d, fp16 m, then 16 nibble bytes
        ws = fp16_to_fp32(w[5 * r] & 0xffffu);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = w[5 * r + 1 + i];
      } else {
        // record r at byte 18 r: fp16 d, then 16 nibble bytes
        if (r == 0) {
          ws = fp16_to_fp32(w[0] & 0xffffu);
#pragma unroll
          for (int i = 0; i < 4; ++i) q[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
        } else {
          ws = fp16_to_fp32(w[4] >> 16);
#pragma unroll
          for (int i = 0; i < 4; ++i) q[i] = w[5 + i];
        }
      }
      const int xlv[4] = {xl[r].x, xl[r].y, xl[r].z, xl[r].w};
      const int xhv[4] = {xh[r].x, xh[r].y, xh[r].z, xh[r].w};
      int I = kMx || kQ1 ? 0 : s8[r];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t lo = q[i] & 0x0f0f0f0fu, hi = (q[i] >> 4) & 0x0f0f0f0fu;
        if constexpr (kMx) {
          I = dot4(rec_lookup16(lo, c0, c1, c2, c3), xlv[i], I);
          I = dot4(rec_lookup16(hi, c0, c1, c2, c3), xhv[i], I);
        } else {
          I = dot4((int)lo, xlv[i], I);
          I = dot4((int)hi, xhv[i], I);
        }
      }
      if constexpr (kMx)
        acc = ggml_scaled_term(acc, dx[r], ws, (float)I);
      else if constexpr (kQ1)
        acc += (ws * dx[r]) * (float)I + fp16_to_fp32(w[5 * r] >> 16) * sx[r];
      else
        acc += (float)I * ws * dx[r];
    }
    // lanes past the row's last record duplicate it: they add exactly 0
    const float tot = wave_sum_f(live ? acc : 0.f);
    if (lane == 0) a.Y[row_first + k * kRecWaves] = tot;
  };

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

}  // namespace

// Launches the kernel above when the call suits it: one activation row of
// K <= 4096 (K a multiple of 64), 16-byte aligned X, weight rows at 4-byte
// aligned addresses, the MXFP4 / NVFP4 scale table 4-byte aligned.
// fmt: Q4_0 0, MXFP4 1, NVFP4 5, Q4_1 6.
bool decode_rec_m1(int fmt, const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* codebook,
                   const float* scale, float* Y, size_t N, size_t K, const RowStrides& st) {
  const bool mx = fmt == 1 || fmt == 5;  // a codebook and a scale table
  const size_t rec = fmt == 1 ? kMxfp4Bytes : fmt == 5 ? kNvfp4Bytes / 2 : fmt == 6 ? kQ4_1Bytes : kQ4_0Bytes;
  if (fmt != 0 && fmt != 1 && fmt != 5 && fmt != 6) return false;
  const size_t rb = K / 32 * rec;
  const size_t ldw = N > 1 ? st.ldw : rb;
  if (N == 0 || K == 0 || K > 4096 || K % 64 != 0 || X == nullptr || Xq == nullptr || W == nullptr ||
      Y == nullptr || !aligned(X, 16) || !aligned(W, 4) || ldw % 4 != 0 || !aligned(Y, 4) ||
      !aligned(Xq, 2) || N > (size_t)INT32_MAX || (N > 1 && ldw < rb) || ldw >= ((size_t)1 << 40) ||
      (mx && (codebook == nullptr || scale == nullptr || !aligned(scale, 4))))
    return false;
  const int cus = cu_count();
  // 16 rows per workgroup at least (one per wave), two workgroups per CU at most
  const size_t wgs = std::max<size_t>(1, std::min<size_t>(2 * (size_t)cus, (N + kRecWaves - 1) / kRecWaves));
  RecArgs a;
  a.W = W;
  a.X = X;
  a.xq_out = Xq;
  a.codebook = codebook;
  a.scale = scale;
  a.Y = Y;
  a.N = (int)N;
  a.K = (int)K;
  // a CompileOptions NC binding sets the weight rows per workgroup
  const int nc = tile_bindings().nc;
  a.rows_per_wg = nc > 0 ? (int)std::min<size_t>(N, (size_t)nc) : (int)((N + wgs - 1) / wgs);
  a.ldw = ldw;
  const int grid = (int)((N + a.rows_per_wg - 1) / a.rows_per_wg);
  const size_t lds = 1024 + (fmt == 6 ? q81_lds_row_bytes((int)K) : q80_lds_row_bytes((int)K));
  switch (fmt) {
    case 1: rec_gemv_m1_kernel<RF::MXFP4><<<grid, kRecThreads, lds, current_stream()>>>(a); break;
    case 5: rec_gemv_m1_kernel<RF::NVFP4><<<grid, kRecThreads, lds, current_stream()>>>(a); break;
    case 6: rec_gemv_m1_kernel<RF::Q4_1><<<grid, kRecThreads, lds, current_stream()>>>(a); break;
    default: rec_gemv_m1_kernel<RF::Q4_0><<<grid, kRecThreads, lds, current_stream()>>>(a); break;
  }
  check_launch("rec_gemv_m1_kernel");
  return true;
}

}  // namespace weft
