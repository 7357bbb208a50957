// Activation staging for the decode (GEMV) kernels: the M x K fp32
// activation is quantized inside every workgroup into LDS (so the fused
// mul_mat needs one launch), or a caller-supplied quantized activation is
// copied into LDS (vec_dot).  Workgroup 0 also writes the quantized rows to
// the caller's Xq workspace, bit-exact with GGML's quantize_row_q8_*_ref.
#pragma once

#include "weft_common.h"

namespace weft {

// ---------------------------------------------------------------- Q8_K
// LDS image of one Q8_K activation row of K elements (K a multiple of 256,
// so every part and every row stays 16-byte aligned):
//   int8 qs[K] | float d[K/256] (padded to 16 B) | int bp[K/32]
// bp[s] = bsums[2s] + bsums[2s+1], the Q8_K block sum of 32-sub-block s.
struct Q8KView {
  int8_t* qs;
  float* d;
  int* bp;
};

// the d array is padded to 16 bytes so bp is 16-byte aligned
__host__ __device__ inline size_t q8k_d_bytes(int K) {
  return (4 * (size_t)(K / 256) + 15) & ~(size_t)15;
}

__host__ __device__ inline size_t q8k_lds_row_bytes(int K) {
  return (size_t)K + q8k_d_bytes(K) + 4 * (size_t)(K / 32);
}

__device__ inline Q8KView q8k_view(char* base, int K, int m) {
  char* p = base + (size_t)m * q8k_lds_row_bytes(K);
  Q8KView v;
  v.qs = reinterpret_cast<int8_t*>(p);
  v.d = reinterpret_cast<float*>(p + K);
  v.bp = reinterpret_cast<int*>(p + K + q8k_d_bytes(K));
  return v;
}

__device__ inline float4 load_x4(const float* p, bool a16) {
  if (a16) return *reinterpret_cast<const float4*>(p);
  return make_float4(p[0], p[1], p[2], p[3]);
}

// X rows start ldx floats apart; 16-byte loads need every row start aligned
__host__ __device__ inline bool x_rows_a16(const float* X, size_t ldx) {
  return (reinterpret_cast<uintptr_t>(X) & 15) == 0 && ldx % 4 == 0;
}

// Store one quantized Q8_K superblock (index idx = m * nsb + s of this
// launch's activation rows) into LDS, and into xq_out when non-null.
__device__ inline void q8k_store(const Q8KLane& r, int idx, int nsb, int K, int m0,
                                 uint8_t* __restrict__ xq_out, char* lds, int lane) {
  const int m = idx / nsb, s = idx - m * nsb;
  const Q8KView v = q8k_view(lds, K, m);
  const int packed = pack4_i8(r.q);
  reinterpret_cast<int*>(v.qs + 256 * s)[lane] = packed;
  // bsum16 is replicated in its 4 lanes; the 32-sub-block sum adds groups
  // 2t and 2t+1, whose first lanes are 8t and 8t+4.
  const int pair = sum8_of_sum4(r.bsum16);
  if ((lane & 7) == 0) v.bp[8 * s + lane / 8] = pair;
  if (lane == 0) v.d[s] = r.d;
  if (xq_out != nullptr) {
    uint8_t* rec = xq_out + ((size_t)(m0 + m) * nsb + s) * kQ8_KBytes;
    if (lane == 0) *reinterpret_cast<float*>(rec) = r.d;
    reinterpret_cast<int*>(rec + 4)[lane] = packed;
    if (!r.zero && (lane & 3) == 0)
      reinterpret_cast<int16_t*>(rec + 260)[lane / 4] = (int16_t)r.bsum16;
  }
}

// Quantize one Q8_K superblock held as this lane's float4 and store it.
__device__ inline void q8k_quantize_store(float4 x, int idx, int nsb, int K, int m0,
                                          uint8_t* __restrict__ xq_out, char* lds, int lane) {
  q8k_store(q8k_quantize_wave(x, lane), idx, nsb, K, m0, xq_out, lds, lane);
}

// Two-phase Q8_K staging so a kernel can put the activation's loads in front
// of its weight stream: prefetch() issues the loads of this wave's first
// P superblocks (vector loads complete in issue order, so waiting for
// these does not wait for weight loads issued after them); finish()
// quantizes them into LDS and handles any remaining superblocks.  A kernel
// that knows its row length picks P = superblocks per wave, so no load is
// issued twice.
template <int P>
struct Q8KStagerT {
  static constexpr int kPrefetch = P;
  float4 x[kPrefetch];

  __device__ inline void prefetch(const float* __restrict__ X, size_t ldx, int K, int m0, int mb) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int nwaves = blockDim.x / kWave;
    const int nsb = K / 256, total = mb * nsb;
    const bool a16 = x_rows_a16(X, ldx);
#pragma unroll
    for (int i = 0; i < kPrefetch; ++i) {
      const int idx = min(wave + i * nwaves, total - 1);  // clamped: always a valid load
      const int m = idx / nsb, s = idx - m * nsb;
      x[i] = load_x4(X + (size_t)(m0 + m) * ldx + 256 * s + 4 * lane, a16);
    }
  }

  __device__ inline void finish(const float* __restrict__ X, size_t ldx, uint8_t* __restrict__ xq_out,
                                int K, int m0, int mb, char* lds) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int nwaves = blockDim.x / kWave;
    const int nsb = K / 256, total = mb * nsb;
    // quantize every prefetched superblock first (independent straight-line
    // chains the scheduler interleaves), then store the live ones
    Q8KLane r[kPrefetch];
#pragma unroll
    for (int i = 0; i < kPrefetch; ++i) r[i] = q8k_quantize_wave(x[i], lane);
#pragma unroll
    for (int i = 0; i < kPrefetch; ++i) {
      const int idx = wave + i * nwaves;
      if (idx < total) q8k_store(r[i], idx, nsb, K, m0, xq_out, lds, lane);
    }
    const bool a16 = x_rows_a16(X, ldx);
    for (int idx = wave + kPrefetch * nwaves; idx < total; idx += nwaves) {
      const int m = idx / nsb, s = idx - m * nsb;
      const float4 v = load_x4(X + (size_t)(m0 + m) * ldx + 256 * s + 4 * lane, a16);
      q8k_quantize_store(v, idx, nsb, K, m0, xq_out, lds, lane);
    }
  }
};
using Q8KStager = Q8KStagerT<4>;

// Q8_K staging with 16 lanes per superblock (q8k_quantize_16lanes): pass i
// of wave w quantizes superblock 4 (w + i * nwaves) + lane / 16 of the
// launch's rows; P passes are prefetched (a kernel picks P so that they
// cover every superblock), further superblocks are loaded in finish().
template <int P>
struct Q8KStager16 {
  float4 x[P][4];

  __device__ inline void prefetch(const float* __restrict__ X, size_t ldx, int K, int m0, int mb) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int nwaves = blockDim.x / kWave;
    const int nsb = K / 256, total = mb * nsb;
    const bool a16 = x_rows_a16(X, ldx);
#pragma unroll
    for (int i = 0; i < P; ++i) {
      // a wave whose pass i is past the end loads nothing (uniform branch)
      if (4 * (wave + i * nwaves) >= total) break;
      const int idx = min(4 * (wave + i * nwaves) + lane / 16, total - 1);  // clamped: a valid load
      const int m = idx / nsb, s = idx - m * nsb;
      const float* src = X + (size_t)(m0 + m) * ldx + 256 * s + 16 * (lane & 15);
#pragma unroll
      for (int j = 0; j < 4; ++j) x[i][j] = load_x4(src + 4 * j, a16);
    }
  }

  __device__ static inline void store(const Q8K16& r, int idx, int nsb, int K, int m0,
                                      uint8_t* __restrict__ xq_out, char* lds, int part) {
    const int m = idx / nsb, s = idx - m * nsb;
    const Q8KView v = q8k_view(lds, K, m);
    *reinterpret_cast<uint4*>(v.qs + 256 * s + 16 * part) = make_uint4(r.qs[0], r.qs[1], r.qs[2], r.qs[3]);
    // 32-sub-block sum = groups 2t and 2t+1, held by parts 2t and 2t+1
    const int pair = r.bsum + dpp_row_i<kDppXor1>(r.bsum);
    if ((part & 1) == 0) v.bp[8 * s + part / 2] = pair;
    if (part == 0) v.d[s] = r.d;
    if (xq_out != nullptr) {
      uint8_t* rec = xq_out + ((size_t)(m0 + m) * nsb + s) * kQ8_KBytes;
      if (part == 0) *reinterpret_cast<float*>(rec) = r.d;
      uint32_t* q = reinterpret_cast<uint32_t*>(rec + 4 + 16 * part);
      q[0] = r.qs[0];
      q[1] = r.qs[1];
      q[2] = r.qs[2];
      q[3] = r.qs[3];
      if (!r.zero) reinterpret_cast<int16_t*>(rec + 260)[part] = (int16_t)r.bsum;
    }
  }

  __device__ inline void finish(const float* __restrict__ X, size_t ldx, uint8_t* __restrict__ xq_out,
                                int K, int m0, int mb, char* lds) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int nwaves = blockDim.x / kWave;
    const int nsb = K / 256, total = mb * nsb;
    const int part = lane & 15;
    // passes are all-or-nothing per wave except the last superblocks of the
    // final pass; waves without work skip straight to the caller's barrier
    int live = 0;
#pragma unroll
    for (int i = 0; i < P; ++i) live += 4 * (wave + i * nwaves) < total ? 1 : 0;
    if (live == P) {
      Q8K16 r[P];
#pragma unroll
      for (int i = 0; i < P; ++i) r[i] = q8k_quantize_16lanes(x[i], part);
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const int idx = 4 * (wave + i * nwaves) + lane / 16;
        if (idx < total) store(r[i], idx, nsb, K, m0, xq_out, lds, part);
      }
    } else {
#pragma unroll
      for (int i = 0; i < P; ++i) {
        if (i >= live) break;
        const int idx = 4 * (wave + i * nwaves) + lane / 16;
        const Q8K16 r = q8k_quantize_16lanes(x[i], part);
        if (idx < total) store(r, idx, nsb, K, m0, xq_out, lds, part);
      }
    }
    const bool a16 = x_rows_a16(X, ldx);
    for (int w = wave + P * nwaves; 4 * w < total; w += nwaves) {
      const int idx = min(4 * w + lane / 16, total - 1);
      const int m = idx / nsb, s = idx - m * nsb;
      const float* src = X + (size_t)(m0 + m) * ldx + 256 * s + 16 * part;
      float4 v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = load_x4(src + 4 * j, a16);
      const Q8K16 q = q8k_quantize_16lanes(v, part);
      if (4 * w + lane / 16 < total) store(q, idx, nsb, K, m0, xq_out, lds, part);
    }
  }
};

// Quantize rows [m0, m0+mb) of X (row stride ldx floats) into LDS; when
// xq_out is non-null also store the records (Xq row stride K/256 records).
__device__ inline void stage_q8k_quantize(const float* __restrict__ X, size_t ldx,
                                          uint8_t* __restrict__ xq_out, int K, int m0, int mb,
                                          char* lds) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int nwaves = blockDim.x / kWave;
  const int nsb = K / 256;
  const bool a16 = x_rows_a16(X, ldx);
  for (int idx = wave; idx < mb * nsb; idx += nwaves) {
    const int m = idx / nsb, s = idx - m * nsb;
    const float4 x = load_x4(X + (size_t)(m0 + m) * ldx + 256 * s + 4 * lane, a16);
    q8k_quantize_store(x, idx, nsb, K, m0, xq_out, lds, lane);
  }
}

// Copy rows [m0, m0+mb) of a quantized Q8_K activation into LDS.
__device__ inline void stage_q8k_load(const uint8_t* __restrict__ xq, int K, int m0, int mb,
                                      char* lds) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int nwaves = blockDim.x / kWave;
  const int nsb = K / 256;
  for (int idx = wave; idx < mb * nsb; idx += nwaves) {
    const int m = idx / nsb, s = idx - m * nsb;
    const uint8_t* rec = xq + ((size_t)(m0 + m) * nsb + s) * kQ8_KBytes;
    const Q8KView v = q8k_view(lds, K, m);
    reinterpret_cast<int*>(v.qs + 256 * s)[lane] = reinterpret_cast<const int*>(rec + 4)[lane];
    if (lane < 8) {
      const int16_t* bs = reinterpret_cast<const int16_t*>(rec + 260);
      v.bp[8 * s + lane] = (int)bs[2 * lane] + (int)bs[2 * lane + 1];
    }
    if (lane == 0) v.d[s] = *reinterpret_cast<const float*>(rec);
  }
}

// ---------------------------------------------------------------- Q8_0
// LDS image of one Q8_0 activation row: int8 qs[K] | float d[K/32]
// (d is the fp16 scale widened to fp32, as the vec_dot reads it).
struct Q80View {
  int8_t* qs;
  float* d;
};

__host__ __device__ inline size_t q80_lds_row_bytes(int K) {
  return ((size_t)K + 4 * (size_t)(K / 32) + 15) & ~(size_t)15;
}

__device__ inline Q80View q80_view(char* base, int K, int m) {
  char* p = base + (size_t)m * q80_lds_row_bytes(K);
  Q80View v;
  v.qs = reinterpret_cast<int8_t*>(p);
  v.d = reinterpret_cast<float*>(p + K);
  return v;
}

// K must be a multiple of 32; a wave covers 8 blocks (256 values) per step,
// 8 lanes per block.
__device__ inline void stage_q80_quantize(const float* __restrict__ X, size_t ldx,
                                          uint8_t* __restrict__ xq_out, int K, int m0, int mb,
                                          char* lds) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int nwaves = blockDim.x / kWave;
  const int nb = K / 32;
  const int steps = (nb + 7) / 8;
  const bool a16 = x_rows_a16(X, ldx);
  for (int idx = wave; idx < mb * steps; idx += nwaves) {
    const int m = idx / steps, st = idx - m * steps;
    const int b = 8 * st + lane / 8;
    const bool live = b < nb;  // uniform per 8-lane group
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) x = load_x4(X + (size_t)(m0 + m) * ldx + 32 * b + 4 * (lane & 7), a16);
    const Q8_0Lane r = q80_quantize_8lanes(x);
    if (!live) continue;
    const Q80View v = q80_view(lds, K, m);
    const int packed = pack4_i8(r.q);
    reinterpret_cast<int*>(v.qs + 32 * b)[lane & 7] = packed;
    if ((lane & 7) == 0) v.d[b] = fp16_to_fp32(r.dh);
    if (xq_out != nullptr) {
      uint8_t* rec = xq_out + ((size_t)(m0 + m) * nb + b) * kQ8_0Bytes;
      uint16_t* q16 = reinterpret_cast<uint16_t*>(rec + 2 + 4 * (lane & 7));
      q16[0] = (uint16_t)((uint32_t)packed & 0xffffu);
      q16[1] = (uint16_t)((uint32_t)packed >> 16);
      if ((lane & 7) == 0) *reinterpret_cast<uint16_t*>(rec) = (uint16_t)r.dh;
    }
  }
}

__device__ inline void stage_q80_load(const uint8_t* __restrict__ xq, int K, int m0, int mb,
                                      char* lds) {
  const int nb = K / 32;
  const int total = mb * nb * 8;  // 8 lanes per block
  for (int i = threadIdx.x; i < total; i += blockDim.x) {
    const int m = i / (nb * 8);
    const int rem = i - m * nb * 8;
    const int b = rem >> 3, part = rem & 7;
    const uint8_t* rec = xq + ((size_t)(m0 + m) * nb + b) * kQ8_0Bytes;
    const Q80View v = q80_view(lds, K, m);
    const uint16_t* q16 = reinterpret_cast<const uint16_t*>(rec + 2 + 4 * part);
    reinterpret_cast<int*>(v.qs + 32 * b)[part] = (int)((uint32_t)q16[0] | ((uint32_t)q16[1] << 16));
    if (part == 0) v.d[b] = fp16_to_fp32(*reinterpret_cast<const uint16_t*>(rec));
  }
}

// ---------------------------------------------------------------- Q8_1
// LDS image of one Q8_1 activation row: int8 qs[K] | float d[K/32] |
// float s[K/32] (the fp16 d and s widened to fp32, as the vec_dot reads them)
struct Q81View {
  int8_t* qs;
  float* d;
  float* s;
};

__host__ __device__ inline size_t q81_lds_row_bytes(int K) {
  return ((size_t)K + 8 * (size_t)(K / 32) + 15) & ~(size_t)15;
}

__device__ inline Q81View q81_view(char* base, int K, int m) {
  char* p = base + (size_t)m * q81_lds_row_bytes(K);
  Q81View v;
  v.qs = reinterpret_cast<int8_t*>(p);
  v.d = reinterpret_cast<float*>(p + K);
  v.s = v.d + K / 32;
  return v;
}

// as stage_q80_quantize, plus each block's s (quantize_row_q8_1_ref)
__device__ inline void stage_q81_quantize(const float* __restrict__ X, size_t ldx,
                                          uint8_t* __restrict__ xq_out, int K, int m0, int mb,
                                          char* lds) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int nwaves = blockDim.x / kWave;
  const int nb = K / 32;
  const int steps = (nb + 7) / 8;
  const bool a16 = x_rows_a16(X, ldx);
  for (int idx = wave; idx < mb * steps; idx += nwaves) {
    const int m = idx / steps, st = idx - m * steps;
    const int b = 8 * st + lane / 8;
    const bool live = b < nb;  // uniform per 8-lane group
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) x = load_x4(X + (size_t)(m0 + m) * ldx + 32 * b + 4 * (lane & 7), a16);
    const Q8_0Lane r = q80_quantize_8lanes(x);
    const uint32_t sh = q81_sum_half(r);
    if (!live) continue;
    const Q81View v = q81_view(lds, K, m);
    const int packed = pack4_i8(r.q);
    reinterpret_cast<int*>(v.qs + 32 * b)[lane & 7] = packed;
    if ((lane & 7) == 0) {
      v.d[b] = fp16_to_fp32(r.dh);
      v.s[b] = fp16_to_fp32(sh);
    }
    if (xq_out != nullptr) {
      uint8_t* rec = xq_out + ((size_t)(m0 + m) * nb + b) * kQ8_1Bytes;
      uint16_t* q16 = reinterpret_cast<uint16_t*>(rec + 4 + 4 * (lane & 7));
      q16[0] = (uint16_t)((uint32_t)packed & 0xffffu);
      q16[1] = (uint16_t)((uint32_t)packed >> 16);
      if ((lane & 7) == 0) {
        reinterpret_cast<uint16_t*>(rec)[0] = (uint16_t)r.dh;
        reinterpret_cast<uint16_t*>(rec)[1] = (uint16_t)sh;
      }
    }
  }
}

__device__ inline void stage_q81_load(const uint8_t* __restrict__ xq, int K, int m0, int mb,
                                      char* lds) {
  const int nb = K / 32;
  const int total = mb * nb * 8;  // 8 lanes per block
  for (int i = threadIdx.x; i < total; i += blockDim.x) {
    const int m = i / (nb * 8);
    const int rem = i - m * nb * 8;
    const int b = rem >> 3, part = rem & 7;
    const uint8_t* rec = xq + ((size_t)(m0 + m) * nb + b) * kQ8_1Bytes;
    const Q81View v = q81_view(lds, K, m);
    const uint16_t* q16 = reinterpret_cast<const uint16_t*>(rec + 4 + 4 * part);
    reinterpret_cast<int*>(v.qs + 32 * b)[part] = (int)((uint32_t)q16[0] | ((uint32_t)q16[1] << 16));
    if (part == 0) {
      v.d[b] = fp16_to_fp32(reinterpret_cast<const uint16_t*>(rec)[0]);
      v.s[b] = fp16_to_fp32(reinterpret_cast<const uint16_t*>(rec)[1]);
    }
  }
}

}  // namespace weft
