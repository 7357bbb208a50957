// Row dequantize: row_dequantize_{q4_0,q4_k,iq2_xxs,mxfp4,q6_k,q5_k,nvfp4,q4_1,iq2_xs}
// (examples/kernels/dequantize/*.py; GGML dequantize_row_* in
// ggml-quants.c:401-419, :511-529, :1471-1493, :2416-2440, :1881-1910,
// :1673-1697, :531-552).
//
// Every product here is exact in fp32 (at most 22 significant bits), and
// Q4_K's single subtraction rounds once, so the outputs are bit-exact with
// GGML regardless of contraction.  Q6_K's (d * sc) * q rounds at the second
// product, which has no addend to contract with, so it is bit-exact too.
//
// HBM-bound, mostly writes (Q4_K: 0.56 B read, 4 B written per element).
// The mapping is output-major: lane l of a wave writes elements 4l..4l+3 of
// a 256-element span with one 16-byte store, so each wave store instruction
// covers 1 KB of contiguous output.  The record bytes a lane needs are
// re-read by its neighbours from L2/L1 (the records are 7x smaller than the
// output); Q4_K (config 2) instead stages whole chunks of records in LDS by
// 16-byte direct loads (dq_q4k_lds_kernel).
#include <algorithm>

#include "runtime.h"
#include "weft_common.h"
#include "weft_hip.h"

namespace weft {
namespace {

constexpr int kThreads = 256;

// Y16 (16-byte aligned output) is a template parameter, not a runtime flag:
// with a runtime choice the compiler merges both paths into four strided
// dword stores per lane, which halves the write bandwidth of these
// store-bound kernels.  The 16-byte stores are nontemporal: the output is a
// stream no kernel here reads back.  Measured on config 2 with the outputs
// rotated past the Infinity Cache: 48.2 -> 44.9 us with the weights in HBM,
// 46.6 -> 31.3 us with the weights cache-resident (into one reused output
// buffer, which the cache partly keeps, cached stores are faster).
template <bool Y16>
__device__ __forceinline__ void store4(float* p, float a, float b, float c, float d) {
  if constexpr (Y16) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    const v4f v = {a, b, c, d};
    __builtin_nontemporal_store(v, reinterpret_cast<v4f*>(p));
  } else {
    p[0] = a;
    p[1] = b;
    p[2] = c;
    p[3] = d;
  }
}

__device__ __forceinline__ uint32_t ld32(const uint8_t* p, bool a4) {
  return a4 ? *reinterpret_cast<const uint32_t*>(p) : ld_u32_a2(p);
}

// Q4_K: a wave dequantizes U superblocks per pass, lane l writing elements
// 4l..4l+3 of each; all U passes' loads (the 16-byte header and the lane's
// nibble word) are issued before the first is used, so a wave keeps U
// records in flight instead of one.
template <int U, bool A16, bool Y16>
__global__ void __launch_bounds__(kThreads) dq_q4k_kernel(const uint8_t* __restrict__ W,
                                                          float* __restrict__ Y, long long nsb) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long wave = ((long long)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const long long nwaves = (long long)gridDim.x * blockDim.x / kWave;
  const bool a4 = (reinterpret_cast<uintptr_t>(W) & 3) == 0;
  const int g = lane >> 4;           // 64-element group
  const int e = (lane & 15) * 4;     // offset inside the group
  const int sub = 2 * g + (e >= 32); // 32-element sub-block
  const int qoff = 16 + 32 * g + (e & 31);
  const int shift = e >= 32 ? 4 : 0;
  for (long long s0 = wave * U; s0 < nsb; s0 += nwaves * U) {
    uint4 h[U];
    uint32_t qs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint8_t* rec = W + min(s0 + u, nsb - 1) * kQ4_KBytes;  // clamped: a valid record
      if constexpr (A16) {
        h[u] = *reinterpret_cast<const uint4*>(rec);
        qs[u] = *reinterpret_cast<const uint32_t*>(rec + qoff);
      } else {
        h[u] = make_uint4(ld32(rec, a4), ld32(rec + 4, a4), ld32(rec + 8, a4), ld32(rec + 12, a4));
        qs[u] = ld32(rec + qoff, a4);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (s0 + u >= nsb) break;
      int sc, m;
      q4k_scale_min(sub, h[u].y, h[u].z, h[u].w, sc, m);
      const float d = fp16_to_fp32(h[u].x & 0xffffu), dmin = fp16_to_fp32(h[u].x >> 16);
      const float d1 = d * (float)sc, m1 = dmin * (float)m;
      const uint32_t n = (qs[u] >> shift) & 0x0f0f0f0fu;
      store4<Y16>(Y + (s0 + u) * 256 + 4 * lane, d1 * (float)(n & 0xff) - m1,
                  d1 * (float)((n >> 8) & 0xff) - m1, d1 * (float)((n >> 16) & 0xff) - m1,
                  d1 * (float)(n >> 24) - m1);
    }
  }
}

// Q4_K from LDS-staged chunks: a workgroup (4 waves) walks chunks of 64
// superblocks (9216 record bytes), copying each with nine wave-wide 16-byte
// direct loads -- whole cache lines, one request per 16 bytes -- into one of
// two LDS buffers a chunk ahead, then each wave dequantizes 16 superblocks
// from LDS (the header broadcast, the lane's nibble word) and writes them as
// 16 KB of contiguous 16-byte nontemporal stores.  The small per-lane record
// reads of dq_q4k_kernel interleaved with the write stream are what held
// that kernel at ~1.5 x the streaming-write time of the output.
typedef __attribute__((address_space(3))) void* dq_lds_ptr;
constexpr int kDqChunk = 64;                        // superblocks per chunk
constexpr int kDqChunkBytes = kDqChunk * kQ4_KBytes;  // 9216
static_assert(kDqChunkBytes % 1024 == 0, "whole wave-wide loads");

// 16 bytes per lane from g into LDS [lds + 16 lane, +16); the kernel waits
// (s_waitcnt) itself
__device__ __forceinline__ void dq_dma16(const uint8_t* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(g)
               : "memory", "m0");
}

__global__ void __launch_bounds__(kThreads) dq_q4k_lds_kernel(const uint8_t* __restrict__ W,
                                                              float* __restrict__ Y, long long nsb) {
  __shared__ __align__(16) uint8_t buf[2][kDqChunkBytes];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  const int g = lane >> 4;
  const int e = (lane & 15) * 4;
  const int sub = 2 * g + (e >= 32);
  const int qoff = 16 + 32 * g + (e & 31);
  const int shift = e >= 32 ? 4 : 0;
  const long long nchunks = (nsb + kDqChunk - 1) / kDqChunk;
  const long long total = nsb * kQ4_KBytes;  // record bytes (a multiple of 16)
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(dq_lds_ptr)&buf[0][0]);
  // chunk c's loads: wave w issues wave-wide loads i = w + 4 j (< 9); bytes
  // past the last record re-read the last 16 (never used)
  auto issue = [&](long long c, int slot) {
    const long long base = c * kDqChunkBytes;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int i = wave + 4 * j;
      if (i < kDqChunkBytes / 1024) {
        const long long off = min(base + 1024 * i + 16 * lane, total - 16);
        dq_dma16(W + off, lds0 + (uint32_t)(slot * kDqChunkBytes + 1024 * i));
      }
    }
  };
  long long c = blockIdx.x;
  if (c < nchunks) issue(c, 0);
  for (int k = 0; c < nchunks; c += gridDim.x, ++k) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // chunk c is in LDS for every wave; the other buffer is free
    if (c + gridDim.x < nchunks) issue(c + gridDim.x, (k + 1) & 1);
    const uint8_t* cb = buf[k & 1];
#pragma unroll 4
    for (int u = 0; u < kDqChunk / 4; ++u) {
      const int sl = 16 * wave + u;
      const long long sb = c * kDqChunk + sl;
      if (sb >= nsb) break;
      const uint4 h = *reinterpret_cast<const uint4*>(cb + kQ4_KBytes * sl);
      const uint32_t qs = *reinterpret_cast<const uint32_t*>(cb + kQ4_KBytes * sl + qoff);
      int sc, m;
      q4k_scale_min(sub, h.y, h.z, h.w, sc, m);
      const float d = fp16_to_fp32(h.x & 0xffffu), dmin = fp16_to_fp32(h.x >> 16);
      const float d1 = d * (float)sc, m1 = dmin * (float)m;
      const uint32_t n = (qs >> shift) & 0x0f0f0f0fu;
      store4<true>(Y + sb * 256 + 4 * lane, d1 * (float)(n & 0xff) - m1, d1 * (float)((n >> 8) & 0xff) - m1,
                   d1 * (float)((n >> 16) & 0xff) - m1, d1 * (float)(n >> 24) - m1);
    }
  }
}

// The other formats staged the same way: a 256-value unit (8 Q4_0 / Q4_1 /
// MXFP4 records, 4 NVFP4 records, one Q5_K / Q6_K superblock) per wave
// step, lane l producing elements 4l..4l+3 from the unit's bytes in LDS with
// the per-lane arithmetic of the kernels below (bit-identical results).
struct DqTab {
  const int8_t* codebook;
  const float* scale;
};
struct DqQ40 {
  static constexpr int kVals = 32, kRec = kQ4_0Bytes;
  __device__ static float4 lane4(const uint8_t* u, int lane, const DqTab&) {
    const int p = lane & 7, shift = p >= 4 ? 4 : 0;
    const uint8_t* rec = u + (lane >> 3) * kRec;
    const float d = fp16_to_fp32(ld_u16(rec));
    const uint32_t qs = ld_u32_a2(rec + 2 + 4 * (p & 3));
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)((int)((qs >> (8 * i + shift)) & 0xf) - 8) * d;
    return make_float4(v[0], v[1], v[2], v[3]);
  }
};
struct DqMx {
  static constexpr int kVals = 32, kRec = kMxfp4Bytes;
  __device__ static float4 lane4(const uint8_t* u, int lane, const DqTab& t) {
    const int p = lane & 7, shift = p >= 4 ? 4 : 0;
    const uint8_t* rec = u + (lane >> 3) * kRec;
    const float d = t.scale[rec[0]];
    const uint32_t qs = ld_u32_a1(rec + 1 + 4 * (p & 3));
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)t.codebook[(qs >> (8 * i + shift)) & 0xf] * d;
    return make_float4(v[0], v[1], v[2], v[3]);
  }
};
struct DqQ41 {
  static constexpr int kVals = 32, kRec = kQ4_1Bytes;
  __device__ static float4 lane4(const uint8_t* u, int lane, const DqTab&) {
#pragma clang fp contract(off)
    const int p = lane & 7, shift = p >= 4 ? 4 : 0;
    const uint8_t* rec = u + (lane >> 3) * kRec;
    const float d = fp16_to_fp32(ld_u16(rec)), m = fp16_to_fp32(ld_u16(rec + 2));
    const uint32_t qs = ld_u32_a2(rec + 4 + 4 * (p & 3));
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)((qs >> (8 * i + shift)) & 0xf) * d + m;
    return make_float4(v[0], v[1], v[2], v[3]);
  }
};
struct DqNv {
  static constexpr int kVals = 64, kRec = kNvfp4Bytes;
  __device__ static float4 lane4(const uint8_t* u, int lane, const DqTab& t) {
    const int p = lane & 15, s = p >> 2, shift = (p & 2) ? 4 : 0;
    const uint8_t* rec = u + (lane >> 4) * kRec;
    const float d = t.scale[rec[s]];
    const uint32_t qs = ld_u32_a1(rec + 4 + 8 * s + 4 * (p & 1));
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)t.codebook[(qs >> (8 * i + shift)) & 0xf] * d;
    return make_float4(v[0], v[1], v[2], v[3]);
  }
};
struct DqQ6K {
  static constexpr int kVals = 256, kRec = kQ6_KBytes;
  __device__ static float4 lane4(const uint8_t* rec, int lane, const DqTab&) {
    const int e = 4 * lane, h = e >> 7, i = e & 127;
    const uint32_t ql = ld_u32_a1(rec + 64 * h + (i & 63));
    const uint32_t qh = ld_u32_a1(rec + 128 + 32 * h + (i & 31));
    const int sc = (int)(int8_t)rec[192 + (e >> 4)];
    const uint32_t dh = (uint32_t)rec[208] | ((uint32_t)rec[209] << 8);
    const float dsc = fp16_to_fp32(dh) * (float)sc;
    const uint32_t q = ((ql >> (4 * (i >> 6))) & 0x0f0f0f0fu) | (((qh >> (2 * (i >> 5))) & 0x03030303u) << 4);
    return make_float4(dsc * (float)((int)(q & 0xff) - 32), dsc * (float)((int)((q >> 8) & 0xff) - 32),
                       dsc * (float)((int)((q >> 16) & 0xff) - 32), dsc * (float)((int)(q >> 24) - 32));
  }
};
struct DqQ5K {
  static constexpr int kVals = 256, kRec = kQ5_KBytes;
  __device__ static float4 lane4(const uint8_t* rec, int lane, const DqTab&) {
    const int g = lane >> 4, e = (lane & 15) * 4, sub = 2 * g + (e >= 32);
    const int shift = e >= 32 ? 4 : 0;
    uint32_t hw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) hw[i] = ld_u32_a2(rec + 4 * i);
    const uint32_t qs = ld_u32_a2(rec + 48 + 32 * g + (e & 31)), qh = ld_u32_a2(rec + 16 + (e & 31));
    int sc, m;
    q4k_scale_min(sub, hw[1], hw[2], hw[3], sc, m);
    const float d = fp16_to_fp32(hw[0] & 0xffffu), dmin = fp16_to_fp32(hw[0] >> 16);
    const float d1 = d * (float)sc, m1 = dmin * (float)m;
    const uint32_t n = ((qs >> shift) & 0x0f0f0f0fu) | (((qh >> sub) & 0x01010101u) << 4);
    return make_float4(d1 * (float)(n & 0xff) - m1, d1 * (float)((n >> 8) & 0xff) - m1,
                       d1 * (float)((n >> 16) & 0xff) - m1, d1 * (float)(n >> 24) - m1);
  }
};

template <class F>
__global__ void __launch_bounds__(kThreads) dq_chunk_kernel(const uint8_t* __restrict__ W, DqTab t,
                                                            float* __restrict__ Y, long long K) {
  constexpr int kUnit = 256 / F::kVals * F::kRec;               // bytes per 256 values
  constexpr int kLoads = (kDqChunk * kUnit + 1023) / 1024;      // wave-wide loads per chunk
  __shared__ __align__(16) uint8_t buf[2][kLoads * 1024];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  const long long nunits = (K + 255) / 256;
  const long long nchunks = (nunits + kDqChunk - 1) / kDqChunk;
  const long long total = K / F::kVals * F::kRec;  // record bytes (a multiple of 4)
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(dq_lds_ptr)&buf[0][0]);
  auto issue = [&](long long c, int slot) {
    const long long base = c * kDqChunk * kUnit;
#pragma unroll
    for (int j = 0; j < (kLoads + 3) / 4; ++j) {
      const int i = wave + 4 * j;
      if (i < kLoads) {
        const long long off = min(base + 1024 * i + 16 * lane, total - 16);  // past the end: re-read
        dq_dma16(W + off, lds0 + (uint32_t)(slot * kLoads * 1024 + 1024 * i));
      }
    }
  };
  long long c = blockIdx.x;
  if (c < nchunks) issue(c, 0);
  for (int k = 0; c < nchunks; c += gridDim.x, ++k) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // chunk c is in LDS for every wave; the other buffer is free
    if (c + gridDim.x < nchunks) issue(c + gridDim.x, (k + 1) & 1);
    const uint8_t* cb = buf[k & 1];
#pragma unroll 4
    for (int u = 0; u < kDqChunk / 4; ++u) {
      const int ul = 16 * wave + u;
      const long long e0 = (c * kDqChunk + ul) * 256 + 4 * lane;
      if (e0 >= K) break;  // K is a multiple of 32: a lane's four values are all in or all out
      const float4 v = F::lane4(cb + kUnit * ul, lane, t);
      store4<true>(Y + e0, v.x, v.y, v.z, v.w);
    }
  }
}

// The chunk kernel when W is 4-byte aligned (16-byte direct loads), Y
// 16-byte aligned and the record bytes whole 16-byte chunks (no lane's 16
// bytes straddle the end); false: the caller runs its per-lane kernel.
template <class F>
bool launch_dq_chunk(const uint8_t* W, DqTab t, float* Y, long long K) {
  if (!aligned(W, 4) || !aligned(Y, 16) || (K / F::kVals * F::kRec) % 16 != 0) return false;
  const long long nchunks = ((K + 255) / 256 + kDqChunk - 1) / kDqChunk;
  const int g = (int)std::max<long long>(1, std::min<long long>(nchunks, 2LL * cu_count()));
  dq_chunk_kernel<F><<<g, kThreads, 0, current_stream()>>>(W, t, Y, K);
  check_launch("dq_chunk_kernel");
  return true;
}

// Q4_0 / MXFP4: 8 lanes per 32-block, 8 blocks per wave step
template <bool MX, bool Y16>
__global__ void __launch_bounds__(kThreads) dq_32_kernel(const uint8_t* __restrict__ W,
                                                         const int8_t* __restrict__ codebook,
                                                         const float* __restrict__ scale,
                                                         float* __restrict__ Y, long long nb) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long wave = ((long long)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const long long nwaves = (long long)gridDim.x * blockDim.x / kWave;
  const int p = lane & 7;
  const int shift = p >= 4 ? 4 : 0;
  const long long steps = (nb + 7) / 8;
  for (long long st = wave; st < steps; st += nwaves) {
    const long long b = 8 * st + lane / 8;
    if (b >= nb) continue;
    float v[4];
    if constexpr (MX) {
      const uint8_t* rec = W + b * kMxfp4Bytes;
      const float d = scale[rec[0]];
      const uint32_t qs = ld_u32_a1(rec + 1 + 4 * (p & 3));
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (float)codebook[(qs >> (8 * i + shift)) & 0xf] * d;
    } else {
      const uint8_t* rec = W + b * kQ4_0Bytes;
      const float d = fp16_to_fp32(ld_u16(rec));
      const uint32_t qs = ld_u32_a2(rec + 2 + 4 * (p & 3));
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (float)((int)((qs >> (8 * i + shift)) & 0xf) - 8) * d;
    }
    store4<Y16>(Y + b * 32 + 4 * p, v[0], v[1], v[2], v[3]);
  }
}

// NVFP4 (dequantize_row_nvfp4, ggml-quants.c:531-552): 16 lanes per 36-byte
// record, lane p writing elements 4p..4p+3 of sub-block s = p / 4: the low
// (p % 4 < 2) or high nibbles of qs word 4 + 8 s + 4 (p % 2), times the
// decoded UE4M3 scale scale[d[s]].  Records carry no alignment.
template <bool Y16>
__global__ void __launch_bounds__(kThreads) dq_nvfp4_kernel(const uint8_t* __restrict__ W,
                                                            const int8_t* __restrict__ codebook,
                                                            const float* __restrict__ scale,
                                                            float* __restrict__ Y, long long nb) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long wave = ((long long)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const long long nwaves = (long long)gridDim.x * blockDim.x / kWave;
  const int p = lane & 15, s = p >> 2;
  const int shift = (p & 2) ? 4 : 0;
  for (long long st = wave; 4 * st < nb; st += nwaves) {
    const long long b = 4 * st + lane / 16;
    if (b >= nb) continue;
    const uint8_t* rec = W + b * kNvfp4Bytes;
    const float d = scale[rec[s]];
    const uint32_t qs = ld_u32_a1(rec + 4 + 8 * s + 4 * (p & 1));
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)codebook[(qs >> (8 * i + shift)) & 0xf] * d;
    store4<Y16>(Y + b * 64 + 4 * p, v[0], v[1], v[2], v[3]);
  }
}

// Q6_K (dequantize_row_q6_K, ggml-quants.c:1881-1910): lane l of a wave
// writes elements e = 4l..4l+3 of a superblock; they share one ql word (half
// h = e / 128, byte 64 h + e % 64, nibble (e % 128) / 64), one qh word (byte
// 128 + 32 h + e % 32, bits 2 ((e % 128) / 32)) and one scale (e / 16).
// y = (d * sc) * (q - 32): two fp32 products rounded in GGML's order.
// Records are 210 bytes with no alignment (the Weft encoding declares none),
// so every load is bytewise; U superblocks are in flight per wave.
template <int U, bool Y16>
__global__ void __launch_bounds__(kThreads) dq_q6k_kernel(const uint8_t* __restrict__ W,
                                                          float* __restrict__ Y, long long nsb) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long wave = ((long long)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const long long nwaves = (long long)gridDim.x * blockDim.x / kWave;
  const int e = 4 * lane, h = e >> 7, i = e & 127;
  const int qlo = 64 * h + (i & 63), qls = 4 * (i >> 6);
  const int qho = 128 + 32 * h + (i & 31), qhs = 2 * (i >> 5);
  for (long long s0 = wave * U; s0 < nsb; s0 += nwaves * U) {
    uint32_t ql[U], qh[U], dh[U];
    int sc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint8_t* rec = W + min(s0 + u, nsb - 1) * kQ6_KBytes;  // clamped: a valid record
      ql[u] = ld_u32_a1(rec + qlo);
      qh[u] = ld_u32_a1(rec + qho);
      sc[u] = (int)(int8_t)rec[192 + (e >> 4)];
      dh[u] = (uint32_t)rec[208] | ((uint32_t)rec[209] << 8);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (s0 + u >= nsb) break;
      const float dsc = fp16_to_fp32(dh[u]) * (float)sc[u];
      const uint32_t q = ((ql[u] >> qls) & 0x0f0f0f0fu) | (((qh[u] >> qhs) & 0x03030303u) << 4);
      store4<Y16>(Y + (s0 + u) * 256 + e, dsc * (float)((int)(q & 0xff) - 32),
                  dsc * (float)((int)((q >> 8) & 0xff) - 32), dsc * (float)((int)((q >> 16) & 0xff) - 32),
                  dsc * (float)((int)(q >> 24) - 32));
    }
  }
}

// Q5_K (dequantize_row_q5_K, ggml-quants.c:1673-1697): as Q4_K, lane l
// writing elements 4l..4l+3, with the fifth bit of each code from qh byte
// e % 32, bit e / 32.  d * sc * q (<= 22 bits) and dmin * m are exact, the
// subtraction rounds once: bit-exact.
template <int U, bool Y16>
__global__ void __launch_bounds__(kThreads) dq_q5k_kernel(const uint8_t* __restrict__ W,
                                                          float* __restrict__ Y, long long nsb) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long wave = ((long long)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const long long nwaves = (long long)gridDim.x * blockDim.x / kWave;
  const int g = lane >> 4;           // 64-element group
  const int e = (lane & 15) * 4;     // offset inside the group
  const int sub = 2 * g + (e >= 32); // 32-element sub-block
  const int qoff = 48 + 32 * g + (e & 31), hoff = 16 + (e & 31);
  const int shift = e >= 32 ? 4 : 0;
  for (long long s0 = wave * U; s0 < nsb; s0 += nwaves * U) {
    uint32_t hw[U][4], qs[U], qh[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint8_t* rec = W + min(s0 + u, nsb - 1) * kQ5_KBytes;  // clamped: a valid record
#pragma unroll
      for (int i = 0; i < 4; ++i) hw[u][i] = ld_u32_a2(rec + 4 * i);
      qs[u] = ld_u32_a2(rec + qoff);
      qh[u] = ld_u32_a2(rec + hoff);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (s0 + u >= nsb) break;
      int sc, m;
      q4k_scale_min(sub, hw[u][1], hw[u][2], hw[u][3], sc, m);
      const float d = fp16_to_fp32(hw[u][0] & 0xffffu), dmin = fp16_to_fp32(hw[u][0] >> 16);
      const float d1 = d * (float)sc, m1 = dmin * (float)m;
      const uint32_t n = ((qs[u] >> shift) & 0x0f0f0f0fu) | (((qh[u] >> sub) & 0x01010101u) << 4);
      store4<Y16>(Y + (s0 + u) * 256 + 4 * lane, d1 * (float)(n & 0xff) - m1,
                  d1 * (float)((n >> 8) & 0xff) - m1, d1 * (float)((n >> 16) & 0xff) - m1,
                  d1 * (float)(n >> 24) - m1);
    }
  }
}

// IQ2_XXS: one wave per superblock; lane l -> elements 4l..4l+3
template <bool Y16>
__global__ void __launch_bounds__(kThreads) dq_iq2xxs_kernel(const uint8_t* __restrict__ W,
                                                             const int8_t* __restrict__ grid,
                                                             const int8_t* __restrict__ signs,
                                                             float* __restrict__ Y, long long nsb) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long wave = ((long long)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const long long nwaves = (long long)gridDim.x * blockDim.x / kWave;
  const int c = lane >> 1;     // 8-element chunk 0..31
  const int h = lane & 1;      // which 4 of the 8
  const int g = c >> 2, l = c & 3;
  for (long long s = wave; s < nsb; s += nwaves) {
    const uint8_t* rec = W + s * kIq2xxsBytes;
    const float d = fp16_to_fp32(ld_u16(rec));
    const uint32_t idx = rec[2 + 8 * g + l];
    const uint32_t meta = ld_u32_a2(rec + 2 + 8 * g + 4);
    const float db = d * (0.5f + (float)(meta >> 28)) * 0.25f;
    const int sidx = (int)((meta >> (7 * l)) & 127u);
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * h + i;
      v[i] = (float)((int)grid[8 * idx + j] * (int)signs[8 * sidx + j]) * db;
    }
    store4<Y16>(Y + s * 256 + 4 * lane, v[0], v[1], v[2], v[3]);
  }
}

// Q4_1 (dequantize_row_q4_1, ggml-quants.c:421-439): 8 lanes per 32-block;
// q * d rounded, then + m rounded, as the C expression states
template <bool Y16>
__global__ void __launch_bounds__(kThreads) dq_q41_kernel(const uint8_t* __restrict__ W,
                                                          float* __restrict__ Y, long long nb) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & (kWave - 1);
  const long long wave = ((long long)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const long long nwaves = (long long)gridDim.x * blockDim.x / kWave;
  const int p = lane & 7;
  const int shift = p >= 4 ? 4 : 0;
  const long long steps = (nb + 7) / 8;
  for (long long st = wave; st < steps; st += nwaves) {
    const long long b = 8 * st + lane / 8;
    if (b >= nb) continue;
    const uint8_t* rec = W + b * kQ4_1Bytes;
    const float d = fp16_to_fp32(ld_u16(rec)), m = fp16_to_fp32(ld_u16(rec + 2));
    const uint32_t qs = ld_u32_a2(rec + 4 + 4 * (p & 3));
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (float)((qs >> (8 * i + shift)) & 0xf) * d + m;
    store4<Y16>(Y + b * 32 + 4 * p, v[0], v[1], v[2], v[3]);
  }
}

// IQ2_XS (dequantize_row_iq2_xs, ggml-quants.c:2444-2467): one wave per
// superblock, lane l -> elements 4l..4l+3 of 8-element entry c = l / 2:
// grid row = bits 0-8 of u16 word c, sign row = bits 9-15, scale nibble
// c % 4 < 2 ? low : high of scales[c / 4], db = (d (0.5 + s)) 0.25
template <bool Y16>
__global__ void __launch_bounds__(kThreads) dq_iq2xs_kernel(const uint8_t* __restrict__ W,
                                                            const int8_t* __restrict__ grid,
                                                            const int8_t* __restrict__ signs,
                                                            float* __restrict__ Y, long long nsb) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long wave = ((long long)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const long long nwaves = (long long)gridDim.x * blockDim.x / kWave;
  const int c = lane >> 1, h = lane & 1;
  for (long long s = wave; s < nsb; s += nwaves) {
    const uint8_t* rec = W + s * kIq2xsBytes;
    const float d = fp16_to_fp32(ld_u16(rec));
    const uint32_t word = ld_u16(rec + 2 + 2 * c);
    const uint32_t sb = rec[66 + (c >> 2)];
    const uint32_t sc = (c & 3) < 2 ? sb & 0xfu : sb >> 4;
    const float db = d * (0.5f + (float)sc) * 0.25f;
    const int gi = (int)(word & 511u), si = (int)(word >> 9);
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = 4 * h + i;
      v[i] = (float)((int)grid[8 * gi + j] * (int)signs[8 * si + j]) * db;
    }
    store4<Y16>(Y + s * 256 + 4 * lane, v[0], v[1], v[2], v[3]);
  }
}

int grid_for(long long waves_needed) {
  const long long per_block = kThreads / kWave;
  const long long cap = (long long)cu_count() * 16;
  return (int)std::max<long long>(1, std::min<long long>(cap, (waves_needed + per_block - 1) / per_block));
}

bool bad(const void* W, size_t wa, const float* Y) {
  return W == nullptr || Y == nullptr || !aligned(W, wa) || !aligned(Y, 4);
}

}  // namespace
}  // namespace weft

extern "C" {

void row_dequantize_q4_k(const uint8_t* W, float* Y, size_t K) {
  using namespace weft;
  if (K == 0) return;
  if (K % 256 || bad(W, 2, Y)) return set_error(hipErrorInvalidValue);
  const long long nsb = (long long)(K / 256);
  constexpr int U = 4;
  const int g = grid_for((nsb + U - 1) / U);
  const bool w16 = aligned(W, 16), y16 = aligned(Y, 16);
  if (aligned(W, 4) && y16) {
    // LDS-staged chunks, two workgroups per CU (measured on config 2: 35.3 us
    // against 44.6 for dq_q4k_kernel; 1 per CU 36.3, 3-16 per CU 36.8-38.6,
    // each wave on chunks of its own 38.0)
    const long long nchunks = (nsb + kDqChunk - 1) / kDqChunk;
    const int gl = (int)std::max<long long>(1, std::min<long long>(nchunks, 2LL * cu_count()));
    dq_q4k_lds_kernel<<<gl, kThreads, 0, current_stream()>>>(W, Y, nsb);
    check_launch("dq_q4k_lds_kernel");
    return;
  }
  if (w16 && y16)
    dq_q4k_kernel<U, true, true><<<g, kThreads, 0, current_stream()>>>(W, Y, nsb);
  else if (y16)
    dq_q4k_kernel<U, false, true><<<g, kThreads, 0, current_stream()>>>(W, Y, nsb);
  else
    dq_q4k_kernel<U, false, false><<<g, kThreads, 0, current_stream()>>>(W, Y, nsb);
  check_launch("dq_q4k_kernel");
}

void row_dequantize_nvfp4(const uint8_t* W, const int8_t* codebook, const float* scale, float* Y,
                          size_t K) {
  using namespace weft;
  if (K == 0) return;
  if (K % 64 || bad(W, 1, Y) || codebook == nullptr || scale == nullptr || !aligned(scale, 4))
    return set_error(hipErrorInvalidValue);
  if (launch_dq_chunk<DqNv>(W, DqTab{codebook, scale}, Y, (long long)K)) return;
  const long long nb = (long long)(K / 64);
  const int g = grid_for((nb + 3) / 4);
  if (aligned(Y, 16))
    dq_nvfp4_kernel<true><<<g, kThreads, 0, current_stream()>>>(W, codebook, scale, Y, nb);
  else
    dq_nvfp4_kernel<false><<<g, kThreads, 0, current_stream()>>>(W, codebook, scale, Y, nb);
  check_launch("dq_nvfp4_kernel");
}

void row_dequantize_q5_k(const uint8_t* W, float* Y, size_t K) {
  using namespace weft;
  if (K == 0) return;
  if (K % 256 || bad(W, 2, Y)) return set_error(hipErrorInvalidValue);
  if (launch_dq_chunk<DqQ5K>(W, DqTab{nullptr, nullptr}, Y, (long long)K)) return;
  const long long nsb = (long long)(K / 256);
  constexpr int U = 4;
  const int g = grid_for((nsb + U - 1) / U);
  if (aligned(Y, 16))
    dq_q5k_kernel<U, true><<<g, kThreads, 0, current_stream()>>>(W, Y, nsb);
  else
    dq_q5k_kernel<U, false><<<g, kThreads, 0, current_stream()>>>(W, Y, nsb);
  check_launch("dq_q5k_kernel");
}

void row_dequantize_q6_k(const uint8_t* W, float* Y, size_t K) {
  using namespace weft;
  if (K == 0) return;
  if (K % 256 || bad(W, 1, Y)) return set_error(hipErrorInvalidValue);
  if (launch_dq_chunk<DqQ6K>(W, DqTab{nullptr, nullptr}, Y, (long long)K)) return;
  const long long nsb = (long long)(K / 256);
  constexpr int U = 4;
  const int g = grid_for((nsb + U - 1) / U);
  if (aligned(Y, 16))
    dq_q6k_kernel<U, true><<<g, kThreads, 0, current_stream()>>>(W, Y, nsb);
  else
    dq_q6k_kernel<U, false><<<g, kThreads, 0, current_stream()>>>(W, Y, nsb);
  check_launch("dq_q6k_kernel");
}

void row_dequantize_q4_0(const uint8_t* W, float* Y, size_t K) {
  using namespace weft;
  if (K == 0) return;
  if (K % 32 || bad(W, 2, Y)) return set_error(hipErrorInvalidValue);
  if (launch_dq_chunk<DqQ40>(W, DqTab{nullptr, nullptr}, Y, (long long)K)) return;
  const long long nb = (long long)(K / 32);
  const int g = grid_for((nb + 7) / 8);
  if (aligned(Y, 16))
    dq_32_kernel<false, true><<<g, kThreads, 0, current_stream()>>>(W, nullptr, nullptr, Y, nb);
  else
    dq_32_kernel<false, false><<<g, kThreads, 0, current_stream()>>>(W, nullptr, nullptr, Y, nb);
  check_launch("dq_32_kernel");
}

void row_dequantize_mxfp4(const uint8_t* W, const int8_t* codebook, const float* scale, float* Y,
                          size_t K) {
  using namespace weft;
  if (K == 0) return;
  if (K % 32 || bad(W, 1, Y) || codebook == nullptr || scale == nullptr || !aligned(scale, 4))
    return set_error(hipErrorInvalidValue);
  if (launch_dq_chunk<DqMx>(W, DqTab{codebook, scale}, Y, (long long)K)) return;
  const long long nb = (long long)(K / 32);
  const int g = grid_for((nb + 7) / 8);
  if (aligned(Y, 16))
    dq_32_kernel<true, true><<<g, kThreads, 0, current_stream()>>>(W, codebook, scale, Y, nb);
  else
    dq_32_kernel<true, false><<<g, kThreads, 0, current_stream()>>>(W, codebook, scale, Y, nb);
  check_launch("dq_32_kernel");
}

void row_dequantize_iq2_xxs(const uint8_t* W, const int8_t* grid, const int8_t* signs, float* Y,
                            size_t K) {
  using namespace weft;
  if (K == 0) return;
  if (K % 256 || bad(W, 2, Y) || grid == nullptr || signs == nullptr)
    return set_error(hipErrorInvalidValue);
  const long long nsb = (long long)(K / 256);
  if (aligned(Y, 16))
    dq_iq2xxs_kernel<true><<<grid_for(nsb), kThreads, 0, current_stream()>>>(W, grid, signs, Y, nsb);
  else
    dq_iq2xxs_kernel<false><<<grid_for(nsb), kThreads, 0, current_stream()>>>(W, grid, signs, Y, nsb);
  check_launch("dq_iq2xxs_kernel");
}

void row_dequantize_q4_1(const uint8_t* W, float* Y, size_t K) {
  using namespace weft;
  if (K == 0) return;
  if (K % 32 || bad(W, 2, Y)) return set_error(hipErrorInvalidValue);
  if (launch_dq_chunk<DqQ41>(W, DqTab{nullptr, nullptr}, Y, (long long)K)) return;
  const long long nb = (long long)(K / 32);
  const int g = grid_for((nb + 7) / 8);
  if (aligned(Y, 16))
    dq_q41_kernel<true><<<g, kThreads, 0, current_stream()>>>(W, Y, nb);
  else
    dq_q41_kernel<false><<<g, kThreads, 0, current_stream()>>>(W, Y, nb);
  check_launch("dq_q41_kernel");
}

void row_dequantize_iq2_xs(const uint8_t* W, const int8_t* grid, const int8_t* signs, float* Y,
                           size_t K) {
  using namespace weft;
  if (K == 0) return;
  if (K % 256 || bad(W, 2, Y) || grid == nullptr || signs == nullptr)
    return set_error(hipErrorInvalidValue);
  const long long nsb = (long long)(K / 256);
  if (aligned(Y, 16))
    dq_iq2xs_kernel<true><<<grid_for(nsb), kThreads, 0, current_stream()>>>(W, grid, signs, Y, nsb);
  else
    dq_iq2xs_kernel<false><<<grid_for(nsb), kThreads, 0, current_stream()>>>(W, grid, signs, Y, nsb);
  check_launch("dq_iq2xs_kernel");
}

}  // extern "C"
