// Standalone activation quantizers q8_0_quantize, q8_K_quantize and
// q8_1_quantize (examples/kernels/quantize/q8_0.py:26-28, q8_k.py:38-40,
// q8_1.py:28-30), bit-exact with GGML's quantize_row_q8_0_ref /
// quantize_row_q8_K_ref / quantize_row_q8_1_ref (ggml-quants.c:238-261,
// :2696-2733, :264-295).
//
// HBM-bound (read 4 B, write ~1.1 B per element).  Q8_K: 16 lanes per
// superblock, lane p owns x[16p..16p+15] (four 16-byte loads), so the
// 16-sums are in-lane and the first-index |max| is a 16-lane reduction.
// Q8_0: 8 lanes per block, 8 blocks per wave step.  The grid is sized to a
// few waves per CU and strides over the blocks.
//
// The row forms (quantize_q8_k_rows / quantize_q8_0_rows) take M rows of K
// values ldx floats apart, as GGML's MUL_MAT quantizes a strided src1 into
// its contiguous work buffer (ggml-cpu/ggml-cpu.c:1309-1340).
#include <algorithm>

#include "kernels.h"
#include "runtime.h"
#include "weft_common.h"
#include "weft_hip.h"

namespace weft {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float4 ldx4(const float* p, bool a16) {
  if (a16) return *reinterpret_cast<const float4*>(p);
  return make_float4(p[0], p[1], p[2], p[3]);
}

// Source of record b: flat (record-contiguous X) or row r = b / nbr of a
// strided matrix.
struct XRows {
  long long nbr;  // records per row; 0 = flat
  long long ldx;  // floats between rows
  __device__ __forceinline__ const float* at(const float* X, long long b, int elems) const {
    if (nbr == 0) return X + b * elems;
    const long long r = b / nbr;
    return X + r * ldx + (b - r * nbr) * elems;
  }
};

// 16 lanes per superblock (q8k_quantize_16lanes): lane part p holds bsum
// group p, a wave quantizes four superblocks per pass.  The grid gives each
// wave one pass (two waves per SIMD for a prefill-sized activation): with a
// single wave per SIMD the quantization arithmetic issues at half the rate.
__global__ void __launch_bounds__(kThreads) q8k_quantize_kernel(const float* __restrict__ X,
                                                                uint8_t* __restrict__ Y, long long nb,
                                                                XRows xr, bool a16) {
  constexpr int U = 1;  // passes in flight per wave
  const int lane = threadIdx.x & (kWave - 1);
  const int part = lane & 15;
  const long long wave = ((long long)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const long long nwaves = (long long)gridDim.x * blockDim.x / kWave;
  for (long long p0 = wave * U; 4 * p0 < nb; p0 += nwaves * U) {
    float4 x[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long b = min(4 * (p0 + u) + lane / 16, nb - 1);  // clamped: a valid load
      const float* src = xr.at(X, b, 256) + 16 * part;
#pragma unroll
      for (int j = 0; j < 4; ++j) x[u][j] = ldx4(src + 4 * j, a16);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long b = 4 * (p0 + u) + lane / 16;
      const Q8K16 r = q8k_quantize_16lanes(x[u], part);
      if (b < nb) {
        uint8_t* rec = Y + b * kQ8_KBytes;
        if (part == 0) *reinterpret_cast<float*>(rec) = r.d;
        uint32_t* q = reinterpret_cast<uint32_t*>(rec + 4 + 16 * part);
        q[0] = r.qs[0];
        q[1] = r.qs[1];
        q[2] = r.qs[2];
        q[3] = r.qs[3];
        if (!r.zero) reinterpret_cast<int16_t*>(rec + 260)[part] = (int16_t)r.bsum;
      }
    }
  }
}

__global__ void __launch_bounds__(kThreads) q80_quantize_kernel(const float* __restrict__ X,
                                                                uint8_t* __restrict__ Y, long long nb,
                                                                XRows xr, bool a16) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long wave = ((long long)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const long long nwaves = (long long)gridDim.x * blockDim.x / kWave;
  const long long steps = (nb + 7) / 8;
  for (long long st = wave; st < steps; st += nwaves) {
    const long long b = 8 * st + lane / 8;
    const bool live = b < nb;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) x = ldx4(xr.at(X, b, 32) + 4 * (lane & 7), a16);
    const Q8_0Lane r = q80_quantize_8lanes(x);
    if (!live) continue;
    uint8_t* rec = Y + b * kQ8_0Bytes;
    const uint32_t packed = (uint32_t)pack4_i8(r.q);
    uint16_t* q16 = reinterpret_cast<uint16_t*>(rec + 2 + 4 * (lane & 7));
    q16[0] = (uint16_t)(packed & 0xffffu);
    q16[1] = (uint16_t)(packed >> 16);
    if ((lane & 7) == 0) *reinterpret_cast<uint16_t*>(rec) = (uint16_t)r.dh;
  }
}

// Q8_1: Q8_0's lanes plus the block's s; the 36-byte records are 2-byte
// aligned, so the codes go out as halfwords
__global__ void __launch_bounds__(kThreads) q81_quantize_kernel(const float* __restrict__ X,
                                                                uint8_t* __restrict__ Y, long long nb,
                                                                XRows xr, bool a16) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long wave = ((long long)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const long long nwaves = (long long)gridDim.x * blockDim.x / kWave;
  const long long steps = (nb + 7) / 8;
  for (long long st = wave; st < steps; st += nwaves) {
    const long long b = 8 * st + lane / 8;
    const bool live = b < nb;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) x = ldx4(xr.at(X, b, 32) + 4 * (lane & 7), a16);
    const Q8_0Lane r = q80_quantize_8lanes(x);
    const uint32_t sh = q81_sum_half(r);
    if (!live) continue;
    uint8_t* rec = Y + b * kQ8_1Bytes;
    const uint32_t packed = (uint32_t)pack4_i8(r.q);
    uint16_t* q16 = reinterpret_cast<uint16_t*>(rec + 4 + 4 * (lane & 7));
    q16[0] = (uint16_t)(packed & 0xffffu);
    q16[1] = (uint16_t)(packed >> 16);
    if ((lane & 7) == 0) {
      reinterpret_cast<uint16_t*>(rec)[0] = (uint16_t)r.dh;
      reinterpret_cast<uint16_t*>(rec)[1] = (uint16_t)sh;
    }
  }
}

int grid_for(long long waves_needed) {
  const long long per_block = kThreads / kWave;
  const long long cap = (long long)cu_count() * 8;  // 8 workgroups (32 waves) per CU
  return (int)std::max<long long>(1, std::min<long long>(cap, (waves_needed + per_block - 1) / per_block));
}

}  // namespace

void quantize_q8_k_rows(const float* X, size_t ldx, uint8_t* Y, size_t M, size_t K) {
  if (K == 0 || M == 0) return;
  if (K % 256 || X == nullptr || Y == nullptr || !aligned(X, 4) || !aligned(Y, 4) ||
      (M > 1 && ldx < K))
    return set_error(hipErrorInvalidValue);
  const bool flat = M == 1 || ldx == K;
  const long long nb = (long long)(M * (K / 256));
  const XRows xr{flat ? 0 : (long long)(K / 256), (long long)ldx};
  const bool a16 = aligned(X, 16) && (flat || ldx % 4 == 0);
  // one pass (four superblocks) per wave, four waves per workgroup
  const long long blocks = std::max<long long>(1, (nb + 15) / 16);
  q8k_quantize_kernel<<<(int)std::min<long long>(blocks, INT32_MAX), kThreads, 0, current_stream()>>>(
      X, Y, nb, xr, a16);
  check_launch("q8k_quantize_kernel");
}

void quantize_q8_0_rows(const float* X, size_t ldx, uint8_t* Y, size_t M, size_t K) {
  if (K == 0 || M == 0) return;
  if (K % 32 || X == nullptr || Y == nullptr || !aligned(X, 4) || !aligned(Y, 2) ||
      (M > 1 && ldx < K))
    return set_error(hipErrorInvalidValue);
  const bool flat = M == 1 || ldx == K;
  const long long nb = (long long)(M * (K / 32));
  const XRows xr{flat ? 0 : (long long)(K / 32), (long long)ldx};
  const bool a16 = aligned(X, 16) && (flat || ldx % 4 == 0);
  q80_quantize_kernel<<<grid_for((nb + 7) / 8), kThreads, 0, current_stream()>>>(X, Y, nb, xr, a16);
  check_launch("q80_quantize_kernel");
}

void quantize_q8_1_rows(const float* X, size_t ldx, uint8_t* Y, size_t M, size_t K) {
  if (K == 0 || M == 0) return;
  if (K % 32 || X == nullptr || Y == nullptr || !aligned(X, 4) || !aligned(Y, 2) ||
      (M > 1 && ldx < K))
    return set_error(hipErrorInvalidValue);
  const bool flat = M == 1 || ldx == K;
  const long long nb = (long long)(M * (K / 32));
  const XRows xr{flat ? 0 : (long long)(K / 32), (long long)ldx};
  const bool a16 = aligned(X, 16) && (flat || ldx % 4 == 0);
  q81_quantize_kernel<<<grid_for((nb + 7) / 8), kThreads, 0, current_stream()>>>(X, Y, nb, xr, a16);
  check_launch("q81_quantize_kernel");
}

void quantize_q8_k(const float* X, uint8_t* Y, size_t K) { quantize_q8_k_rows(X, K, Y, 1, K); }

void quantize_q8_0(const float* X, uint8_t* Y, size_t K) { quantize_q8_0_rows(X, K, Y, 1, K); }

}  // namespace weft

extern "C" {

void q8_0_quantize(const float* X, uint8_t* Y, size_t K) { weft::quantize_q8_0(X, Y, K); }

void q8_K_quantize(const float* X, uint8_t* Y, size_t K) { weft::quantize_q8_k(X, Y, K); }

void q8_1_quantize(const float* X, uint8_t* Y, size_t K) { weft::quantize_q8_1_rows(X, K, Y, 1, K); }

}  // extern "C"
