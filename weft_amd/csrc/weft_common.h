// Device helpers shared by the libweft_hip kernels (gfx950 / CDNA4, wave64).
//
// Record layouts are GGML's block formats, byte for byte (vendored
// ggml-common.h of the reference: block_q4_0 :184-189, block_mxfp4 :204-209,
// block_q8_0 :241-246, block_q4_K :317-328, block_q8_K :361-366,
// block_iq2_xxs :371-375).  Kernels read them as raw little-endian bytes.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace weft {

constexpr int kWave = 64;

// Record geometry: elements per record, bytes per record.
constexpr int kQ4_0Elems = 32, kQ4_0Bytes = 18;
constexpr int kMxfp4Elems = 32, kMxfp4Bytes = 17;
constexpr int kQ8_0Elems = 32, kQ8_0Bytes = 34;
constexpr int kQ4_KElems = 256, kQ4_KBytes = 144;
constexpr int kQ8_KElems = 256, kQ8_KBytes = 292;
constexpr int kIq2xxsElems = 256, kIq2xxsBytes = 66;
constexpr int kQ6_KElems = 256, kQ6_KBytes = 210;  // ql[128] qh[64] scales[16] d
constexpr int kQ5_KElems = 256, kQ5_KBytes = 176;  // d dmin scales[12] qh[32] qs[128]
constexpr int kNvfp4Elems = 64, kNvfp4Bytes = 36;  // ue4m3 d[4] qs[32]
constexpr int kQ4_1Elems = 32, kQ4_1Bytes = 20;    // d m qs[16]
constexpr int kQ8_1Elems = 32, kQ8_1Bytes = 36;    // d s qs[32]
constexpr int kIq2xsElems = 256, kIq2xsBytes = 74; // d qs[32] (u16) scales[8]

// ---------------------------------------------------------------- numerics
// IEEE binary16 -> binary32 with v_cvt_f32_f16.  Exact for every input
// (zero, subnormal, normal, inf; NaN stays NaN): the kernels run with fp16
// denormals preserved (amdhsa_float_denorm_mode_16_64 = 3).
__device__ __forceinline__ float fp16_to_fp32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// fp32 -> two bf16 (round to nearest even) packed low | high << 16, and the
// low one back as fp32.  An outer-product factor dx * f is formed on a bf16
// MFMA from dx = h + m + l (bf16 parts, exact to 2^-24 relative) and an fp16
// f = f_h + f_l (exactly two bf16 parts): six exact products summed in fp32.
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
  const v2bf v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf16_lo_to_f32(uint32_t p) { return __uint_as_float(p << 16); }

// the token-side operand of that product: (h,h), (m,m), (l,l), 0 for d
__device__ __forceinline__ uint4 bf16_split3(float d) {
  const uint32_t ph = pk_bf16(d, d);
  const float r1 = d - bf16_lo_to_f32(ph);
  const uint32_t pm = pk_bf16(r1, r1);
  const float r2 = r1 - bf16_lo_to_f32(pm);
  return make_uint4(ph, pm, pk_bf16(r2, r2), 0u);
}

// the row-side operand: (f_h, f_l) for an fp16 value f, three times, then 0
__device__ __forceinline__ uint32_t bf16_split2(float f) {
  return pk_bf16(f, f - bf16_lo_to_f32(pk_bf16(f, f)));
}

// IEEE binary32 -> binary16, round to nearest even; NaN -> 0x7E00 (sign
// kept), as GGML's software conversion (ggml-impl.h:407-431).
__device__ __forceinline__ uint32_t fp32_to_fp16(float f) {
  const uint32_t x = __float_as_uint(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return sign | 0x7e00u;
  if (ax == 0x7f800000u) return sign | 0x7c00u;
  const int e = (int)(ax >> 23) - 112;
  uint32_t m = ax & 0x7fffffu;
  if (e >= 31) return sign | 0x7c00u;
  if (e <= 0) {
    if ((ax >> 23) == 0 && m == 0) return sign;
    m |= (ax >> 23) ? 0x800000u : 0u;
    const int shift = 14 - e;
    if (shift >= 32) return sign;
    const uint32_t res = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    return sign | (res + ((rem > half || (rem == half && (res & 1u))) ? 1u : 0u));
  }
  uint32_t r = ((uint32_t)e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1fffu;
  r += (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ? 1u : 0u;
  return sign | r;
}

// ------------------------------------------------------ DPP lane exchange
// gfx9 DPP controls used by the reductions below.
constexpr int kDppXor1 = 0xB1;          // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;          // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;   // lane i <-> 7-i inside 8
constexpr int kDppMirror = 0x140;       // lane i <-> 15-i inside 16
constexpr int kDppBcast15 = 0x142;      // lane 15 of a row -> next row
constexpr int kDppBcast31 = 0x143;      // lane 31 -> rows 2 and 3

template <int Ctrl, int RowMask = 0xF>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, Ctrl, RowMask, 0xF, false);
}
template <int Ctrl, int RowMask = 0xF>
__device__ __forceinline__ float dppf(float v) {
  return __int_as_float(dpp<Ctrl, RowMask>(__float_as_int(v)));
}

// Sum over aligned groups of 4 / 8 lanes, result in every lane of the group.
__device__ __forceinline__ int sum4(int v) {
  v += dpp<kDppXor1>(v);
  return v + dpp<kDppXor2>(v);
}
__device__ __forceinline__ int sum8_of_sum4(int v4) { return v4 + dpp<kDppHalfMirror>(v4); }

// Whole-wave sum / max (max of non-negative values), returned to all lanes.
__device__ __forceinline__ float wave_sum_f(float v) {
  v += dppf<kDppXor1>(v);
  v += dppf<kDppXor2>(v);
  v += dppf<kDppHalfMirror>(v);
  v += dppf<kDppMirror>(v);
  v += dppf<kDppBcast15, 0xA>(v);
  v += dppf<kDppBcast31, 0xC>(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_max_nonneg(float v) {
  v = fmaxf(v, dppf<kDppXor1>(v));
  v = fmaxf(v, dppf<kDppXor2>(v));
  v = fmaxf(v, dppf<kDppHalfMirror>(v));
  v = fmaxf(v, dppf<kDppMirror>(v));
  v = fmaxf(v, dppf<kDppBcast15, 0xA>(v));
  v = fmaxf(v, dppf<kDppBcast31, 0xC>(v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// ---------------------------------------------------------- unaligned loads
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) {
  return (uint32_t)(*reinterpret_cast<const uint16_t*>(p));
}
// 4 bytes at a 2-byte aligned address
__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t* p) {
  const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
  return (uint32_t)q[0] | ((uint32_t)q[1] << 16);
}
// 4 bytes at any address
__device__ __forceinline__ uint32_t ld_u32_a1(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// -------------------------------------------------------- wave reductions
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
// sum over aligned groups of G lanes (G a power of two <= 64)
template <int G, typename T>
__device__ __forceinline__ T group_sum(T v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
template <int G>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = G / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// int8 x int8 dot of 4 packed bytes, accumulated (v_dot4_i32_i8)
__device__ __forceinline__ int dot4(int a, int b, int c) {
  return __builtin_amdgcn_sdot4(a, b, c, false);
}

// Q4_K 6-bit scale and min of sub-block s (0..7) from the 12 scale bytes
// held as three little-endian words q0 = bytes 0-3, q1 = 4-7, q2 = 8-11
// (get_scale_min_k4, ggml-quants.c:822-829).
__device__ __forceinline__ void q4k_scale_min(int s, uint32_t q0, uint32_t q1, uint32_t q2,
                                              int& sc, int& m) {
  if (s < 4) {
    sc = (q0 >> (8 * s)) & 63;
    m = (q1 >> (8 * s)) & 63;
  } else {
    const int t = 8 * (s - 4);
    const uint32_t hi = (q2 >> t) & 0xffu;  // byte s+4
    sc = (hi & 0xF) | (((q0 >> t) >> 6 & 3) << 4);
    m = (hi >> 4) | (((q1 >> t) >> 6 & 3) << 4);
  }
}

// ------------------------------------------------- activation quantizers
// One Q8_K superblock (256 fp32) quantized by one wave: lane l holds
// x[4l .. 4l+3].  quantize_row_q8_K_ref, ggml-quants.c:2696-2733:
// the value at the first index of the largest |x| gives iscale = -127/max,
// q = min(127, rne(iscale * x)), d = 1/iscale; all-zero -> d = 0, q = 0,
// bsums not written (signalled by zero == true).
struct Q8KLane {
  int q[4];       // quantized values of this lane
  float d;        // block scale (wave-uniform)
  int bsum16;     // sum over this lane's 16-group (lanes 4g..4g+3), valid in every lane
  bool zero;      // all-zero block
};

__device__ __forceinline__ Q8KLane q8k_quantize_wave(float4 x, int lane) {
#pragma clang fp contract(off)
  // Straight-line code (no early exit for the all-zero block): a wave that
  // quantizes several superblocks runs their dependency chains interleaved.
  Q8KLane r;
  const float xv[4] = {x.x, x.y, x.z, x.w};
  const float amax = wave_max_nonneg(fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))));
  r.zero = !(amax > 0.f);
  // the signed value at the first index whose |x| is amax: first lane with
  // a match (ballot), then that lane's first match
  float first = 0.f;
  bool hit = false;
#pragma unroll
  for (int i = 3; i >= 0; --i) {
    if (fabsf(xv[i]) == amax) {
      first = xv[i];
      hit = true;
    }
  }
  const unsigned long long hits = __ballot(hit);
  const int src = hits ? __ffsll(hits) - 1 : 0;
  const float bval = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(first), src));
  // an all-zero block divides by a stand-in 1 and selects zeros below
  const float iscale = __fdiv_rn(-127.f, r.zero ? 1.f : bval);
  int s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float p = iscale * xv[i];
    const int v = (int)rintf(p);
    r.q[i] = r.zero ? 0 : (v < 127 ? v : 127);
    s += r.q[i];
  }
  r.bsum16 = sum4(s);
  const float d = __fdiv_rn(1.f, iscale);
  r.d = r.zero ? 0.f : d;
  return r;
}

// One Q8_K superblock quantized by 16 lanes (four superblocks per wave):
// lane part p = lane % 16 holds x[16p .. 16p+15], which is exactly bsum
// group p, so the block sums need no cross-lane step.  Same arithmetic as
// q8k_quantize_wave / quantize_row_q8_K_ref:
//   * amax over the superblock: 4-step DPP max inside the 16-lane row;
//   * the signed value at the first index with |x| == amax: each lane's
//     first match, then the lowest matching lane (DPP min of its part
//     index) and that lane's value (DPP sum of a one-hot value);
//   * q = nearest_int(iscale * x) with GGML's 1.5 * 2^23 bias, whose float
//     bits carry q in their low byte; GGML's MIN(127, q) never binds since
//     |iscale * x| <= 127 (1 + 2^-24)^2 < 127.5.
struct Q8K16 {
  uint32_t qs[4];  // this lane's 16 quantized values, packed little-endian
  float d;         // block scale (uniform in the 16 lanes)
  int bsum;        // sum of this lane's 16 values (GGML bsums[p])
  bool zero;       // all-zero block: d = 0, q = 0, bsums left untouched
};

template <int Ctrl>
__device__ __forceinline__ float dpp_row(float v) {  // DPP inside 16-lane rows
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xF, 0xF, false));
}
template <int Ctrl>
__device__ __forceinline__ int dpp_row_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, Ctrl, 0xF, 0xF, false);
}

__device__ __forceinline__ Q8K16 q8k_quantize_16lanes(const float4 (&x4)[4], int part) {
#pragma clang fp contract(off)
  float x[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[4 * i] = x4[i].x;
    x[4 * i + 1] = x4[i].y;
    x[4 * i + 2] = x4[i].z;
    x[4 * i + 3] = x4[i].w;
  }
  // reductions are written as trees: the dependent chain is what the
  // workgroup waits for
  float m8[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) m8[i] = fmaxf(fabsf(x[2 * i]), fabsf(x[2 * i + 1]));
#pragma unroll
  for (int i = 0; i < 4; ++i) m8[i] = fmaxf(m8[2 * i], m8[2 * i + 1]);
  float am = fmaxf(fmaxf(m8[0], m8[1]), fmaxf(m8[2], m8[3]));
  am = fmaxf(am, dpp_row<kDppXor1>(am));
  am = fmaxf(am, dpp_row<kDppXor2>(am));
  am = fmaxf(am, dpp_row<kDppHalfMirror>(am));
  am = fmaxf(am, dpp_row<kDppMirror>(am));
  Q8K16 r;
  r.zero = !(am > 0.f);
  // this lane's first match: a tree over pairs, the lower index winning
  float fv[16];
  bool fh[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    fv[i] = x[i];
    fh[i] = fabsf(x[i]) == am;
  }
#pragma unroll
  for (int w = 1; w < 16; w *= 2) {
#pragma unroll
    for (int i = 0; i < 16; i += 2 * w) {
      fv[i] = fh[i] ? fv[i] : fv[i + w];
      fh[i] = fh[i] || fh[i + w];
    }
  }
  const float first = fv[0];
  const bool hit = fh[0];
  int key = hit ? part : 16;
  key = min(key, dpp_row_i<kDppXor1>(key));
  key = min(key, dpp_row_i<kDppXor2>(key));
  key = min(key, dpp_row_i<kDppHalfMirror>(key));
  key = min(key, dpp_row_i<kDppMirror>(key));
  float bv = part == key ? first : 0.f;  // one lane holds the value, the rest +0
  bv += dpp_row<kDppXor1>(bv);
  bv += dpp_row<kDppXor2>(bv);
  bv += dpp_row<kDppHalfMirror>(bv);
  bv += dpp_row<kDppMirror>(bv);
  const float iscale = __fdiv_rn(-127.f, r.zero ? 1.f : bv);
  uint32_t b[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float p = iscale * x[i];
    b[i] = __float_as_uint(p + 12582912.f);  // 0x4B400000 + q
  }
  // modulo 2^32 the sixteen biases cancel exactly
  uint32_t t4[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) t4[i] = (b[4 * i] + b[4 * i + 1]) + (b[4 * i + 2] + b[4 * i + 3]);
  const uint32_t sum = (t4[0] + t4[1]) + (t4[2] + t4[3]) - 16u * 0x4B400000u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // low bytes of four biased floats -> one packed word
    const uint32_t lo = __builtin_amdgcn_perm(b[4 * i + 1], b[4 * i], 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(b[4 * i + 3], b[4 * i + 2], 0x04000c0cu);
    r.qs[i] = r.zero ? 0u : (lo | hi);
  }
  r.bsum = r.zero ? 0 : (int)sum;
  r.d = r.zero ? 0.f : __fdiv_rn(1.f, iscale);
  return r;
}

// One Q8_0 block (32 fp32) quantized by 8 lanes, lane holds 4 values.
// quantize_row_q8_0_ref, ggml-quants.c:238-261: d = amax/127,
// q = roundf(x * (1/d)) (half away from zero), fp16(d) stored.
struct Q8_0Lane {
  int q[4];
  float d;        // fp32 d (before fp16 rounding)
  uint32_t dh;    // fp16 bits of d
};

__device__ __forceinline__ Q8_0Lane q80_quantize_8lanes(float4 x) {
#pragma clang fp contract(off)
  Q8_0Lane r;
  float amax = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
  amax = group_max<8>(amax);
  const float d = __fdiv_rn(amax, 127.f);
  const float id = d != 0.f ? __fdiv_rn(1.f, d) : 0.f;
  const float xv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) r.q[i] = (int)roundf(xv[i] * id);
  r.d = d;
  r.dh = fp32_to_fp16(d);
  return r;
}

// Q8_1's block sum term (quantize_row_q8_1_ref, ggml-quants.c:264-295):
// s = fp16(sum(q) * d) with the fp32 d, over the 8 lanes of a block (every
// lane of the wave calls this)
__device__ __forceinline__ uint32_t q81_sum_half(const Q8_0Lane& r) {
  int t = r.q[0] + r.q[1] + r.q[2] + r.q[3];
  t += __shfl_xor(t, 1, kWave);
  t += __shfl_xor(t, 2, kWave);
  t += __shfl_xor(t, 4, kWave);
  return fp32_to_fp16((float)t * r.d);
}

// ggml_e8m0_to_fp32_half (ggml-impl.h:477-495): 2^(e-128), e < 2 as fp32
// subnormals
__device__ __forceinline__ float e8m0_half(uint32_t e) {
  return __uint_as_float(e < 2 ? 0x00200000u << e : (e - 1) << 23);
}

// One MXFP4 x Q8_0 block term added in GGML's order and rounding
// (ggml-cpu/quants.c:265-273): d = fp16(dx) * ws, then acc + d * I, each
// step rounded (so an overflow to inf, and inf * 0 = NaN, happen where
// GGML's do).
__device__ __forceinline__ float ggml_scaled_term(float acc, float dx, float ws, float i) {
#pragma clang fp contract(off)
  const float d = dx * ws;
  const float t = d * i;
  return acc + t;
}

// IQ2 lookup tables (IQ2_XXS / IQ2_XS grid and sign rows, I8X8).  The
// reference multiplies a grid byte by its sign byte as i8 x i8 -> i8
// (examples/kernels/vec_dot/iq2_xxs_q8_k.py:39, functions/quantization.py:77:
// equal element types are not promoted, python/weft/frontend/compiler.py:
// 1276-1292), so the product wraps modulo 256.  The fast kernels take signs
// as byte masks and negate with (g ^ 0xff) + 1, which is that product
// exactly when every sign byte is +1 or -1 and no grid byte is 0 (a 0 byte
// would carry into its neighbour); GGML's tables (magnitudes 8, 25, 43 and
// +-1 signs) meet it.  Other tables take the byte product below.
__device__ __forceinline__ bool iq2_grid_word_ok(uint32_t g) {
  return ((g - 0x01010101u) & ~g & 0x80808080u) == 0u;  // no zero byte
}
__device__ __forceinline__ bool iq2_sign_word_ok(uint32_t s) {
  const uint32_t m = ((s >> 7) & 0x01010101u) * 0xffu;
  return s == (m | 0x01010101u);  // every byte 0x01 or 0xff
}
// Workgroup-wide "any bad table word" without a reducing barrier: before a
// barrier every wave stores whether any of its lanes saw one (flags: one
// word per wave of the workgroup, in LDS); after it, every lane ORs them.
__device__ __forceinline__ void iq2_flag_wave(uint32_t* flags, bool bad) {
  const bool any = __builtin_amdgcn_ballot_w64(bad) != 0;
  if ((threadIdx.x & 63) == 0) flags[threadIdx.x >> 6] = any ? 1u : 0u;
}
__device__ __forceinline__ bool iq2_flags_clear(const uint32_t* flags, int nwaves) {
  uint32_t any = 0;
  for (int w = 0; w < nwaves; ++w) any |= flags[w];
  return __builtin_amdgcn_readfirstlane(any) == 0;  // wave-uniform: scalar branches
}

// four i8 x i8 -> i8 products, byte by byte, modulo 256
__device__ __forceinline__ uint32_t mul8x4(uint32_t g, uint32_t s) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  const u16x2 lo = __builtin_bit_cast(u16x2, g & 0x00ff00ffu) * __builtin_bit_cast(u16x2, s & 0x00ff00ffu);
  const u16x2 hi =
      __builtin_bit_cast(u16x2, (g >> 8) & 0x00ff00ffu) * __builtin_bit_cast(u16x2, (s >> 8) & 0x00ff00ffu);
  // bytes 0 and 2 of each product: lo.b0, hi.b0, lo.b2, hi.b2
  return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, hi), __builtin_bit_cast(uint32_t, lo), 0x06020400u);
}

__device__ __forceinline__ int pack4_i8(const int q[4]) {
  return (int)((uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
               ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24));
}

}  // namespace weft
