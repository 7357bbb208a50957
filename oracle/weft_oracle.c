/*
 * CPU oracle for the quantized mul_mat hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates, function by function, the GGML CPU code that Weft's repro
 * harnesses call as their oracle.  Every function cites the vendored GGML
 * file:line it follows (paths relative to
 * /root/reference/source/c/ggml/llama.cpp/ggml/src/).  Built with
 * -ffp-contract=off so that every product is rounded to fp32 before it is
 * added, as the scalar C semantics of those functions state.
 *
 * Pinning (see tests/test_oracle.py):
 *   fp16 / e8m0 conversions .... numpy float16 and ldexp (library routines)
 *   tables ...................... fixtures parsed from ggml-common.h text
 *   dequantizers ................ closed-form per-element brute force
 *   Q8 quantizers ............... known-answer edge cases + invariants
 *   vec_dots / mul_mat .......... fp64 re-accumulation through an independent
 *                                 numpy dequantize-then-dot path
 *   weight quantizers ........... round-trip error bounds (input generators;
 *                                 the IQ2_XXS one is NOT GGML's algorithm:
 *                                 parity unpinned, see its comment)
 */
#include "weft_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK4_0 32
#define QK8_0 32
#define QK_MXFP4 32
#define QK_K 256

#define Q4_0_BYTES 18
#define Q8_0_BYTES 34
#define MXFP4_BYTES 17
#define Q4_K_BYTES 144
#define Q8_K_BYTES 292
#define IQ2_XXS_BYTES 66
#define Q6_K_BYTES 210
#define Q5_K_BYTES 176
#define QK_NVFP4 64
#define NVFP4_BYTES 36
#define Q4_1_BYTES 20
#define Q8_1_BYTES 36
#define IQ2_XS_BYTES 74
#define GROUP_MAX_EPS 1e-15f

static inline uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t *p, uint16_t v) {
  p[0] = (uint8_t)v;
  p[1] = (uint8_t)(v >> 8);
}
static inline uint32_t rd32(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline float rdf32(const uint8_t *p) { return bits_f32(rd32(p)); }
static inline void wrf32(uint8_t *p, float f) {
  uint32_t u = f32_bits(f);
  p[0] = (uint8_t)u;
  p[1] = (uint8_t)(u >> 8);
  p[2] = (uint8_t)(u >> 16);
  p[3] = (uint8_t)(u >> 24);
}

/* ------------------------------------------------------------------------
 * IEEE binary16 <-> binary32.  GGML's ggml_compute_fp16_to_fp32 /
 * ggml_compute_fp32_to_fp16 (ggml-impl.h:384-431) compute the exact widening
 * and round-to-nearest-even narrowing (NaN -> 0x7E00 with the sign kept).
 * Written here from the IEEE 754 definition with integer arithmetic.
 * ---------------------------------------------------------------------- */
float wo_fp16_to_fp32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24, exact in fp32 */
    const float v = (float)man * 0x1p-24f;
    return bits_f32(sign | f32_bits(v));
  }
  if (exp == 31) return bits_f32(sign | 0x7f800000u | (man << 13));
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t wo_fp32_to_fp16(float f) {
  const uint32_t x = f32_bits(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return sign | 0x7e00u; /* NaN */
  if (ax == 0x7f800000u) return sign | 0x7c00u;
  const int e = (int)(ax >> 23) - 127 + 15; /* biased fp16 exponent */
  uint32_t m = ax & 0x7fffffu;
  if (e >= 31) return sign | 0x7c00u; /* overflow, may be un-rounded below */
  if (e <= 0) {
    /* subnormal fp16 (or zero): value = m' * 2^(e-1-23+... ) */
    if ((ax >> 23) == 0 && m == 0) return sign;
    m |= ((ax >> 23) ? 0x800000u : 0u);
    const int shift = 14 - e; /* 13 mantissa bits dropped + (1 - e) */
    if (shift >= 32) return sign;
    const uint32_t res = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    uint32_t r = res;
    if (rem > half || (rem == half && (res & 1u))) r += 1;
    return sign | (uint16_t)r;
  }
  uint32_t r = ((uint32_t)e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r += 1; /* may carry to inf */
  return sign | (uint16_t)r;
}

/* ggml_e8m0_to_fp32_half, ggml-impl.h:477-495: 2^(e-128); e<2 are fp32
 * subnormals. */
float wo_e8m0_to_fp32_half(uint8_t e) {
  const uint32_t bits = e < 2 ? (0x00200000u << e) : ((uint32_t)(e - 1) << 23);
  return bits_f32(bits);
}

void wo_fp16_to_fp32_array(const uint16_t *h, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = wo_fp16_to_fp32(h[i]);
}
void wo_fp32_to_fp16_array(const float *f, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = wo_fp32_to_fp16(f[i]);
}

/* ------------------------------------------------------------------------
 * Tables.
 * iq2xxs_grid (ggml-common.h:550-615) is the 256 entries of
 * kgrid_2bit_256 (ggml-quants.c:2787-2804) expanded lane by lane, two bits
 * per lane, through {0 -> 0x08, 1 -> 0x19, 2 -> 0x2b}.
 * ksigns_iq2xs (ggml-common.h:503-512) is i | parity(i) << 7, so each 8-wide
 * sign pattern has an even number of minus signs.
 * ---------------------------------------------------------------------- */
static const uint16_t kIq2xxsCodes[256] = {
    0,     2,     5,     8,     10,    17,    20,    32,    34,    40,    42,    65,    68,    80,    88,    97,
    100,   128,   130,   138,   162,   257,   260,   272,   277,   320,   388,   408,   512,   514,   546,   642,
    1025,  1028,  1040,  1057,  1060,  1088,  1090,  1096,  1120,  1153,  1156,  1168,  1188,  1280,  1282,  1288,
    1312,  1350,  1385,  1408,  1425,  1545,  1552,  1600,  1668,  1700,  2048,  2053,  2056,  2068,  2088,  2113,
    2116,  2128,  2130,  2184,  2308,  2368,  2562,  2580,  4097,  4100,  4112,  4129,  4160,  4192,  4228,  4240,
    4245,  4352,  4360,  4384,  4432,  4442,  4480,  4644,  4677,  5120,  5128,  5152,  5157,  5193,  5248,  5400,
    5474,  5632,  5654,  6145,  6148,  6160,  6208,  6273,  6400,  6405,  6560,  6737,  8192,  8194,  8202,  8260,
    8289,  8320,  8322,  8489,  8520,  8704,  8706,  9217,  9220,  9232,  9280,  9302,  9472,  9537,  9572,  9872,
    10248, 10272, 10388, 10820, 16385, 16388, 16400, 16408, 16417, 16420, 16448, 16456, 16470, 16480, 16513, 16516,
    16528, 16640, 16672, 16737, 16768, 16773, 16897, 16912, 16968, 16982, 17000, 17408, 17416, 17440, 17536, 17561,
    17682, 17700, 17920, 18433, 18436, 18448, 18496, 18501, 18688, 18776, 18785, 18818, 19013, 19088, 20480, 20488,
    20497, 20505, 20512, 20608, 20616, 20740, 20802, 20900, 21137, 21648, 21650, 21770, 22017, 22100, 22528, 22545,
    22553, 22628, 22848, 23048, 24580, 24592, 24640, 24680, 24832, 24917, 25112, 25184, 25600, 25605, 25872, 25874,
    25988, 26690, 32768, 32770, 32778, 32833, 32898, 33028, 33048, 33088, 33297, 33793, 33796, 33808, 33813, 33856,
    33888, 34048, 34118, 34196, 34313, 34368, 34400, 34818, 35076, 35345, 36868, 36880, 36900, 36928, 37025, 37142,
    37248, 37445, 37888, 37922, 37956, 38225, 39041, 39200, 40962, 41040, 41093, 41225, 41472, 42008, 43088, 43268,
};

void wo_iq2xxs_grid(uint8_t out[2048]) {
  static const uint8_t lane_value[4] = {0x08, 0x19, 0x2b, 0x00};
  for (int i = 0; i < 256; ++i)
    for (int j = 0; j < 8; ++j) out[8 * i + j] = lane_value[(kIq2xxsCodes[i] >> (2 * j)) & 3];
}

/* iq2xs_grid (ggml-common.h:617-746): 512 entries of 8 magnitudes in
 * {0x08, 0x19, 0x2b}, here as two bits per lane (0, 1, 2), lane 0 in the low
 * bits; the codes ascend with the table index. */
static const uint16_t kIq2xsCodes[512] = {
        0,     2,     5,     8,    10,    17,    20,    22,    25,    32,    34,    37,    40,    65,    68,    70,
       73,    80,    82,    85,    88,    97,   100,   128,   130,   133,   136,   145,   148,   153,   160,   257,
      260,   262,   265,   272,   274,   277,   280,   282,   289,   292,   320,   322,   325,   328,   337,   340,
      352,   360,   385,   388,   400,   512,   514,   517,   520,   529,   532,   544,   577,   580,   592,   597,
      640,   650,  1025,  1028,  1030,  1033,  1040,  1042,  1045,  1048,  1057,  1060,  1088,  1090,  1093,  1096,
     1105,  1108,  1110,  1120,  1153,  1156,  1168,  1280,  1282,  1285,  1288,  1297,  1300,  1312,  1345,  1348,
     1360,  1377,  1408,  1537,  1540,  1552,  1574,  1600,  1602,  1668,  2048,  2050,  2053,  2056,  2058,  2065,
     2068,  2080,  2085,  2113,  2116,  2128,  2136,  2176,  2208,  2218,  2305,  2308,  2320,  2368,  2433,  2441,
     2560,  2592,  2600,  2710,  2720,  4097,  4100,  4102,  4105,  4112,  4114,  4117,  4120,  4129,  4132,  4160,
     4162,  4165,  4168,  4177,  4180,  4192,  4202,  4225,  4228,  4240,  4352,  4354,  4357,  4360,  4369,  4372,
     4384,  4417,  4420,  4432,  4480,  4500,  4502,  4609,  4612,  4614,  4624,  4672,  4704,  5120,  5122,  5125,
     5128,  5137,  5140,  5152,  5185,  5188,  5193,  5200,  5220,  5248,  5377,  5380,  5392,  5440,  5632,  5652,
     5705,  6145,  6148,  6160,  6162,  6208,  6228,  6278,  6400,  6405,  6502,  6737,  6825,  8192,  8194,  8197,
     8200,  8202,  8209,  8212,  8224,  8257,  8260,  8272,  8320,  8352,  8449,  8452,  8464,  8512,  8520,  8549,
     8704,  8738,  8832,  8872,  9217,  9220,  9232,  9257,  9280,  9472,  9537,  9554,  9625,  9729,  9754,  9894,
    10240, 10248, 10250, 10272, 10325, 10376, 10402, 10600, 10640, 10760, 10784, 10882, 10888, 10890, 16385, 16388,
    16390, 16393, 16400, 16402, 16405, 16408, 16417, 16420, 16448, 16450, 16453, 16456, 16458, 16465, 16468, 16480,
    16485, 16513, 16516, 16528, 16640, 16642, 16645, 16648, 16657, 16660, 16672, 16705, 16708, 16720, 16768, 16773,
    16802, 16897, 16900, 16912, 16914, 16937, 16960, 17408, 17410, 17413, 17416, 17425, 17428, 17433, 17440, 17473,
    17476, 17488, 17536, 17556, 17665, 17668, 17680, 17700, 17728, 17818, 17920, 17930, 17988, 18000, 18433, 18436,
    18448, 18496, 18501, 18516, 18530, 18688, 18705, 18756, 18768, 18793, 18948, 20480, 20482, 20485, 20488, 20497,
    20500, 20512, 20520, 20545, 20548, 20560, 20608, 20737, 20740, 20752, 20757, 20800, 20802, 20992, 21060, 21162,
    21505, 21508, 21520, 21537, 21568, 21600, 21633, 21665, 21760, 21768, 21888, 21896, 22049, 22120, 22177, 22528,
    22548, 22593, 22608, 22681, 22810, 22848, 22850, 23173, 24577, 24580, 24592, 24640, 24660, 24674, 24710, 24745,
    24832, 25124, 25162, 25234, 25600, 25622, 25872, 25920, 25925, 26020, 26625, 26730, 26917, 27142, 27220, 27234,
    32768, 32770, 32773, 32776, 32785, 32788, 32800, 32810, 32833, 32836, 32848, 32896, 32898, 32936, 32938, 33025,
    33028, 33030, 33040, 33088, 33105, 33113, 33280, 33312, 33408, 33410, 33440, 33448, 33793, 33796, 33808, 33810,
    33813, 33856, 33888, 33929, 34048, 34116, 34213, 34328, 34410, 34816, 34824, 34853, 34906, 34944, 34946, 34984,
    35078, 35362, 35456, 35464, 35478, 35496, 36865, 36868, 36880, 36928, 36950, 36996, 37120, 37154, 37220, 37462,
    37513, 37888, 37893, 37956, 37968, 37976, 38185, 38288, 38290, 38465, 38993, 39078, 39241, 39445, 39520, 40960,
    40962, 40968, 40970, 40992, 41002, 41120, 41297, 41305, 41382, 41472, 41474, 41480, 41514, 41600, 41632, 42048,
    42133, 42597, 42648, 43018, 43040, 43042, 43048, 43168, 43176, 43268, 43396, 43398, 43560, 43562, 43665, 43690,
};

void wo_iq2xs_grid(uint8_t out[4096]) {
  static const uint8_t lane_value[4] = {0x08, 0x19, 0x2b, 0x00};
  for (int i = 0; i < 512; ++i)
    for (int j = 0; j < 8; ++j) out[8 * i + j] = lane_value[(kIq2xsCodes[i] >> (2 * j)) & 3];
}

void wo_ksigns_iq2xs(uint8_t out[128]) {
  for (int i = 0; i < 128; ++i) out[i] = (uint8_t)(i | ((__builtin_popcount(i) & 1) << 7));
}

void wo_signs_i8x8(int8_t out[1024]) {
  uint8_t ks[128];
  wo_ksigns_iq2xs(ks);
  for (int i = 0; i < 128; ++i)
    for (int j = 0; j < 8; ++j) out[8 * i + j] = (ks[i] >> j) & 1 ? -1 : 1;
}

/* kvalues_mxfp4 (ggml-common.h:1116-1118): twice the E2M1 values. */
void wo_kvalues_mxfp4(int8_t out[16]) {
  static const float e2m1[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
  for (int i = 0; i < 16; ++i) out[i] = (int8_t)((i & 8 ? -2.f : 2.f) * e2m1[i & 7]);
}

void wo_e8m0_half_table(float out[256]) {
  for (int e = 0; e < 256; ++e) out[e] = wo_e8m0_to_fp32_half((uint8_t)e);
}

/* nearest_int, ggml-quants.c:563-568: round half to even of a value that
 * has already been rounded to fp32 (|v| <= 2^22). */
static inline int nearest_int(float v) {
  const float biased = v + 12582912.f;
  return (int)(f32_bits(biased) & 0x007fffffu) - 0x00400000;
}

/* get_scale_min_k4, ggml-quants.c:822-829 */
static inline void scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* ------------------------------------------------------------------------
 * Weight quantizers (input generators)
 * ---------------------------------------------------------------------- */

/* quantize_row_q4_0_ref, ggml-quants.c:75-110 */
void wo_quantize_row_q4_0(const float *x, uint8_t *y, int64_t k) {
  const int64_t nb = k / QK4_0;
  for (int64_t i = 0; i < nb; ++i) {
    const float *xb = x + i * QK4_0;
    uint8_t *rec = y + i * Q4_0_BYTES;
    float amax = 0.f, max = 0.f;
    for (int j = 0; j < QK4_0; ++j) {
      if (amax < fabsf(xb[j])) {
        amax = fabsf(xb[j]);
        max = xb[j];
      }
    }
    const float d = max / -8;
    const float id = d ? 1.0f / d : 0.0f;
    wr16(rec, wo_fp32_to_fp16(d));
    for (int j = 0; j < QK4_0 / 2; ++j) {
      const float x0 = xb[j] * id;
      const float x1 = xb[QK4_0 / 2 + j] * id;
      int8_t t0 = (int8_t)(x0 + 8.5f);
      int8_t t1 = (int8_t)(x1 + 8.5f);
      const uint8_t q0 = (uint8_t)(t0 < 15 ? t0 : 15);
      const uint8_t q1 = (uint8_t)(t1 < 15 ? t1 : 15);
      rec[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
  }
}

/* best_index_mxfp4 / quantize_row_mxfp4_ref, ggml-quants.c:299-344 */
void wo_quantize_row_mxfp4(const float *x, uint8_t *y, int64_t k) {
  int8_t kv[16];
  wo_kvalues_mxfp4(kv);
  const int64_t nb = k / QK_MXFP4;
  for (int64_t i = 0; i < nb; ++i) {
    const float *xb = x + i * QK_MXFP4;
    uint8_t *rec = y + i * MXFP4_BYTES;
    float amax = 0.f;
    for (int j = 0; j < QK_MXFP4; ++j)
      if (amax < fabsf(xb[j])) amax = fabsf(xb[j]);
    const uint8_t e = amax > 0.0f ? (uint8_t)(floorf(log2f(amax)) - 2 + 127) : 0;
    const float d = wo_e8m0_to_fp32_half(e);
    rec[0] = e;
    for (int j = 0; j < QK_MXFP4 / 2; ++j) {
      uint8_t best[2];
      for (int h = 0; h < 2; ++h) {
        const float v = xb[h * (QK_MXFP4 / 2) + j];
        int bi = 0;
        float be = fabsf(kv[0] * d - v);
        for (int c = 1; c < 16; ++c) {
          const float err = fabsf(kv[c] * d - v);
          if (err < be) {
            bi = c;
            be = err;
          }
        }
        best[h] = (uint8_t)bi;
      }
      rec[1 + j] = (uint8_t)(best[0] | (best[1] << 4));
    }
  }
}

/* make_qkx2_quants, ggml-quants.c:741-820 (use_mad = false path only) */
static float make_qkx2(int n, int nmax, const float *x, const float *weights, uint8_t *L,
                       float *the_min, uint8_t *Laux, float rmin, float rdelta, int nstep) {
  float min = x[0], max = x[0];
  float sum_w = weights[0];
  float sum_x = sum_w * x[0];
  for (int i = 1; i < n; ++i) {
    if (x[i] < min) min = x[i];
    if (x[i] > max) max = x[i];
    const float w = weights[i];
    sum_w += w;
    sum_x += w * x[i];
  }
  if (min > 0) min = 0;
  if (max == min) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    *the_min = -min;
    return 0.f;
  }
  float iscale = nmax / (max - min);
  float scale = 1 / iscale;
  float best_error = 0;
  for (int i = 0; i < n; ++i) {
    int l = nearest_int(iscale * (x[i] - min));
    l = l < 0 ? 0 : (l > nmax ? nmax : l);
    L[i] = (uint8_t)l;
    float diff = scale * L[i] + min - x[i];
    diff = diff * diff;
    best_error += weights[i] * diff;
  }
  if (nstep < 1) {
    *the_min = -min;
    return scale;
  }
  for (int is = 0; is <= nstep; ++is) {
    iscale = (rmin + rdelta * is + nmax) / (max - min);
    float sum_l = 0, sum_l2 = 0, sum_xl = 0;
    for (int i = 0; i < n; ++i) {
      int l = nearest_int(iscale * (x[i] - min));
      l = l < 0 ? 0 : (l > nmax ? nmax : l);
      Laux[i] = (uint8_t)l;
      const float w = weights[i];
      sum_l += w * l;
      sum_l2 += w * l * l;
      sum_xl += w * l * x[i];
    }
    const float D = sum_w * sum_l2 - sum_l * sum_l;
    if (D > 0) {
      float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
      float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
      if (this_min > 0) {
        this_min = 0;
        this_scale = sum_xl / sum_l2;
      }
      float cur_error = 0;
      for (int i = 0; i < n; ++i) {
        float diff = this_scale * Laux[i] + this_min - x[i];
        diff = diff * diff;
        cur_error += weights[i] * diff;
      }
      if (cur_error < best_error) {
        for (int i = 0; i < n; ++i) L[i] = Laux[i];
        best_error = cur_error;
        scale = this_scale;
        min = this_min;
      }
    }
  }
  *the_min = -min;
  return scale;
}

/* quantize_row_q4_K_ref, ggml-quants.c:1399-1469 */
void wo_quantize_row_q4_K(const float *x, uint8_t *y, int64_t k) {
  const int64_t nb = k / QK_K;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < nb; ++i) {
    uint8_t L[QK_K], Laux[32];
    float weights[32], mins[QK_K / 32], scales[QK_K / 32];
    const float *xb = x + i * QK_K;
    uint8_t *rec = y + i * Q4_K_BYTES;
    uint8_t *sc12 = rec + 4;
    memset(sc12, 0, 12);
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < QK_K / 32; ++j) {
      float sum_x2 = 0;
      for (int l = 0; l < 32; ++l) sum_x2 += xb[32 * j + l] * xb[32 * j + l];
      const float av_x = sqrtf(sum_x2 / 32);
      for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(xb[32 * j + l]);
      scales[j] = make_qkx2(32, 15, xb + 32 * j, weights, L + 32 * j, &mins[j], Laux, -1.f, 0.1f, 20);
      if (scales[j] > max_scale) max_scale = scales[j];
      if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    for (int j = 0; j < QK_K / 32; ++j) {
      uint8_t ls = (uint8_t)nearest_int(inv_scale * scales[j]);
      uint8_t lm = (uint8_t)nearest_int(inv_min * mins[j]);
      ls = ls < 63 ? ls : 63;
      lm = lm < 63 ? lm : 63;
      if (j < 4) {
        sc12[j] = ls;
        sc12[j + 4] = lm;
      } else {
        sc12[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
        sc12[j - 4] |= (uint8_t)((ls >> 4) << 6);
        sc12[j - 0] |= (uint8_t)((lm >> 4) << 6);
      }
    }
    wr16(rec + 0, wo_fp32_to_fp16(max_scale / 63.f));
    wr16(rec + 2, wo_fp32_to_fp16(max_min / 63.f));
    for (int j = 0; j < QK_K / 32; ++j) {
      uint8_t sc, m;
      scale_min_k4(j, sc12, &sc, &m);
      const float d = wo_fp16_to_fp32(rd16(rec)) * sc;
      if (!d) continue;
      const float dm = wo_fp16_to_fp32(rd16(rec + 2)) * m;
      for (int ii = 0; ii < 32; ++ii) {
        int l = nearest_int((xb[32 * j + ii] + dm) / d);
        l = l < 0 ? 0 : (l > 15 ? 15 : l);
        L[32 * j + ii] = (uint8_t)l;
      }
    }
    uint8_t *q = rec + 16;
    for (int j = 0; j < QK_K; j += 64) {
      for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
      q += 32;
    }
  }
}

/* quantize_row_q5_K_ref, ggml-quants.c:1586-1671 (input generator):
 * record d | dmin | scales[12] | qh[32] | qs[128] */
void wo_quantize_row_q5_K(const float *x, uint8_t *y, int64_t k) {
  const int64_t nb = k / QK_K;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < nb; ++i) {
    uint8_t L[QK_K], Laux[32];
    float weights[32], mins[QK_K / 32], scales[QK_K / 32];
    const float *xb = x + i * QK_K;
    uint8_t *rec = y + i * Q5_K_BYTES;
    uint8_t *sc12 = rec + 4;
    memset(sc12, 0, 12);
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < QK_K / 32; ++j) {
      float sum_x2 = 0;
      for (int l = 0; l < 32; ++l) sum_x2 += xb[32 * j + l] * xb[32 * j + l];
      const float av_x = sqrtf(sum_x2 / 32);
      for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(xb[32 * j + l]);
      scales[j] = make_qkx2(32, 31, xb + 32 * j, weights, L + 32 * j, &mins[j], Laux, -0.5f, 0.1f, 15);
      if (scales[j] > max_scale) max_scale = scales[j];
      if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    for (int j = 0; j < QK_K / 32; ++j) {
      uint8_t ls = (uint8_t)nearest_int(inv_scale * scales[j]);
      uint8_t lm = (uint8_t)nearest_int(inv_min * mins[j]);
      ls = ls < 63 ? ls : 63;
      lm = lm < 63 ? lm : 63;
      if (j < 4) {
        sc12[j] = ls;
        sc12[j + 4] = lm;
      } else {
        sc12[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
        sc12[j - 4] |= (uint8_t)((ls >> 4) << 6);
        sc12[j - 0] |= (uint8_t)((lm >> 4) << 6);
      }
    }
    wr16(rec + 0, wo_fp32_to_fp16(max_scale / 63.f));
    wr16(rec + 2, wo_fp32_to_fp16(max_min / 63.f));
    for (int j = 0; j < QK_K / 32; ++j) {
      uint8_t sc, m;
      scale_min_k4(j, sc12, &sc, &m);
      const float d = wo_fp16_to_fp32(rd16(rec)) * sc;
      if (!d) continue;
      const float dm = wo_fp16_to_fp32(rd16(rec + 2)) * m;
      for (int ii = 0; ii < 32; ++ii) {
        int l = nearest_int((xb[32 * j + ii] + dm) / d);
        l = l < 0 ? 0 : (l > 31 ? 31 : l);
        L[32 * j + ii] = (uint8_t)l;
      }
    }
    uint8_t *qh = rec + 16, *ql = rec + 48;
    memset(qh, 0, 32);
    uint8_t m1 = 1, m2 = 2;
    for (int n = 0; n < QK_K; n += 64) {
      for (int j = 0; j < 32; ++j) {
        int l1 = L[n + j], l2 = L[n + j + 32];
        if (l1 > 15) { l1 -= 16; qh[j] |= m1; }
        if (l2 > 15) { l2 -= 16; qh[j] |= m2; }
        ql[j] = (uint8_t)(l1 | (l2 << 4));
      }
      m1 <<= 2;
      m2 <<= 2;
      ql += 32;
    }
  }
}

/* Fast IQ2_XXS input generator, beside GGML's own quantizer
 * (wo_quantize_row_iq2_xxs_ggml below, which searches the iq2xs_init_impl
 * neighbour tables with an importance matrix and is far slower).  This one
 * makes valid records of the same distribution by exhaustive nearest-grid
 * search: per 32-group an
 * amax-derived 4-bit scale, per 8-chunk the sign pattern of x with an even
 * number of minus signs (the smallest |x| is flipped when needed) and the
 * grid row with the least squared error.  Parity unpinned as a quantizer;
 * the GPU path only ever consumes its bytes. */
void wo_quantize_row_iq2_xxs(const float *x, uint8_t *y, int64_t k) {
  uint8_t grid[2048];
  wo_iq2xxs_grid(grid);
  const int64_t nb = k / QK_K;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < nb; ++i) {
    const float *xb = x + i * QK_K;
    uint8_t *rec = y + i * IQ2_XXS_BYTES;
    float gmax[8], tmax = 0.f;
    for (int g = 0; g < 8; ++g) {
      float a = 0.f;
      for (int l = 0; l < 32; ++l) a = fmaxf(a, fabsf(xb[32 * g + l]));
      gmax[g] = a / 43.f; /* wanted element scale: largest |x| on grid value 43 */
      tmax = fmaxf(tmax, gmax[g]);
    }
    /* element scale = d * (2s+1) / 8, s <= 15 */
    const uint16_t dh = wo_fp32_to_fp16(tmax * 8.f / 31.f);
    const float d = wo_fp16_to_fp32(dh);
    wr16(rec, dh);
    for (int g = 0; g < 8; ++g) {
      int s = 0;
      if (d > 0.f) {
        s = (int)lrintf((8.f * gmax[g] / d - 1.f) * 0.5f);
        s = s < 0 ? 0 : (s > 15 ? 15 : s);
      }
      const float db = d * (0.5f + s) * 0.25f;
      uint32_t idx_word = 0, meta = (uint32_t)s << 28;
      for (int c = 0; c < 4; ++c) {
        const float *xc = xb + 32 * g + 8 * c;
        int neg = 0, nneg = 0, smallest = 0;
        for (int j = 0; j < 8; ++j) {
          if (xc[j] < 0) {
            neg |= 1 << j;
            ++nneg;
          }
          if (fabsf(xc[j]) < fabsf(xc[smallest])) smallest = j;
        }
        if (nneg & 1) neg ^= 1 << smallest;
        int best = 0;
        double best_err = INFINITY;
        for (int r = 0; r < 256; ++r) {
          double err = 0;
          for (int j = 0; j < 8; ++j) {
            const double v = (double)db * grid[8 * r + j] * ((neg >> j) & 1 ? -1.0 : 1.0);
            err += (v - xc[j]) * (v - xc[j]);
          }
          if (err < best_err) {
            best_err = err;
            best = r;
          }
        }
        idx_word |= (uint32_t)best << (8 * c);
        meta |= (uint32_t)(neg & 127) << (7 * c);
      }
      uint8_t *qs = rec + 2 + 8 * g;
      for (int b = 0; b < 4; ++b) qs[b] = (uint8_t)(idx_word >> (8 * b));
      for (int b = 0; b < 4; ++b) qs[4 + b] = (uint8_t)(meta >> (8 * b));
    }
  }
}

/* ------------------------------------------------------------------------
 * GGML's IQ2_XXS and IQ2_XS weight quantizers: quantize_iq2_xxs /
 * quantize_iq2_xs (ggml-quants.c:3580-3602), one row at a time through
 * quantize_row_iq2_xxs_impl (:3222-3398) and quantize_row_iq2_xs_impl
 * (:3400-3578), with the search tables of iq2xs_init_impl (:2781-3186) and
 * the helpers make_qp_quants (:1018-1085) and iq2_find_best_neighbour
 * (:3198-3220).  The C is restated with its types: make_qp_quants keeps its
 * levels in uint8_t, so the one negated value of an odd-sign 8-chunk wraps
 * there exactly as in GGML.  GGML asserts an importance matrix; qw == NULL
 * here means every importance is 1, the matrix the reference's repro passes
 * (examples/repro/weft/mul_mat_runtime.cpp:762-776).
 * ---------------------------------------------------------------------- */

/* Search tables of one grid (iq2xs_init_impl): every 8-lane point u of
 * 2-bit levels (lane i in bits 2i, 2i+1; 0 <= u < 43692) is either a grid
 * entry (map[u] = its index) or has a neighbour list: the grid entries whose
 * squared distance to u, taken on the odd integers 2l + 1 of both points,
 * is one of the two smallest distances present, in order of (distance,
 * index).  lists holds, per off-grid point, the count then the indices. */
#define IQ2_KMAP 43692
typedef struct {
  int ngrid;
  const uint16_t *codes;
  int32_t map[IQ2_KMAP];
  int32_t off[IQ2_KMAP];
  uint16_t *lists;
  int8_t pos[512][8];
} Iq2Search;

static Iq2Search g_iq2_search[2];
static pthread_once_t g_iq2_once[2] = {PTHREAD_ONCE_INIT, PTHREAD_ONCE_INIT};

static int iq2_distance(const int8_t a[8], const int8_t b[8]) {
  int d2 = 0;
  for (int k = 0; k < 8; ++k) d2 += (a[k] - b[k]) * (a[k] - b[k]);
  return d2;
}

static void iq2_search_build(Iq2Search *s) {
  for (int j = 0; j < s->ngrid; ++j)
    for (int k = 0; k < 8; ++k) s->pos[j][k] = (int8_t)(2 * ((s->codes[j] >> (2 * k)) & 3) + 1);
  for (int u = 0; u < IQ2_KMAP; ++u) s->map[u] = -1;
  for (int j = 0; j < s->ngrid; ++j) s->map[s->codes[j]] = j;
  /* pass 1: list lengths (the two smallest distances and how many entries
   * lie at them), pass 2: the lists */
  int64_t total = 0;
  for (int u = 0; u < IQ2_KMAP; ++u) {
    s->off[u] = -1;
    if (s->map[u] >= 0) continue;
    int8_t p[8];
    for (int k = 0; k < 8; ++k) p[k] = (int8_t)(2 * ((u >> (2 * k)) & 3) + 1);
    int d1 = INT32_MAX, d2 = INT32_MAX, n = 0;
    for (int j = 0; j < s->ngrid; ++j) {
      const int d = iq2_distance(p, s->pos[j]);
      if (d < d1) {
        d2 = d1;
        d1 = d;
      } else if (d > d1 && d < d2) {
        d2 = d;
      }
    }
    for (int j = 0; j < s->ngrid; ++j) {
      const int d = iq2_distance(p, s->pos[j]);
      n += d == d1 || d == d2;
    }
    s->off[u] = (int32_t)total;
    total += 1 + n;
  }
  s->lists = (uint16_t *)malloc((size_t)total * sizeof(uint16_t));
  for (int u = 0; u < IQ2_KMAP; ++u) {
    if (s->off[u] < 0) continue;
    int8_t p[8];
    for (int k = 0; k < 8; ++k) p[k] = (int8_t)(2 * ((u >> (2 * k)) & 3) + 1);
    int d1 = INT32_MAX, d2 = INT32_MAX;
    for (int j = 0; j < s->ngrid; ++j) {
      const int d = iq2_distance(p, s->pos[j]);
      if (d < d1) {
        d2 = d1;
        d1 = d;
      } else if (d > d1 && d < d2) {
        d2 = d;
      }
    }
    uint16_t *out = s->lists + s->off[u];
    int n = 0;
    for (int pass = 0; pass < 2; ++pass) { /* distance d1 first, then d2; ascending index in each */
      const int want = pass == 0 ? d1 : d2;
      if (pass == 1 && d2 == INT32_MAX) break;
      for (int j = 0; j < s->ngrid; ++j)
        if (iq2_distance(p, s->pos[j]) == want) out[1 + n++] = (uint16_t)j;
    }
    out[0] = (uint16_t)n;
  }
}

static void iq2_search_init_xxs(void) {
  g_iq2_search[0].ngrid = 256;
  g_iq2_search[0].codes = kIq2xxsCodes;
  iq2_search_build(&g_iq2_search[0]);
}
static void iq2_search_init_xs(void) {
  g_iq2_search[1].ngrid = 512;
  g_iq2_search[1].codes = kIq2xsCodes;
  iq2_search_build(&g_iq2_search[1]);
}

static const Iq2Search *iq2_search(int xs) {
  pthread_once(&g_iq2_once[xs], xs ? iq2_search_init_xs : iq2_search_init_xxs);
  return &g_iq2_search[xs];
}

int wo_iq2_grid_index(int xs, int u) {
  if (u < 0 || u >= IQ2_KMAP) return -2;
  return iq2_search(xs != 0)->map[u];
}

int wo_iq2_neighbours(int xs, int u, uint16_t *out) {
  if (u < 0 || u >= IQ2_KMAP) return -1;
  const Iq2Search *s = iq2_search(xs != 0);
  if (s->off[u] < 0) return 0;
  const uint16_t *l = s->lists + s->off[u];
  for (int i = 0; i < l[0]; ++i) out[i] = l[1 + i];
  return l[0];
}

/* make_qp_quants, ggml-quants.c:1018-1085 */
static float make_qp_quants(int n, int nmax, const float *x, uint8_t *L, const float *quant_weights) {
  float max = 0;
  for (int i = 0; i < n; ++i) max = max > x[i] ? max : x[i];
  if (max < 1e-15f) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    return 0.f;
  }
  float iscale = nmax / max;
  for (int i = 0; i < n; ++i) L[i] = (uint8_t)nearest_int(iscale * x[i]);
  float scale = 1 / iscale;
  float best_mse = 0;
  for (int i = 0; i < n; ++i) {
    const float diff = x[i] - scale * L[i];
    const float w = quant_weights[i];
    best_mse += w * diff * diff;
  }
  for (int is = -4; is <= 4; ++is) {
    if (is == 0) continue;
    const float iscale_is = (0.1f * is + nmax) / max;
    const float scale_is = 1 / iscale_is;
    float mse = 0;
    for (int i = 0; i < n; ++i) {
      int l = nearest_int(iscale_is * x[i]);
      l = l < nmax ? l : nmax;
      const float diff = x[i] - scale_is * l;
      const float w = quant_weights[i];
      mse += w * diff * diff;
    }
    if (mse < best_mse) {
      best_mse = mse;
      iscale = iscale_is;
    }
  }
  float sumlx = 0, suml2 = 0;
  for (int i = 0; i < n; ++i) {
    int l = nearest_int(iscale * x[i]);
    l = l < nmax ? l : nmax;
    L[i] = (uint8_t)l;
    const float w = quant_weights[i];
    sumlx += w * x[i] * l;
    suml2 += w * l * l;
  }
  for (int itry = 0; itry < 5; ++itry) {
    int n_changed = 0;
    for (int i = 0; i < n; ++i) {
      const float w = quant_weights[i];
      float slx = sumlx - w * x[i] * L[i];
      float sl2 = suml2 - w * L[i] * L[i];
      if (slx > 0 && sl2 > 0) {
        int new_l = nearest_int(x[i] * sl2 / slx);
        new_l = new_l < nmax ? new_l : nmax;
        if (new_l != L[i]) {
          slx += w * x[i] * new_l;
          sl2 += w * new_l * new_l;
          if (slx * slx * suml2 > sumlx * sumlx * sl2) {
            L[i] = (uint8_t)new_l;
            sumlx = slx;
            suml2 = sl2;
            ++n_changed;
          }
        }
      }
    }
    if (!n_changed) break;
  }
  return suml2 > 0.0f ? sumlx / suml2 : 0.0f;
}

/* iq2_find_best_neighbour, ggml-quants.c:3198-3220: the neighbour with the
 * least weighted squared error at this scale (first one on ties) */
static int iq2_best_neighbour(const Iq2Search *s, int u, const float *xval, const float *weight, float scale,
                              int8_t *L) {
  const uint16_t *nb = s->lists + s->off[u];
  float best_d2 = FLT_MAX;
  int grid_index = -1;
  for (int j = 1; j <= nb[0]; ++j) {
    const int8_t *pg = s->pos[nb[j]];
    float d2 = 0;
    for (int i = 0; i < 8; ++i) {
      const float q = pg[i];
      const float diff = scale * q - xval[i];
      d2 += weight[i] * diff * diff;
    }
    if (d2 < best_d2) {
      best_d2 = d2;
      grid_index = nb[j];
    }
  }
  const int8_t *pg = s->pos[grid_index];
  for (int i = 0; i < 8; ++i) L[i] = (int8_t)((pg[i] - 1) / 2);
  return grid_index;
}

/* the sign pattern of an 8-chunk with an even number of minus signs
 * (ggml-quants.c:3260-3279): the least weighted x^2 of an odd pattern is
 * negated in xval and its sign bit flipped; returns the 7 stored bits */
static uint8_t iq2_chunk_signs(const float *xb, const float *weight, float *xval) {
  int nflip = 0;
  uint8_t s = 0;
  for (int i = 0; i < 8; ++i) {
    if (xb[i] >= 0) {
      xval[i] = xb[i];
    } else {
      xval[i] = -xb[i];
      ++nflip;
      s |= (uint8_t)(1 << i);
    }
  }
  if (nflip % 2) {
    int imin = 0;
    float min = weight[imin] * xb[imin] * xb[imin];
    for (int i = 1; i < 8; ++i) {
      const float ax = weight[i] * xb[i] * xb[i];
      if (ax < min) {
        min = ax;
        imin = i;
      }
    }
    xval[imin] = -xval[imin];
    s ^= (uint8_t)(1 << imin);
  }
  return s & 127;
}

/* the 2-bit levels of 8 values at inverse scale id, clamped to [0, 2] */
static uint16_t iq2_levels(const float *xval, float id, int8_t *L) {
  uint16_t u = 0;
  for (int i = 0; i < 8; ++i) {
    int l = nearest_int(0.5f * (id * xval[i] - 1));
    l = l < 0 ? 0 : (l > 2 ? 2 : l);
    L[i] = (int8_t)l;
    u |= (uint16_t)(l << 2 * i);
  }
  return u;
}

/* quantize_row_iq2_xxs_impl, ggml-quants.c:3222-3398 */
void wo_quantize_row_iq2_xxs_ggml(const float *x, uint8_t *y, int64_t k, const float *quant_weights) {
  const Iq2Search *s = iq2_search(0);
  const int kMaxQ = 3;
  const int64_t nbl = k / QK_K;
#pragma omp parallel for schedule(dynamic, 16)
  for (int64_t ibl = 0; ibl < nbl; ++ibl) {
    float scales[QK_K / 32], weight[32], xval[32], waux[32], ones[32];
    int8_t L[32], Laux[32];
    uint8_t block_signs[4];
    uint32_t q2[2 * (QK_K / 32)];
    uint8_t *rec = y + ibl * IQ2_XXS_BYTES;
    for (int i = 0; i < 32; ++i) ones[i] = 1.f;
    wr16(rec, wo_fp32_to_fp16(0.f));
    memset(q2, 0, sizeof q2);
    float max_scale = 0;
    const float *xbl = x + QK_K * ibl;
    float sumx2 = 0;
    for (int i = 0; i < QK_K; ++i) sumx2 += xbl[i] * xbl[i];
    const float sigma2 = sumx2 / QK_K;
    for (int ib = 0; ib < QK_K / 32; ++ib) {
      const float *xb = xbl + 32 * ib;
      const float *qw = quant_weights ? quant_weights + QK_K * ibl + 32 * ib : ones;
      for (int i = 0; i < 32; ++i) weight[i] = qw[i] * sqrtf(sigma2 + xb[i] * xb[i]);
      for (int i = 0; i < 32; ++i) waux[i] = sqrtf(weight[i]);
      for (int c = 0; c < 4; ++c) block_signs[c] = iq2_chunk_signs(xb + 8 * c, weight + 8 * c, xval + 8 * c);
      float max = xval[0];
      for (int i = 1; i < 32; ++i) max = max > xval[i] ? max : xval[i];
      if (max < 1e-15f) {
        scales[ib] = 0;
        memset(L, 0, 32);
        continue;
      }
      float scale = make_qp_quants(32, kMaxQ + 1, xval, (uint8_t *)L, weight);
      const float eff_max = scale * kMaxQ;
      if (eff_max <= 0) {
        scales[ib] = 0;
        memset(L, 0, 32);
        continue;
      }
      float best = 0;
      for (int is = -6; is <= 6; ++is) {
        const float id = (2 * kMaxQ - 1 + is * 0.1f) / eff_max;
        const float this_scale = 1 / id;
        for (int c = 0; c < 4; ++c) {
          const uint16_t u = iq2_levels(xval + 8 * c, id, Laux + 8 * c);
          if (s->map[u] < 0) iq2_best_neighbour(s, u, xval + 8 * c, waux + 8 * c, this_scale, Laux + 8 * c);
        }
        float sumqx = 0, sumq2 = 0;
        for (int i = 0; i < 32; ++i) {
          const float w = weight[i];
          const float q = 2 * Laux[i] + 1;
          sumqx += w * xval[i] * q;
          sumq2 += w * q * q;
        }
        if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
          scale = sumqx / sumq2;
          best = scale * sumqx;
          memcpy(L, Laux, 32);
        }
      }
      if (scale > 0) {
        const float id = 1 / scale;
        for (int c = 0; c < 4; ++c) {
          const uint16_t u = iq2_levels(xval + 8 * c, id, L + 8 * c);
          const int gi = s->map[u] >= 0 ? s->map[u] : iq2_best_neighbour(s, u, xval + 8 * c, waux + 8 * c, scale, L + 8 * c);
          for (int i = 0; i < 8; ++i) L[8 * c + i] = (int8_t)((s->pos[gi][i] - 1) / 2);
        }
        float sumqx = 0, sumq2 = 0;
        for (int i = 0; i < 32; ++i) {
          const float w = weight[i];
          const float q = 2 * L[i] + 1;
          sumqx += w * xval[i] * q;
          sumq2 += w * q * q;
        }
        if (sumq2 > 0) scale = sumqx / sumq2;
      }
      if (scale < 0) {
        scale = -scale;
        for (int c = 0; c < 4; ++c) block_signs[c] = (uint8_t)(~block_signs[c] & 127);
      }
      for (int c = 0; c < 4; ++c) {
        uint16_t u = 0;
        for (int i = 0; i < 8; ++i) u |= (uint16_t)(L[8 * c + i] << 2 * i);
        const int gi = s->map[u]; /* on the grid by construction (GGML aborts otherwise) */
        q2[2 * ib + 0] |= (uint32_t)gi << 8 * c;
        q2[2 * ib + 1] |= (uint32_t)block_signs[c] << 7 * c;
      }
      scales[ib] = scale;
      max_scale = max_scale > scale ? max_scale : scale;
    }
    if (!max_scale) {
      memset(rec + 2, 0, QK_K / 4);
      continue;
    }
    const float d = max_scale / 31;
    wr16(rec, wo_fp32_to_fp16(d));
    const float id = 1 / d;
    for (int ib = 0; ib < QK_K / 32; ++ib) {
      int l = nearest_int(0.5f * (id * scales[ib] - 1));
      l = l < 0 ? 0 : (l > 15 ? 15 : l);
      q2[2 * ib + 1] |= (uint32_t)l << 28;
    }
    for (int w = 0; w < 16; ++w)
      for (int b = 0; b < 4; ++b) rec[2 + 4 * w + b] = (uint8_t)(q2[w] >> (8 * b));
  }
}

/* quantize_row_iq2_xs_impl, ggml-quants.c:3400-3578 */
void wo_quantize_row_iq2_xs_ggml(const float *x, uint8_t *y, int64_t k, const float *quant_weights) {
  const Iq2Search *s = iq2_search(1);
  const int kMaxQ = 3;
  const int64_t nbl = k / QK_K;
#pragma omp parallel for schedule(dynamic, 16)
  for (int64_t ibl = 0; ibl < nbl; ++ibl) {
    float scales[QK_K / 16], weight[16], xval[16], waux[16], ones[16];
    int8_t L[16], Laux[16];
    int on_grid[2], on_grid_aux[2];
    uint8_t block_signs[2];
    uint16_t q2[2 * (QK_K / 16)];
    uint8_t *rec = y + ibl * IQ2_XS_BYTES;
    for (int i = 0; i < 16; ++i) ones[i] = 1.f;
    wr16(rec, wo_fp32_to_fp16(0.f));
    memset(q2, 0, sizeof q2);
    memset(rec + 2 + QK_K / 4, 0, QK_K / 32);
    float max_scale = 0;
    const float *xbl = x + QK_K * ibl;
    float sumx2 = 0;
    for (int i = 0; i < QK_K; ++i) sumx2 += xbl[i] * xbl[i];
    const float sigma2 = sumx2 / QK_K;
    for (int ib = 0; ib < QK_K / 16; ++ib) {
      const float *xb = xbl + 16 * ib;
      const float *qw = quant_weights ? quant_weights + QK_K * ibl + 16 * ib : ones;
      for (int i = 0; i < 16; ++i) weight[i] = qw[i] * sqrtf(sigma2 + xb[i] * xb[i]);
      for (int i = 0; i < 16; ++i) waux[i] = sqrtf(weight[i]);
      for (int c = 0; c < 2; ++c) block_signs[c] = iq2_chunk_signs(xb + 8 * c, weight + 8 * c, xval + 8 * c);
      float max = xval[0];
      for (int i = 1; i < 16; ++i) max = max > xval[i] ? max : xval[i];
      memset(L, 0, 16);
      if (max < 1e-15f) {
        scales[ib] = 0;
        continue;
      }
      float best = 0;
      float scale = max / (2 * kMaxQ - 1);
      on_grid[0] = on_grid[1] = 1;
      for (int is = -9; is <= 9; ++is) {
        const float id = (2 * kMaxQ - 1 + is * 0.1f) / max;
        const float this_scale = 1 / id;
        for (int c = 0; c < 2; ++c) {
          const uint16_t u = iq2_levels(xval + 8 * c, id, Laux + 8 * c);
          on_grid_aux[c] = s->map[u] >= 0;
          if (!on_grid_aux[c]) iq2_best_neighbour(s, u, xval + 8 * c, waux + 8 * c, this_scale, Laux + 8 * c);
        }
        float sumqx = 0, sumq2 = 0;
        for (int i = 0; i < 16; ++i) {
          const float w = weight[i];
          const float q = 2 * Laux[i] + 1;
          sumqx += w * xval[i] * q;
          sumq2 += w * q * q;
        }
        if (sumq2 > 0 && sumqx * sumqx > best * sumq2) {
          scale = sumqx / sumq2;
          best = scale * sumqx;
          memcpy(L, Laux, 16);
          on_grid[0] = on_grid_aux[0];
          on_grid[1] = on_grid_aux[1];
        }
      }
      if ((!on_grid[0] || !on_grid[1]) && scale > 0) {
        const float id = 1 / scale;
        for (int c = 0; c < 2; ++c) {
          if (on_grid[c]) continue;
          const uint16_t u = iq2_levels(xval + 8 * c, id, L + 8 * c);
          if (s->map[u] < 0) iq2_best_neighbour(s, u, xval + 8 * c, waux + 8 * c, scale, L + 8 * c);
        }
        float sumqx = 0, sumq2 = 0;
        for (int i = 0; i < 16; ++i) {
          const float w = weight[i];
          const float q = 2 * L[i] + 1;
          sumqx += w * xval[i] * q;
          sumq2 += w * q * q;
        }
        if (sumq2 > 0) scale = sumqx / sumq2;
      }
      if (scale < 0) {
        scale = -scale;
        for (int c = 0; c < 2; ++c) block_signs[c] = (uint8_t)(~block_signs[c] & 127);
      }
      for (int c = 0; c < 2; ++c) {
        uint16_t u = 0;
        for (int i = 0; i < 8; ++i) u |= (uint16_t)(L[8 * c + i] << 2 * i);
        q2[2 * ib + c] = (uint16_t)(s->map[u] | (block_signs[c] << 9));
      }
      scales[ib] = scale;
      max_scale = max_scale > scale ? max_scale : scale;
    }
    if (!max_scale) {
      memset(rec + 2, 0, QK_K / 4);
      continue;
    }
    const float d = max_scale / 31;
    wr16(rec, wo_fp32_to_fp16(d));
    const float id = 1 / d;
    uint8_t *sc = rec + 2 + QK_K / 4;
    for (int ib = 0; ib < QK_K / 16; ++ib) {
      int l = nearest_int(0.5f * (id * scales[ib] - 1));
      l = l < 0 ? 0 : (l > 15 ? 15 : l);
      if (ib % 2 == 0)
        sc[ib / 2] = (uint8_t)l;
      else
        sc[ib / 2] |= (uint8_t)(l << 4);
    }
    for (int w = 0; w < 32; ++w) wr16(rec + 2 + 2 * w, q2[w]);
  }
}

/* ------------------------------------------------------------------------
 * Activation quantizers
 * ---------------------------------------------------------------------- */

/* quantize_row_q8_0_ref, ggml-quants.c:238-261: d = amax/127, q = roundf(x/d)
 * (round half away from zero), d stored as fp16. */
/* make_qx_quants, ggml-quants.c:570-635 (qw == NULL), with the iteration
 * over is = -9..9 of the candidate scales */
static float make_qx(int n, int nmax, const float *x, int8_t *L, int rmse_type) {
  float max = 0, amax = 0;
  for (int i = 0; i < n; ++i) {
    const float ax = fabsf(x[i]);
    if (ax > amax) { amax = ax; max = x[i]; }
  }
  if (amax < GROUP_MAX_EPS) {
    for (int i = 0; i < n; ++i) L[i] = 0;
    return 0.f;
  }
  float iscale = -nmax / max;
  float sumlx = 0, suml2 = 0;
  for (int i = 0; i < n; ++i) {
    int l = nearest_int(iscale * x[i]);
    l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
    L[i] = (int8_t)(l + nmax);
    const float w = rmse_type == 1 ? x[i] * x[i] : 1.f;
    sumlx += w * x[i] * l;
    suml2 += w * l * l;
  }
  float scale = suml2 ? sumlx / suml2 : 0.0f;
  float best = scale * sumlx;
  for (int is = -9; is <= 9; ++is) {
    if (is == 0) continue;
    iscale = -(nmax + 0.1f * is) / max;
    sumlx = suml2 = 0;
    for (int i = 0; i < n; ++i) {
      int l = nearest_int(iscale * x[i]);
      l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
      const float w = rmse_type == 1 ? x[i] * x[i] : 1.f;
      sumlx += w * x[i] * l;
      suml2 += w * l * l;
    }
    if (suml2 > 0 && sumlx * sumlx > best * suml2) {
      for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
        L[i] = (int8_t)(l + nmax);
      }
      scale = sumlx / suml2;
      best = scale * sumlx;
    }
  }
  return scale;
}

/* quantize_row_q6_K_ref, ggml-quants.c:1811-1879 (input generator).
 * Record: ql[128] | qh[64] | scales[16] (int8) | d (fp16). */
void wo_quantize_row_q6_K(const float *x, uint8_t *y, int64_t k) {
  const int64_t nb = k / QK_K;
  int8_t L[QK_K];
  float scales[QK_K / 16];
  for (int64_t i = 0; i < nb; ++i, x += QK_K, y += Q6_K_BYTES) {
    float max_scale = 0, max_abs_scale = 0;
    for (int ib = 0; ib < QK_K / 16; ++ib) {
      const float scale = make_qx(16, 32, x + 16 * ib, L + 16 * ib, 1);
      scales[ib] = scale;
      const float abs_scale = fabsf(scale);
      if (abs_scale > max_abs_scale) {
        max_abs_scale = abs_scale;
        max_scale = scale;
      }
    }
    if (max_abs_scale < GROUP_MAX_EPS) {
      memset(y, 0, Q6_K_BYTES);
      wr16(y + 208, wo_fp32_to_fp16(0.f));
      continue;
    }
    const float iscale = -128.f / max_scale;
    wr16(y + 208, wo_fp32_to_fp16(1 / iscale));
    int8_t *sc = (int8_t *)(y + 192);
    for (int ib = 0; ib < QK_K / 16; ++ib) {
      const int v = nearest_int(iscale * scales[ib]);
      sc[ib] = (int8_t)(v < 127 ? v : 127);
    }
    for (int j = 0; j < QK_K / 16; ++j) {
      const float d = wo_fp16_to_fp32(rd16(y + 208)) * sc[j];
      if (!d) continue;
      for (int ii = 0; ii < 16; ++ii) {
        int l = nearest_int(x[16 * j + ii] / d);
        l = l < -32 ? -32 : l > 31 ? 31 : l;
        L[16 * j + ii] = (int8_t)(l + 32);
      }
    }
    uint8_t *ql = y, *qh = y + 128;
    for (int j = 0; j < QK_K; j += 128, ql += 64, qh += 32) {
      for (int l = 0; l < 32; ++l) {
        const uint8_t q1 = L[j + l] & 0xF, q2 = L[j + l + 32] & 0xF;
        const uint8_t q3 = L[j + l + 64] & 0xF, q4 = L[j + l + 96] & 0xF;
        ql[l] = q1 | (q3 << 4);
        ql[l + 32] = q2 | (q4 << 4);
        qh[l] = (L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                ((L[j + l + 96] >> 4) << 6);
      }
    }
  }
}

void wo_quantize_row_q8_0(const float *x, uint8_t *y, int64_t k) {
  const int64_t nb = k / QK8_0;
  for (int64_t i = 0; i < nb; ++i) {
    const float *xb = x + i * QK8_0;
    uint8_t *rec = y + i * Q8_0_BYTES;
    float amax = 0.0f;
    for (int j = 0; j < QK8_0; ++j) amax = fmaxf(amax, fabsf(xb[j]));
    const float d = amax / 127;
    const float id = d ? 1.0f / d : 0.0f;
    wr16(rec, wo_fp32_to_fp16(d));
    for (int j = 0; j < QK8_0; ++j) rec[2 + j] = (uint8_t)(int8_t)roundf(xb[j] * id);
  }
}

/* quantize_row_q4_1_ref, ggml-quants.c:112-146: d = (max - min) / 15,
 * m = min, q = MIN(15, (int8_t)((x - min) * id + 0.5f)). */
void wo_quantize_row_q4_1(const float *x, uint8_t *y, int64_t k) {
  const int64_t nb = k / 32;
  for (int64_t i = 0; i < nb; ++i) {
    const float *xb = x + i * 32;
    uint8_t *rec = y + i * Q4_1_BYTES;
    float min = 3.402823466e+38f, max = -3.402823466e+38f;
    for (int j = 0; j < 32; ++j) {
      if (xb[j] < min) min = xb[j];
      if (xb[j] > max) max = xb[j];
    }
    const float d = (max - min) / 15;
    const float id = d ? 1.0f / d : 0.0f;
    wr16(rec, wo_fp32_to_fp16(d));
    wr16(rec + 2, wo_fp32_to_fp16(min));
    for (int j = 0; j < 16; ++j) {
      const float x0 = (xb[j] - min) * id, x1 = (xb[16 + j] - min) * id;
      const int v0 = (int8_t)(x0 + 0.5f), v1 = (int8_t)(x1 + 0.5f);
      const uint8_t q0 = (uint8_t)(v0 < 15 ? v0 : 15), q1 = (uint8_t)(v1 < 15 ? v1 : 15);
      rec[4 + j] = (uint8_t)(q0 | (q1 << 4));
    }
  }
}

/* quantize_row_q8_1_ref, ggml-quants.c:264-295: Q8_0's d and roundf codes,
 * plus s = fp16(sum(q) * d) with the fp32 d. */
void wo_quantize_row_q8_1(const float *x, uint8_t *y, int64_t k) {
  const int64_t nb = k / 32;
  for (int64_t i = 0; i < nb; ++i) {
    const float *xb = x + i * 32;
    uint8_t *rec = y + i * Q8_1_BYTES;
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(xb[j]));
    const float d = amax / 127;
    const float id = d ? 1.0f / d : 0.0f;
    wr16(rec, wo_fp32_to_fp16(d));
    int sum = 0;
    for (int j = 0; j < 32; ++j) {
      const int8_t q = (int8_t)roundf(xb[j] * id);
      rec[4 + j] = (uint8_t)q;
      sum += q;
    }
    wr16(rec + 2, wo_fp32_to_fp16(sum * d));
  }
}

/* quantize_row_q8_K_ref, ggml-quants.c:2696-2733: the signed value at the
 * first index of the largest |x| sets iscale = -127/max; q = RNE(iscale*x)
 * capped at 127; bsums = sums of 16; d = 1/iscale.  An all-zero block writes
 * d = 0 and qs = 0 and leaves bsums as they were. */
void wo_quantize_row_q8_K(const float *x, uint8_t *y, int64_t k) {
  const int64_t nb = k / QK_K;
  for (int64_t i = 0; i < nb; ++i) {
    const float *xb = x + i * QK_K;
    uint8_t *rec = y + i * Q8_K_BYTES;
    float max = 0, amax = 0;
    for (int j = 0; j < QK_K; ++j) {
      const float ax = fabsf(xb[j]);
      if (ax > amax) {
        amax = ax;
        max = xb[j];
      }
    }
    if (!amax) {
      wrf32(rec, 0.f);
      memset(rec + 4, 0, QK_K);
      continue;
    }
    const float iscale = -127.f / max;
    int8_t *qs = (int8_t *)(rec + 4);
    for (int j = 0; j < QK_K; ++j) {
      const int v = nearest_int(iscale * xb[j]);
      qs[j] = (int8_t)(v < 127 ? v : 127);
    }
    for (int j = 0; j < QK_K / 16; ++j) {
      int sum = 0;
      for (int ii = 0; ii < 16; ++ii) sum += qs[16 * j + ii];
      wr16(rec + 260 + 2 * j, (uint16_t)(int16_t)sum);
    }
    wrf32(rec, 1 / iscale);
  }
}

/* ------------------------------------------------------------------------
 * Row dequantizers
 * ---------------------------------------------------------------------- */

/* dequantize_row_q4_0, ggml-quants.c:401-419 */
void wo_dequantize_row_q4_0(const uint8_t *x, float *y, int64_t k) {
  const int64_t nb = k / QK4_0;
  for (int64_t i = 0; i < nb; ++i) {
    const uint8_t *rec = x + i * Q4_0_BYTES;
    const float d = wo_fp16_to_fp32(rd16(rec));
    for (int j = 0; j < QK4_0 / 2; ++j) {
      const int x0 = (rec[2 + j] & 0x0F) - 8;
      const int x1 = (rec[2 + j] >> 4) - 8;
      y[i * QK4_0 + j] = x0 * d;
      y[i * QK4_0 + j + QK4_0 / 2] = x1 * d;
    }
  }
}

/* dequantize_row_q4_1, ggml-quants.c:421-439 */
void wo_dequantize_row_q4_1(const uint8_t *x, float *y, int64_t k) {
  const int64_t nb = k / 32;
  for (int64_t i = 0; i < nb; ++i) {
    const uint8_t *rec = x + i * Q4_1_BYTES;
    const float d = wo_fp16_to_fp32(rd16(rec)), m = wo_fp16_to_fp32(rd16(rec + 2));
    for (int j = 0; j < 16; ++j) {
      y[i * 32 + j] = (rec[4 + j] & 0x0F) * d + m;
      y[i * 32 + j + 16] = (rec[4 + j] >> 4) * d + m;
    }
  }
}

/* dequantize_row_iq2_xs, ggml-quants.c:2444-2467 */
void wo_dequantize_row_iq2_xs(const uint8_t *x, float *y, int64_t k) {
  uint8_t grid[4096], ks[128];
  wo_iq2xs_grid(grid);
  wo_ksigns_iq2xs(ks);
  const int64_t nb = k / QK_K;
  for (int64_t i = 0; i < nb; ++i) {
    const uint8_t *rec = x + i * IQ2_XS_BYTES;
    const float d = wo_fp16_to_fp32(rd16(rec));
    for (int ib32 = 0; ib32 < 8; ++ib32) {
      const uint8_t sc = rec[66 + ib32];
      const float db[2] = {d * (0.5f + (sc & 0xf)) * 0.25f, d * (0.5f + (sc >> 4)) * 0.25f};
      for (int l = 0; l < 4; ++l) {
        const uint16_t q = rd16(rec + 2 + 2 * (4 * ib32 + l));
        const uint8_t *g = grid + 8 * (q & 511);
        const uint8_t signs = ks[q >> 9];
        for (int j = 0; j < 8; ++j) *y++ = db[l / 2] * g[j] * (signs & (1 << j) ? -1.f : 1.f);
      }
    }
  }
}

/* dequantize_row_mxfp4, ggml-quants.c:511-529 */
void wo_dequantize_row_mxfp4(const uint8_t *x, float *y, int64_t k) {
  int8_t kv[16];
  wo_kvalues_mxfp4(kv);
  const int64_t nb = k / QK_MXFP4;
  for (int64_t i = 0; i < nb; ++i) {
    const uint8_t *rec = x + i * MXFP4_BYTES;
    const float d = wo_e8m0_to_fp32_half(rec[0]);
    for (int j = 0; j < QK_MXFP4 / 2; ++j) {
      y[i * QK_MXFP4 + j] = kv[rec[1 + j] & 0x0F] * d;
      y[i * QK_MXFP4 + j + QK_MXFP4 / 2] = kv[rec[1 + j] >> 4] * d;
    }
  }
}

/* dequantize_row_q4_K, ggml-quants.c:1471-1493 */
void wo_dequantize_row_q4_K(const uint8_t *x, float *y, int64_t k) {
  const int64_t nb = k / QK_K;
  for (int64_t i = 0; i < nb; ++i) {
    const uint8_t *rec = x + i * Q4_K_BYTES;
    const uint8_t *q = rec + 16;
    const float d = wo_fp16_to_fp32(rd16(rec));
    const float min = wo_fp16_to_fp32(rd16(rec + 2));
    int is = 0;
    for (int j = 0; j < QK_K; j += 64) {
      uint8_t sc, m;
      scale_min_k4(is + 0, rec + 4, &sc, &m);
      const float d1 = d * sc, m1 = min * m;
      scale_min_k4(is + 1, rec + 4, &sc, &m);
      const float d2 = d * sc, m2 = min * m;
      for (int l = 0; l < 32; ++l) *y++ = d1 * (q[l] & 0xF) - m1;
      for (int l = 0; l < 32; ++l) *y++ = d2 * (q[l] >> 4) - m2;
      q += 32;
      is += 2;
    }
  }
}

/* dequantize_row_iq2_xxs, ggml-quants.c:2416-2440 */
void wo_dequantize_row_iq2_xxs(const uint8_t *x, float *y, int64_t k) {
  uint8_t grid[2048], ks[128];
  wo_iq2xxs_grid(grid);
  wo_ksigns_iq2xs(ks);
  const int64_t nb = k / QK_K;
  for (int64_t i = 0; i < nb; ++i) {
    const uint8_t *rec = x + i * IQ2_XXS_BYTES;
    const float d = wo_fp16_to_fp32(rd16(rec));
    for (int ib32 = 0; ib32 < QK_K / 32; ++ib32) {
      const uint8_t *qs = rec + 2 + 8 * ib32;
      const uint32_t meta = rd32(qs + 4);
      const float db = d * (0.5f + (meta >> 28)) * 0.25f;
      for (int l = 0; l < 4; ++l) {
        const uint8_t *g = grid + 8 * qs[l];
        const uint8_t signs = ks[(meta >> (7 * l)) & 127];
        for (int j = 0; j < 8; ++j) y[j] = db * g[j] * (signs & (1u << j) ? -1.f : 1.f);
        y += 8;
      }
    }
  }
}

/* ------------------------------------------------------------------------
 * vec_dots (ggml-cpu/quants.c generic bodies)
 * ---------------------------------------------------------------------- */

/* ggml_vec_dot_q4_0_q8_0_generic, ggml-cpu/quants.c:174-208 */
float wo_vec_dot_q4_0_q8_0(const uint8_t *w, const uint8_t *x, int64_t k) {
  const int64_t nb = k / QK8_0;
  float sumf = 0;
  for (int64_t ib = 0; ib < nb; ++ib) {
    const uint8_t *wr = w + ib * Q4_0_BYTES;
    const uint8_t *xr = x + ib * Q8_0_BYTES;
    const int8_t *xq = (const int8_t *)(xr + 2);
    int sumi0 = 0, sumi1 = 0;
    for (int j = 0; j < QK8_0 / 2; ++j) {
      const int v0 = (wr[2 + j] & 0x0F) - 8;
      const int v1 = (wr[2 + j] >> 4) - 8;
      sumi0 += v0 * xq[j];
      sumi1 += v1 * xq[j + QK8_0 / 2];
    }
    const int sumi = sumi0 + sumi1;
    sumf += sumi * wo_fp16_to_fp32(rd16(wr)) * wo_fp16_to_fp32(rd16(xr));
  }
  return sumf;
}

/* ggml_vec_dot_q4_1_q8_1_generic, ggml-cpu/quants.c:211-245 */
float wo_vec_dot_q4_1_q8_1(const uint8_t *w, const uint8_t *x, int64_t k) {
  const int64_t nb = k / 32;
  float sumf = 0;
  for (int64_t ib = 0; ib < nb; ++ib) {
    const uint8_t *wr = w + ib * Q4_1_BYTES;
    const uint8_t *xr = x + ib * Q8_1_BYTES;
    const int8_t *xq = (const int8_t *)(xr + 4);
    int sumi0 = 0, sumi1 = 0;
    for (int j = 0; j < 16; ++j) {
      sumi0 += (wr[4 + j] & 0x0F) * xq[j];
      sumi1 += (wr[4 + j] >> 4) * xq[j + 16];
    }
    const int sumi = sumi0 + sumi1;
    sumf += (wo_fp16_to_fp32(rd16(wr)) * wo_fp16_to_fp32(rd16(xr))) * sumi +
            wo_fp16_to_fp32(rd16(wr + 2)) * wo_fp16_to_fp32(rd16(xr + 2));
  }
  return sumf;
}

/* ggml_vec_dot_iq2_xs_q8_K_generic, ggml-cpu/quants.c:897-946 */
float wo_vec_dot_iq2_xs_q8_K(const uint8_t *w, const uint8_t *x, int64_t k) {
  uint8_t grid[4096], ks[128];
  wo_iq2xs_grid(grid);
  wo_ksigns_iq2xs(ks);
  const int64_t nb = k / QK_K;
  float sumf = 0.f;
  for (int64_t i = 0; i < nb; ++i) {
    const uint8_t *wr = w + i * IQ2_XS_BYTES;
    const uint8_t *xr = x + i * Q8_K_BYTES;
    const float d = wo_fp16_to_fp32(rd16(wr)) * rdf32(xr);
    const int8_t *q8 = (const int8_t *)(xr + 4);
    int32_t bsum = 0;
    for (int ib32 = 0; ib32 < 8; ++ib32) {
      const uint8_t sc = wr[66 + ib32];
      const int ls[2] = {2 * (sc & 0xf) + 1, 2 * (sc >> 4) + 1};
      for (int h = 0; h < 2; ++h) {
        int32_t sumi = 0;
        for (int l = 2 * h; l < 2 * h + 2; ++l) {
          const uint16_t q = rd16(wr + 2 + 2 * (4 * ib32 + l));
          const uint8_t *g = grid + 8 * (q & 511);
          const uint8_t signs = ks[q >> 9];
          for (int j = 0; j < 8; ++j) sumi += g[j] * q8[j] * (signs & (1 << j) ? -1 : 1);
          q8 += 8;
        }
        bsum += sumi * ls[h];
      }
    }
    sumf += d * bsum;
  }
  return 0.125f * sumf;
}

/* ggml_vec_dot_mxfp4_q8_0_generic, ggml-cpu/quants.c:247-276 */
float wo_vec_dot_mxfp4_q8_0(const uint8_t *w, const uint8_t *x, int64_t k) {
  int8_t kv[16];
  wo_kvalues_mxfp4(kv);
  const int64_t nb = k / QK_MXFP4;
  float sumf = 0;
  for (int64_t ib = 0; ib < nb; ++ib) {
    const uint8_t *wr = w + ib * MXFP4_BYTES;
    const uint8_t *xr = x + ib * Q8_0_BYTES;
    const int8_t *xq = (const int8_t *)(xr + 2);
    const float d = wo_fp16_to_fp32(rd16(xr)) * wo_e8m0_to_fp32_half(wr[0]);
    int sumi1 = 0, sumi2 = 0;
    for (int j = 0; j < QK_MXFP4 / 2; ++j) {
      sumi1 += xq[j] * kv[wr[1 + j] & 0xf];
      sumi2 += xq[j + QK_MXFP4 / 2] * kv[wr[1 + j] >> 4];
    }
    sumf += d * (sumi1 + sumi2);
  }
  return sumf;
}

/* ggml_vec_dot_q4_K_q8_K_generic, ggml-cpu/quants.c:645-718.  The eight
 * float lanes of `sums` are kept so the rounding order is GGML's. */
float wo_vec_dot_q4_K_q8_K(const uint8_t *w, const uint8_t *x, int64_t k) {
  const int64_t nb = k / QK_K;
  float sums[8] = {0};
  float sumf = 0;
  int8_t aux8[QK_K];
  for (int64_t i = 0; i < nb; ++i) {
    const uint8_t *wr = w + i * Q4_K_BYTES;
    const uint8_t *xr = x + i * Q8_K_BYTES;
    const uint8_t *q4 = wr + 16;
    const int8_t *q8 = (const int8_t *)(xr + 4);
    int32_t aux32[8] = {0};
    int8_t *a = aux8;
    for (int j = 0; j < QK_K / 64; ++j) {
      for (int l = 0; l < 32; ++l) a[l] = (int8_t)(q4[l] & 0xF);
      a += 32;
      for (int l = 0; l < 32; ++l) a[l] = (int8_t)(q4[l] >> 4);
      a += 32;
      q4 += 32;
    }
    uint8_t scales[8], mins[8];
    for (int j = 0; j < 8; ++j) scale_min_k4(j, wr + 4, &scales[j], &mins[j]);
    int sumi = 0;
    for (int j = 0; j < QK_K / 16; ++j) sumi += (int16_t)rd16(xr + 260 + 2 * j) * mins[j / 2];
    a = aux8;
    for (int j = 0; j < QK_K / 32; ++j) {
      const int32_t scale = scales[j];
      for (int c = 0; c < 4; ++c) {
        for (int l = 0; l < 8; ++l) aux32[l] += scale * (int16_t)(q8[l] * a[l]);
        q8 += 8;
        a += 8;
      }
    }
    const float d = wo_fp16_to_fp32(rd16(wr)) * rdf32(xr);
    for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
    const float dmin = wo_fp16_to_fp32(rd16(wr + 2)) * rdf32(xr);
    sumf -= dmin * sumi;
  }
  for (int l = 0; l < 8; ++l) sumf += sums[l];
  return sumf;
}

/* ggml_vec_dot_iq2_xxs_q8_K_generic, ggml-cpu/quants.c:855-895 */
float wo_vec_dot_iq2_xxs_q8_K(const uint8_t *w, const uint8_t *x, int64_t k) {
  uint8_t grid[2048], ks[128];
  wo_iq2xxs_grid(grid);
  wo_ksigns_iq2xs(ks);
  const int64_t nb = k / QK_K;
  float sumf = 0.f;
  for (int64_t i = 0; i < nb; ++i) {
    const uint8_t *wr = w + i * IQ2_XXS_BYTES;
    const uint8_t *xr = x + i * Q8_K_BYTES;
    const float d = wo_fp16_to_fp32(rd16(wr)) * rdf32(xr);
    const int8_t *q8 = (const int8_t *)(xr + 4);
    int32_t bsum = 0;
    for (int ib32 = 0; ib32 < QK_K / 32; ++ib32) {
      const uint8_t *qs = wr + 2 + 8 * ib32;
      const uint32_t meta = rd32(qs + 4);
      const uint32_t ls = 2 * (meta >> 28) + 1;
      int32_t sumi = 0;
      for (int l = 0; l < 4; ++l) {
        const uint8_t *g = grid + 8 * qs[l];
        const uint8_t signs = ks[(meta >> (7 * l)) & 127];
        for (int j = 0; j < 8; ++j) sumi += g[j] * q8[j] * (signs & (1u << j) ? -1 : 1);
        q8 += 8;
      }
      bsum += sumi * (int32_t)ls;
    }
    sumf += d * bsum;
  }
  return 0.125f * sumf;
}

/* dequantize_row_q6_K, ggml-quants.c:1881-1910: y = (d * sc) * q, two
 * rounded products in this order */
void wo_dequantize_row_q6_K(const uint8_t *x, float *y, int64_t k) {
  const int64_t nb = k / QK_K;
  for (int64_t i = 0; i < nb; ++i) {
    const uint8_t *r = x + i * Q6_K_BYTES;
    const float d = wo_fp16_to_fp32(rd16(r + 208));
    const uint8_t *ql = r, *qh = r + 128;
    const int8_t *sc = (const int8_t *)(r + 192);
    for (int n = 0; n < QK_K; n += 128) {
      for (int l = 0; l < 32; ++l) {
        const int is = l / 16;
        const int8_t q1 = (int8_t)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
        const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
        const int8_t q3 = (int8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
        const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        y[l] = d * sc[is] * q1;
        y[l + 32] = d * sc[is + 2] * q2;
        y[l + 64] = d * sc[is + 4] * q3;
        y[l + 96] = d * sc[is + 6] * q4;
      }
      y += 128;
      ql += 64;
      qh += 32;
      sc += 8;
    }
  }
}

/* dequantize_row_q5_K, ggml-quants.c:1673-1697: y = (d * sc) * q - dmin * m */
void wo_dequantize_row_q5_K(const uint8_t *x, float *y, int64_t k) {
  const int64_t nb = k / QK_K;
  for (int64_t i = 0; i < nb; ++i) {
    const uint8_t *r = x + i * Q5_K_BYTES;
    const uint8_t *ql = r + 48, *qh = r + 16;
    const float d = wo_fp16_to_fp32(rd16(r)), min = wo_fp16_to_fp32(rd16(r + 2));
    int is = 0;
    uint8_t sc, m, u1 = 1, u2 = 2;
    for (int j = 0; j < QK_K; j += 64) {
      scale_min_k4(is + 0, r + 4, &sc, &m);
      const float d1 = d * sc, m1 = min * m;
      scale_min_k4(is + 1, r + 4, &sc, &m);
      const float d2 = d * sc, m2 = min * m;
      for (int l = 0; l < 32; ++l) *y++ = d1 * ((ql[l] & 0xF) + (qh[l] & u1 ? 16 : 0)) - m1;
      for (int l = 0; l < 32; ++l) *y++ = d2 * ((ql[l] >> 4) + (qh[l] & u2 ? 16 : 0)) - m2;
      ql += 32;
      is += 2;
      u1 <<= 2;
      u2 <<= 2;
    }
  }
}

/* q of element e (0..255) of a Q5_K record, in [0, 31] */
static inline int q5_value(const uint8_t *r, int e) {
  const int j = e / 64, half = (e % 64) / 32, l = e % 32;
  const uint8_t b = r[48 + 32 * j + l];
  return (half ? b >> 4 : b & 0xF) | (((r[16 + l] >> (2 * j + half)) & 1) << 4);
}

/* ggml_vec_dot_q5_K_q8_K_generic, ggml-cpu/quants.c:720-798 */
float wo_vec_dot_q5_K_q8_K(const uint8_t *w, const uint8_t *x, int64_t k) {
  const int64_t nb = k / QK_K;
  float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float sumf = 0;
  int8_t aux8[QK_K];
  for (int64_t i = 0; i < nb; ++i) {
    const uint8_t *r = w + i * Q5_K_BYTES;
    const uint8_t *xr = x + i * Q8_K_BYTES;
    const int8_t *q8 = (const int8_t *)(xr + 4);
    for (int e = 0; e < QK_K; ++e) aux8[e] = (int8_t)q5_value(r, e);
    uint8_t scales[8], mins[8];
    for (int s = 0; s < 8; ++s) scale_min_k4(s, r + 4, &scales[s], &mins[s]);
    int sumi = 0;
    for (int j = 0; j < QK_K / 16; ++j) sumi += (int16_t)rd16(xr + 260 + 2 * j) * mins[j / 2];
    int32_t aux32[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int8_t *a = aux8;
    for (int j = 0; j < QK_K / 32; ++j) {
      const int32_t scale = scales[j];
      for (int part = 0; part < 4; ++part) {
        int16_t aux16[8];
        for (int l = 0; l < 8; ++l) aux16[l] = (int16_t)(q8[l] * a[l]);
        for (int l = 0; l < 8; ++l) aux32[l] += scale * aux16[l];
        q8 += 8;
        a += 8;
      }
    }
    const float d = wo_fp16_to_fp32(rd16(r)) * rdf32(xr);
    for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
    const float dmin = wo_fp16_to_fp32(rd16(r + 2)) * rdf32(xr);
    sumf -= dmin * sumi;
  }
  for (int l = 0; l < 8; ++l) sumf += sums[l];
  return sumf;
}

/* q of element e (0..255) of a Q6_K record, in [-32, 31] */
static inline int q6_value(const uint8_t *r, int e) {
  const int h = e / 128, i = e % 128, qq = i / 32, l = i % 32;
  const uint8_t b = r[64 * h + l + 32 * (qq & 1)];
  const int nib = qq < 2 ? (b & 0xF) : (b >> 4);
  const int hb = (r[128 + 32 * h + l] >> (2 * qq)) & 3;
  return (nib | (hb << 4)) - 32;
}

/* ggml_vec_dot_q6_K_q8_K_generic, ggml-cpu/quants.c:800-853: int32 lanes
 * aux32[8] per superblock, then sums[l] += (dw * dx) * aux32[l] */
float wo_vec_dot_q6_K_q8_K(const uint8_t *w, const uint8_t *x, int64_t k) {
  const int64_t nb = k / QK_K;
  float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int8_t aux8[QK_K];
  for (int64_t i = 0; i < nb; ++i) {
    const uint8_t *r = w + i * Q6_K_BYTES;
    const uint8_t *xr = x + i * Q8_K_BYTES;
    const int8_t *q8 = (const int8_t *)(xr + 4);
    for (int e = 0; e < QK_K; ++e) aux8[e] = (int8_t)q6_value(r, e);
    int32_t aux32[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int8_t *a = aux8;
    for (int j = 0; j < QK_K / 16; ++j) {
      const int scale = ((const int8_t *)(r + 192))[j];
      for (int half = 0; half < 2; ++half) {
        int16_t aux16[8];
        for (int l = 0; l < 8; ++l) aux16[l] = (int16_t)(q8[l] * a[l]);
        for (int l = 0; l < 8; ++l) aux32[l] += scale * aux16[l];
        q8 += 8;
        a += 8;
      }
    }
    const float d = wo_fp16_to_fp32(rd16(r + 208)) * rdf32(xr);
    for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
  }
  float sumf = 0;
  for (int l = 0; l < 8; ++l) sumf += sums[l];
  return sumf;
}

/* ------------------------------------------------------------------------
 * NVFP4: 64-element records, four UE4M3 sub-block scales then 32 bytes of
 * E2M1 codes; sub-block s holds elements 16 s + j (low nibble of byte
 * 4 + 8 s + j) and 16 s + 8 + j (high nibble), j < 8.
 * ---------------------------------------------------------------------- */

/* ggml_ue4m3_to_fp32 (ggml-impl.h:502-515): E4M3 without sign, 0x00 and
 * 0x7F read as zero, times one half (the E2M1 codebook is doubled). */
float wo_ue4m3_to_fp32(uint8_t x) {
  if (x == 0 || x == 0x7F) return 0.0f;
  const int e = (x >> 3) & 0xF, m = x & 7;
  const float raw = e == 0 ? ldexpf((float)m, -9) : ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return raw * 0.5f;
}

/* ggml_fp32_to_ue4m3 (ggml-impl.h:517-553): clamp to 448, round the
 * mantissa to 3 bits on the next bit (ties up), subnormals m * 2^-9. */
uint8_t wo_fp32_to_ue4m3(float x) {
  if (!(x > 0.0f)) return 0;
  if (x > 448.0f) x = 448.0f;
  uint32_t b;
  memcpy(&b, &x, 4);
  int e = (int)((b >> 23) & 0xFF) - 127 + 7;
  if (e <= 0) {
    int m = (int)(x * 512.0f + 0.5f);
    if (m > 7) m = 7;
    return m < 1 ? 0 : (uint8_t)m;
  }
  if (e >= 15) return 0x7E;
  int m = (int)((b >> 20) & 7) + (int)((b >> 19) & 1);
  if (m > 7) {
    m = 0;
    if (++e >= 15) return 0x7E;
  }
  return (uint8_t)((e << 3) | m);
}

void wo_ue4m3_table(float out[256]) {
  for (int c = 0; c < 256; ++c) out[c] = wo_ue4m3_to_fp32((uint8_t)c);
}

/* quantize_row_nvfp4_ref (ggml-quants.c:346-378) */
void wo_quantize_row_nvfp4(const float *x, uint8_t *y, int64_t k) {
  int8_t kv[16];
  wo_kvalues_mxfp4(kv);
  for (int64_t i = 0; i < k / QK_NVFP4; ++i) {
    uint8_t *rec = y + i * NVFP4_BYTES;
    for (int s = 0; s < 4; ++s) {
      const float *xb = x + i * QK_NVFP4 + 16 * s;
      float amax = 0.f;
      for (int j = 0; j < 16; ++j)
        if (amax < fabsf(xb[j])) amax = fabsf(xb[j]);
      rec[s] = wo_fp32_to_ue4m3(amax / 6.0f);
      const float d = wo_ue4m3_to_fp32(rec[s]);
      for (int j = 0; j < 8; ++j) {
        int best[2];
        for (int h = 0; h < 2; ++h) {
          const float v = xb[8 * h + j];
          int bi = 0;
          float be = fabsf(kv[0] * d - v);
          for (int c = 1; c < 16; ++c) {
            const float err = fabsf(kv[c] * d - v);
            if (err < be) {
              bi = c;
              be = err;
            }
          }
          best[h] = bi;
        }
        rec[4 + 8 * s + j] = (uint8_t)(best[0] | (best[1] << 4));
      }
    }
  }
}

/* dequantize_row_nvfp4 (ggml-quants.c:531-552) */
void wo_dequantize_row_nvfp4(const uint8_t *x, float *y, int64_t k) {
  int8_t kv[16];
  wo_kvalues_mxfp4(kv);
  for (int64_t i = 0; i < k / QK_NVFP4; ++i) {
    const uint8_t *rec = x + i * NVFP4_BYTES;
    for (int s = 0; s < 4; ++s) {
      const float d = wo_ue4m3_to_fp32(rec[s]);
      float *yb = y + i * QK_NVFP4 + 16 * s;
      for (int j = 0; j < 8; ++j) {
        yb[j] = kv[rec[4 + 8 * s + j] & 0x0F] * d;
        yb[j + 8] = kv[rec[4 + 8 * s + j] >> 4] * d;
      }
    }
  }
}

/* ggml_vec_dot_nvfp4_q8_0_generic (ggml-cpu/quants.c:279-313): sub-block s
 * of record i meets half s % 2 of Q8_0 block 2 i + s / 2. */
float wo_vec_dot_nvfp4_q8_0(const uint8_t *w, const uint8_t *x, int64_t k) {
  int8_t kv[16];
  wo_kvalues_mxfp4(kv);
  float sumf = 0.f;
  for (int64_t i = 0; i < k / QK_NVFP4; ++i) {
    const uint8_t *rec = w + i * NVFP4_BYTES;
    for (int s = 0; s < 4; ++s) {
      const uint8_t *xb = x + (2 * i + s / 2) * Q8_0_BYTES;
      const int8_t *xq = (const int8_t *)(xb + 2) + 16 * (s % 2);
      const float d = wo_ue4m3_to_fp32(rec[s]);
      const float dy = wo_fp16_to_fp32(rd16(xb));
      int lo = 0, hi = 0;
      for (int j = 0; j < 8; ++j) {
        const uint8_t q = rec[4 + 8 * s + j];
        lo += xq[j] * kv[q & 0xF];
        hi += xq[j + 8] * kv[q >> 4];
      }
      sumf += dy * d * (float)(lo + hi);
    }
  }
  return sumf;
}

/* ------------------------------------------------------------------------
 * MUL_MAT driver and fp64 re-accumulation
 * ---------------------------------------------------------------------- */
size_t wo_weight_row_bytes(int fmt, int64_t k) {
  switch (fmt) {
  case WO_Q4_0: return (size_t)(k / 32) * Q4_0_BYTES;
  case WO_Q4_K: return (size_t)(k / 256) * Q4_K_BYTES;
  case WO_IQ2_XXS: return (size_t)(k / 256) * IQ2_XXS_BYTES;
  case WO_MXFP4: return (size_t)(k / 32) * MXFP4_BYTES;
  case WO_Q6_K: return (size_t)(k / 256) * Q6_K_BYTES;
  case WO_Q5_K: return (size_t)(k / 256) * Q5_K_BYTES;
  case WO_NVFP4: return (size_t)(k / QK_NVFP4) * NVFP4_BYTES;
  case WO_Q4_1: return (size_t)(k / 32) * Q4_1_BYTES;
  case WO_IQ2_XS: return (size_t)(k / 256) * IQ2_XS_BYTES;
  }
  return 0;
}

size_t wo_act_row_bytes(int fmt, int64_t k) {
  if (fmt == WO_Q4_1) return (size_t)(k / 32) * Q8_1_BYTES;
  if (fmt == WO_Q4_0 || fmt == WO_MXFP4 || fmt == WO_NVFP4) return (size_t)(k / 32) * Q8_0_BYTES;
  return (size_t)(k / 256) * Q8_K_BYTES;
}

typedef float (*vec_dot_fn)(const uint8_t *, const uint8_t *, int64_t);
static vec_dot_fn select_vec_dot(int fmt) {
  switch (fmt) {
  case WO_Q4_0: return wo_vec_dot_q4_0_q8_0;
  case WO_Q4_K: return wo_vec_dot_q4_K_q8_K;
  case WO_IQ2_XXS: return wo_vec_dot_iq2_xxs_q8_K;
  case WO_MXFP4: return wo_vec_dot_mxfp4_q8_0;
  case WO_Q6_K: return wo_vec_dot_q6_K_q8_K;
  case WO_Q5_K: return wo_vec_dot_q5_K_q8_K;
  case WO_NVFP4: return wo_vec_dot_nvfp4_q8_0;
  case WO_Q4_1: return wo_vec_dot_q4_1_q8_1;
  case WO_IQ2_XS: return wo_vec_dot_iq2_xs_q8_K;
  }
  return 0;
}

/* the activation quantizer of a weight format: Q8_0, Q8_1 or Q8_K rows */
static void quantize_act(int fmt, const float *x, uint8_t *y, int64_t k) {
  if (fmt == WO_Q4_1)
    wo_quantize_row_q8_1(x, y, k);
  else if (fmt == WO_Q4_0 || fmt == WO_MXFP4 || fmt == WO_NVFP4)
    wo_quantize_row_q8_0(x, y, k);
  else
    wo_quantize_row_q8_K(x, y, k);
}

int wo_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void wo_mul_mat_q(int fmt, const uint8_t *W, const uint8_t *Xq, float *Y, int64_t N, int64_t K,
                  int64_t M, int nthreads) {
  const vec_dot_fn dot = select_vec_dot(fmt);
  const size_t wrow = wo_weight_row_bytes(fmt, K), xrow = wo_act_row_bytes(fmt, K);
  if (nthreads <= 0) nthreads = wo_max_threads();
  (void)nthreads;
#pragma omp parallel for num_threads(nthreads) schedule(static) collapse(2)
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) Y[m * N + n] = dot(W + n * wrow, Xq + m * xrow, K);
}

void wo_mul_mat(int fmt, const uint8_t *W, const float *X, uint8_t *Xq, float *Y, int64_t N,
                int64_t K, int64_t M, int nthreads) {
  const size_t xrow = wo_act_row_bytes(fmt, K);
  if (nthreads <= 0) nthreads = wo_max_threads();
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (int64_t m = 0; m < M; ++m) quantize_act(fmt, X + m * K, Xq + m * xrow, K);
  wo_mul_mat_q(fmt, W, Xq, Y, N, K, M, nthreads);
}

/* ggml_compute_forward_mul_mat's schedule, ggml-cpu/ggml-cpu.c:1313-1443
 * (from_float split by blocks, ggml_barrier, chunk plan, shared counter) and
 * ggml_compute_forward_mul_mat_one_chunk's 16 x 16 blocking, :1155-1243.
 * 2-D case: ne1 = M activation rows, ne0 = N outputs per row. */
void wo_mul_mat_ggml(int fmt, const uint8_t *W, const float *X, uint8_t *Xq, float *Y,
                     int64_t N, int64_t K, int64_t M, int nthreads) {
  const vec_dot_fn dot = select_vec_dot(fmt);
  const int q80 = (fmt == WO_Q4_0 || fmt == WO_MXFP4 || fmt == WO_NVFP4 || fmt == WO_Q4_1);
  const int64_t bs = q80 ? QK8_0 : QK_K;
  const size_t blk_bytes = fmt == WO_Q4_1 ? Q8_1_BYTES : q80 ? Q8_0_BYTES : Q8_K_BYTES;
  const size_t wrow = wo_weight_row_bytes(fmt, K), xrow = wo_act_row_bytes(fmt, K);
  if (nthreads <= 0) nthreads = wo_max_threads();
  _Atomic int64_t next_chunk = 0;
#pragma omp parallel num_threads(nthreads)
  {
    const int nth = omp_get_num_threads(), ith = omp_get_thread_num();
    const int64_t nb = K / bs;
    for (int64_t m = 0; m < M; ++m) {
      const int64_t b0 = ith * nb / nth, b1 = (ith + 1) * nb / nth;
      if (b1 > b0) quantize_act(fmt, X + m * K + b0 * bs, Xq + m * xrow + b0 * blk_bytes, (b1 - b0) * bs);
    }
    if (ith == 0) next_chunk = nth;  /* every thread starts at its own index */
#pragma omp barrier
    const int64_t nr0 = N, nr1 = M;
    const int64_t chunk_size = (nr0 == 1 || nr1 == 1) ? 64 : 16;
    int64_t nchunk0 = (nr0 + chunk_size - 1) / chunk_size;
    int64_t nchunk1 = (nr1 + chunk_size - 1) / chunk_size;
    if (nchunk0 * nchunk1 < (int64_t)nth * 4) {
      nchunk0 = nr0 > nr1 ? nth : 1;
      nchunk1 = nr0 > nr1 ? 1 : nth;
    }
    const int64_t dr0 = (nr0 + nchunk0 - 1) / nchunk0, dr1 = (nr1 + nchunk1 - 1) / nchunk1;
    int64_t chunk = ith;
    while (chunk < nchunk0 * nchunk1) {
      const int64_t i0 = chunk % nchunk0, i1 = chunk / nchunk0;
      const int64_t r0a = dr0 * i0, r0b = r0a + dr0 < nr0 ? r0a + dr0 : nr0;
      const int64_t r1a = dr1 * i1, r1b = r1a + dr1 < nr1 ? r1a + dr1 : nr1;
      float tmp[16];
      for (int64_t bb1 = r1a; bb1 < r1b; bb1 += 16)
        for (int64_t bb0 = r0a; bb0 < r0b; bb0 += 16)
          for (int64_t r1 = bb1; r1 < bb1 + 16 && r1 < r1b; ++r1) {
            int64_t r0 = bb0;
            for (; r0 < bb0 + 16 && r0 < r0b; ++r0) tmp[r0 - bb0] = dot(W + r0 * wrow, Xq + r1 * xrow, K);
            memcpy(Y + r1 * N + bb0, tmp, (size_t)(r0 - bb0) * sizeof(float));
          }
      if (nth >= nchunk0 * nchunk1) break;
      chunk = __atomic_fetch_add(&next_chunk, 1, __ATOMIC_RELAXED);
    }
  }
}

void wo_evict(uint8_t *buf, size_t bytes) {
  for (size_t i = 0; i < bytes; i += 64) buf[i] = (uint8_t)(buf[i] + 1);
}

int64_t wo_int_partials(int fmt, const uint8_t *w, const uint8_t *x, int64_t k, int32_t *out) {
  int64_t n = 0;
  if (fmt == WO_Q4_0 || fmt == WO_MXFP4) {
    int8_t kv[16];
    wo_kvalues_mxfp4(kv);
    const int64_t nb = k / 32;
    for (int64_t ib = 0; ib < nb; ++ib) {
      const uint8_t *wr = w + ib * (fmt == WO_Q4_0 ? Q4_0_BYTES : MXFP4_BYTES);
      const uint8_t *qs = wr + (fmt == WO_Q4_0 ? 2 : 1);
      const int8_t *xq = (const int8_t *)(x + ib * Q8_0_BYTES + 2);
      int32_t s = 0;
      for (int j = 0; j < 16; ++j) {
        const int lo = qs[j] & 0xF, hi = qs[j] >> 4;
        const int v0 = fmt == WO_Q4_0 ? lo - 8 : kv[lo];
        const int v1 = fmt == WO_Q4_0 ? hi - 8 : kv[hi];
        s += v0 * xq[j] + v1 * xq[j + 16];
      }
      out[n++] = s;
    }
  } else if (fmt == WO_Q4_1) {
    for (int64_t ib = 0; ib < k / 32; ++ib) {
      const uint8_t *qs = w + ib * Q4_1_BYTES + 4;
      const int8_t *xq = (const int8_t *)(x + ib * Q8_1_BYTES + 4);
      int32_t s = 0;
      for (int j = 0; j < 16; ++j) s += (qs[j] & 0xF) * xq[j] + (qs[j] >> 4) * xq[j + 16];
      out[n++] = s;
    }
  } else if (fmt == WO_IQ2_XS) {
    /* one int32 per 16-element half group: the partial its 4-bit scale
     * multiplies */
    uint8_t grid[4096], ks[128];
    wo_iq2xs_grid(grid);
    wo_ksigns_iq2xs(ks);
    for (int64_t i = 0; i < k / QK_K; ++i) {
      const uint8_t *wr = w + i * IQ2_XS_BYTES;
      const int8_t *q8 = (const int8_t *)(x + i * Q8_K_BYTES + 4);
      for (int h = 0; h < 16; ++h) {
        int32_t s = 0;
        for (int l = 2 * h; l < 2 * h + 2; ++l) {
          const uint16_t q = rd16(wr + 2 + 2 * l);
          for (int j = 0; j < 8; ++j)
            s += grid[8 * (q & 511) + j] * q8[8 * l + j] * ((ks[q >> 9] >> j) & 1 ? -1 : 1);
        }
        out[n++] = s;
      }
    }
  } else if (fmt == WO_NVFP4) {
    /* one int32 per 16-element sub-block */
    int8_t kv[16];
    wo_kvalues_mxfp4(kv);
    for (int64_t i = 0; i < k / QK_NVFP4; ++i) {
      const uint8_t *rec = w + i * NVFP4_BYTES;
      for (int s = 0; s < 4; ++s) {
        const int8_t *xq = (const int8_t *)(x + (2 * i + s / 2) * Q8_0_BYTES + 2) + 16 * (s % 2);
        int32_t p = 0;
        for (int j = 0; j < 8; ++j) {
          const uint8_t q = rec[4 + 8 * s + j];
          p += xq[j] * kv[q & 0xF] + xq[j + 8] * kv[q >> 4];
        }
        out[n++] = p;
      }
    }
  } else if (fmt == WO_Q4_K || fmt == WO_Q5_K) {
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; ++i) {
      const uint8_t *wr = w + i * (fmt == WO_Q4_K ? Q4_K_BYTES : Q5_K_BYTES);
      const uint8_t *xr = x + i * Q8_K_BYTES;
      const int8_t *q8 = (const int8_t *)(xr + 4);
      int32_t mn = 0;
      for (int s = 0; s < 8; ++s) {
        uint8_t sc, m;
        scale_min_k4(s, wr + 4, &sc, &m);
        const uint8_t *q4 = wr + 16 + 32 * (s / 2);
        int32_t p = 0;
        for (int l = 0; l < 32; ++l) {
          const int v = fmt == WO_Q5_K ? q5_value(wr, 32 * s + l) : (s & 1) ? (q4[l] >> 4) : (q4[l] & 0xF);
          p += v * q8[32 * s + l];
        }
        out[n++] = p;
        mn += m * ((int16_t)rd16(xr + 260 + 4 * s) + (int16_t)rd16(xr + 262 + 4 * s));
      }
      out[n++] = mn;
    }
  } else if (fmt == WO_IQ2_XXS) {
    uint8_t grid[2048], ks[128];
    wo_iq2xxs_grid(grid);
    wo_ksigns_iq2xs(ks);
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; ++i) {
      const uint8_t *wr = w + i * IQ2_XXS_BYTES;
      const int8_t *q8 = (const int8_t *)(x + i * Q8_K_BYTES + 4);
      /* one int32 per 32-element group: its partial times 2 ls + 1 */
      for (int g = 0; g < 8; ++g) {
        const uint8_t *qs = wr + 2 + 8 * g;
        const uint32_t meta = rd32(qs + 4);
        int32_t s = 0;
        for (int l = 0; l < 4; ++l) {
          const uint8_t sg = ks[(meta >> (7 * l)) & 127];
          for (int j = 0; j < 8; ++j)
            s += grid[8 * qs[l] + j] * q8[32 * g + 8 * l + j] * ((sg >> j) & 1 ? -1 : 1);
        }
        out[n++] = s * (int32_t)(2 * (meta >> 28) + 1);
      }
    }
  } else if (fmt == WO_Q6_K) {
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; ++i) {
      const uint8_t *wr = w + i * Q6_K_BYTES;
      const int8_t *q8 = (const int8_t *)(x + i * Q8_K_BYTES + 4);
      for (int g = 0; g < 16; ++g) {
        int32_t p = 0;
        for (int l = 0; l < 16; ++l) p += q6_value(wr, 16 * g + l) * q8[16 * g + l];
        out[n++] = p;
      }
    }
  }
  return n;
}

void wo_mul_mat_f64(int fmt, const uint8_t *W, const uint8_t *Xq, double *E, double *A, int64_t N,
                    int64_t K, int64_t M, int nthreads) {
  const size_t wrow = wo_weight_row_bytes(fmt, K), xrow = wo_act_row_bytes(fmt, K);
  if (nthreads <= 0) nthreads = wo_max_threads();
#pragma omp parallel for num_threads(nthreads) schedule(static) collapse(2)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      int32_t parts[9 * (65536 / 256) + 8];
      const uint8_t *w = W + n * wrow;
      const uint8_t *x = Xq + m * xrow;
      double e = 0, a = 0;
      if (fmt == WO_Q4_1) {
        for (int64_t base = 0; base < K; base += 8192) {
          const int64_t kk = K - base < 8192 ? K - base : 8192;
          const int64_t nbase = base / 32;
          const int64_t np = wo_int_partials(fmt, w + nbase * Q4_1_BYTES, x + nbase * Q8_1_BYTES, kk, parts);
          for (int64_t b = 0; b < np; ++b) {
            const uint8_t *wr = w + (nbase + b) * Q4_1_BYTES, *xr = x + (nbase + b) * Q8_1_BYTES;
            const double t1 = (double)wo_fp16_to_fp32(rd16(wr)) * wo_fp16_to_fp32(rd16(xr)) * parts[b];
            const double t2 = (double)wo_fp16_to_fp32(rd16(wr + 2)) * wo_fp16_to_fp32(rd16(xr + 2));
            e += t1 + t2;
            a += fabs(t1) + fabs(t2);
          }
        }
      } else if (fmt == WO_IQ2_XS) {
        for (int64_t i = 0; i < K / QK_K; ++i) {
          const uint8_t *wr = w + i * IQ2_XS_BYTES;
          const uint8_t *xr = x + i * Q8_K_BYTES;
          wo_int_partials(fmt, wr, xr, QK_K, parts);
          const double f = 0.125 * wo_fp16_to_fp32(rd16(wr)) * (double)rdf32(xr);
          for (int h = 0; h < 16; ++h) {
            const double t = f * (double)((int64_t)(2 * ((wr[66 + h / 2] >> (4 * (h & 1))) & 0xf) + 1) * parts[h]);
            e += t;
            a += fabs(t);
          }
        }
      } else if (fmt == WO_Q4_0 || fmt == WO_MXFP4) {
        for (int64_t base = 0; base < K; base += 8192) {
          const int64_t kk = K - base < 8192 ? K - base : 8192;
          const int64_t nbase = base / 32;
          const int64_t np = wo_int_partials(
              fmt, w + nbase * (fmt == WO_Q4_0 ? Q4_0_BYTES : MXFP4_BYTES), x + nbase * Q8_0_BYTES,
              kk, parts);
          for (int64_t b = 0; b < np; ++b) {
            const uint8_t *wr = w + (nbase + b) * (fmt == WO_Q4_0 ? Q4_0_BYTES : MXFP4_BYTES);
            const double dx = wo_fp16_to_fp32(rd16(x + (nbase + b) * Q8_0_BYTES));
            const double dw = fmt == WO_Q4_0 ? wo_fp16_to_fp32(rd16(wr)) : wo_e8m0_to_fp32_half(wr[0]);
            const double t = dw * dx * parts[b];
            e += t;
            a += fabs(t);
          }
        }
      } else if (fmt == WO_NVFP4) {
        for (int64_t i = 0; i < K / QK_NVFP4; ++i) {
          const uint8_t *wr = w + i * NVFP4_BYTES;
          wo_int_partials(fmt, wr, x + 2 * i * Q8_0_BYTES, QK_NVFP4, parts);
          for (int s = 0; s < 4; ++s) {
            const double dy = wo_fp16_to_fp32(rd16(x + (2 * i + s / 2) * Q8_0_BYTES));
            const double t = (double)wo_ue4m3_to_fp32(wr[s]) * dy * parts[s];
            e += t;
            a += fabs(t);
          }
        }
      } else if (fmt == WO_Q6_K) {
        const int64_t nb = K / QK_K;
        for (int64_t i = 0; i < nb; ++i) {
          const uint8_t *wr = w + i * Q6_K_BYTES;
          const uint8_t *xr = x + i * Q8_K_BYTES;
          wo_int_partials(fmt, wr, xr, QK_K, parts);
          const double f = (double)wo_fp16_to_fp32(rd16(wr + 208)) * (double)rdf32(xr);
          for (int g = 0; g < 16; ++g) {
            const double t = f * (double)((int64_t)((const int8_t *)(wr + 192))[g] * parts[g]);
            e += t;
            a += fabs(t);
          }
        }
      } else {
        const int64_t nb = K / QK_K;
        for (int64_t i = 0; i < nb; ++i) {
          const uint8_t *wr = w + i * (fmt == WO_Q4_K ? Q4_K_BYTES : fmt == WO_Q5_K ? Q5_K_BYTES : IQ2_XXS_BYTES);
          const uint8_t *xr = x + i * Q8_K_BYTES;
          wo_int_partials(fmt, wr, xr, QK_K, parts);
          const double dx = rdf32(xr);
          const double dw = wo_fp16_to_fp32(rd16(wr));
          if (fmt == WO_Q4_K || fmt == WO_Q5_K) {
            const double dmin = wo_fp16_to_fp32(rd16(wr + 2));
            for (int s = 0; s < 8; ++s) {
              uint8_t sc, mm;
              scale_min_k4(s, wr + 4, &sc, &mm);
              const int32_t bs = (int16_t)rd16(xr + 260 + 4 * s) + (int16_t)rd16(xr + 262 + 4 * s);
              const double t1 = dw * dx * (double)((int64_t)sc * parts[s]), t2 = dmin * dx * (double)(mm * bs);
              e += t1 - t2;
              a += fabs(t1) + fabs(t2);
            }
          } else {
            for (int g = 0; g < 8; ++g) {
              const double t = 0.125 * dw * dx * (double)parts[g];
              e += t;
              a += fabs(t);
            }
          }
        }
      }
      E[m * N + n] = e;
      A[m * N + n] = a;
    }
  }
}
