// GGML's MUL_MAT op on the quantized mul_mat kernels: the contract of
// ggml_compute_forward_mul_mat (ggml-cpu/ggml-cpu.c:1245-1443) for src0 of
// type Q4_0, Q4_K, Q5_K, Q6_K, IQ2_XXS, MXFP4 or NVFP4, so the kernels can sit under a
// ggml-style graph executor.
//
//   dst[i3, i2, i1, i0] = vec_dot(src0 row i0 of plane (i2 / r2, i3 / r3),
//                                 src1 row (i1, i2, i3) quantized to the
//                                 type's vec_dot_type),
//   r2 = ne12 / ne02, r3 = ne13 / ne03 (src0 broadcast over src1's planes).
//
// Strides are GGML's byte strides: src0 rows nb01 apart (nb00 the block
// size: not transposed), src1 rows nb11 apart (nb10 = 4), dst rows nb1
// apart (nb0 = 4).  An F32 src1 is quantized into the caller's work buffer
// as GGML does (rows contiguous, planes nbw2 = ne11 rows and nbw3 = ne12
// planes apart, :1309-1340), so wdata ends holding what GGML's would; a
// src1 already of the vec_dot_type is read in place.  GGML_ASSERT
// conditions become error returns: nothing is launched.
//
// IQ2_XXS and MXFP4 need GGML's tables, which GGML compiles in rather than
// passing; this file holds device copies built at compile time from the
// format definitions (iq2xxs_grid as its kgrid_2bit_256 codes,
// ggml-quants.c:2787-2804, expanded through {0x08, 0x19, 0x2b};
// ksigns_iq2xs = i | parity(i) << 7 as +-1 bytes; kvalues_mxfp4 and
// ggml_e8m0_to_fp32_half, ggml-common.h:1116-1118, ggml-impl.h:477-495).
#include <mutex>
#include <vector>

#include "kernels.h"
#include "runtime.h"
#include "weft_common.h"
#include "weft_hip.h"

namespace weft {
namespace {

// ---------------------------------------------------------------- types
struct TypeInfo {
  int32_t type;
  int64_t blck;
  size_t size;
  int32_t vec_dot;  // -1: not a MUL_MAT src0 type here
};

// ggml.c type_traits (blck_size, type_size) and ggml-cpu.c type_traits_cpu
// (vec_dot_type, :230-239, :277-281, :301-309, :317-321, :327-331) of this
// path's types
constexpr TypeInfo kTypes[] = {
    {WEFT_GGML_TYPE_F32, 1, 4, -1},
    {WEFT_GGML_TYPE_Q4_0, 32, kQ4_0Bytes, WEFT_GGML_TYPE_Q8_0},
    {WEFT_GGML_TYPE_Q8_0, 32, kQ8_0Bytes, -1},
    {WEFT_GGML_TYPE_Q4_K, 256, kQ4_KBytes, WEFT_GGML_TYPE_Q8_K},
    {WEFT_GGML_TYPE_Q5_K, 256, kQ5_KBytes, WEFT_GGML_TYPE_Q8_K},
    {WEFT_GGML_TYPE_Q6_K, 256, kQ6_KBytes, WEFT_GGML_TYPE_Q8_K},
    {WEFT_GGML_TYPE_Q8_K, 256, kQ8_KBytes, -1},
    {WEFT_GGML_TYPE_IQ2_XXS, 256, kIq2xxsBytes, WEFT_GGML_TYPE_Q8_K},
    {WEFT_GGML_TYPE_MXFP4, 32, kMxfp4Bytes, WEFT_GGML_TYPE_Q8_0},
    {WEFT_GGML_TYPE_NVFP4, 64, kNvfp4Bytes, WEFT_GGML_TYPE_Q8_0},
    {WEFT_GGML_TYPE_Q4_1, 32, kQ4_1Bytes, WEFT_GGML_TYPE_Q8_1},
    {WEFT_GGML_TYPE_Q8_1, 32, kQ8_1Bytes, -1},
    {WEFT_GGML_TYPE_IQ2_XS, 256, kIq2xsBytes, WEFT_GGML_TYPE_Q8_K},
};

constexpr int32_t kGgmlTypeI32 = 26;  // GGML_TYPE_I32

const TypeInfo* info(int32_t type) {
  for (const TypeInfo& t : kTypes)
    if (t.type == type) return &t;
  return nullptr;
}

}  // namespace

// ---------------------------------------------------------------- tables
struct GgmlTables {
  int8_t grid[256 * 8];
  int8_t signs[128 * 8];
  int8_t codebook[16];
  float scale[256];  // E8M0 (MXFP4), ggml_e8m0_to_fp32_half
  float ue4m3[256];  // UE4M3 (NVFP4), ggml_ue4m3_to_fp32 (ggml-impl.h:502-515)
  int8_t grid_xs[512 * 8];  // iq2xs_grid (ggml-common.h:617-746)
};

constexpr uint16_t kGridCodes[256] = {
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

// iq2xs_grid as two bits per lane (0x08, 0x19, 0x2b -> 0, 1, 2), lane 0 lowest
constexpr uint16_t kGridXsCodes[512] = {
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

constexpr GgmlTables make_tables() {
  GgmlTables t{};
  constexpr int8_t lane_value[4] = {0x08, 0x19, 0x2b, 0x00};
  for (int i = 0; i < 256; ++i)
    for (int j = 0; j < 8; ++j) t.grid[8 * i + j] = lane_value[(kGridCodes[i] >> (2 * j)) & 3];
  for (int i = 0; i < 512; ++i)
    for (int j = 0; j < 8; ++j) t.grid_xs[8 * i + j] = lane_value[(kGridXsCodes[i] >> (2 * j)) & 3];
  for (int i = 0; i < 128; ++i) {
    int parity = 0;
    for (int b = 0; b < 7; ++b) parity ^= (i >> b) & 1;
    const int ks = i | parity << 7;
    for (int j = 0; j < 8; ++j) t.signs[8 * i + j] = (ks >> j) & 1 ? -1 : 1;
  }
  constexpr int8_t kv[8] = {0, 1, 2, 3, 4, 6, 8, 12};  // twice E2M1
  for (int i = 0; i < 16; ++i) t.codebook[i] = (int8_t)(i & 8 ? -kv[i & 7] : kv[i & 7]);
  for (int e = 0; e < 256; ++e)
    t.scale[e] = __builtin_bit_cast(float, e < 2 ? 0x00200000u << e : (uint32_t)(e - 1) << 23);
  for (int c = 0; c < 256; ++c) {  // half of E4M3 without sign; 0x00 and 0x7F are zero
    const int e = (c >> 3) & 15, m = c & 7;
    t.ue4m3[c] = c == 0 || c == 0x7F ? 0.0f
                 : e == 0            ? (float)m * (1.0f / 1024.0f)
                                     : (float)(8 + m) * __builtin_bit_cast(float, (uint32_t)(116 + e) << 23);
  }
  return t;
}


// External linkage and not const: the device code object must keep the
// symbol the host side registers (an internal const object that no kernel
// reads is dropped from the device code, and its address cannot be looked up).
__device__ GgmlTables g_weft_ggml_tables = make_tables();

namespace {

// Device address of the tables on the current device (one copy per device).
const GgmlTables* device_tables() {
  static std::mutex mu;
  static std::vector<const GgmlTables*> addr;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)addr.size() <= dev) addr.resize(dev + 1, nullptr);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_weft_ggml_tables)) != hipSuccess) return nullptr;
    addr[dev] = static_cast<const GgmlTables*>(p);
  }
  return addr[dev];
}

// The work buffer of weft_ggml_mul_mat_id_noalloc: one copy per device, held
// until the process ends.  Host code never names it past the lookup below:
// there the name is a host-side stand-in, and each device's copy lives at
// the address hipGetSymbolAddress returns with that device current.  Every
// call on a device shares its copy (a call's quantized src1 and expert
// grouping are written in full before they are read, so nothing needs to
// start at zero); calls that overlap on one device race on it.
static __device__ __align__(256) uint8_t scratch[WEFT_GGML_NOALLOC_SCRATCH_BYTES];

// Device address of the current device's scratch, resolved on the first call
// on that device; null (and the error recorded) if the lookup fails.
uint8_t* noalloc_scratch() {
  static std::mutex mu;
  static std::vector<uint8_t*> addr;
  int dev = 0;
  const hipError_t ge = hipGetDevice(&dev);
  if (ge != hipSuccess) {
    set_error(ge);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if ((int)addr.size() <= dev) addr.resize(dev + 1, nullptr);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) {
      set_error(e);
      return nullptr;
    }
    addr[dev] = static_cast<uint8_t*>(p);
  }
  return addr[dev];
}

// ---------------------------------------------------------------- the op
size_t row_size(const TypeInfo* t, int64_t ne) { return t->size * (size_t)(ne / t->blck); }

hipError_t fail(hipError_t e) {
  set_error(e);
  return e;
}

bool nonneg(const weft_ggml_tensor* t) {
  for (int i = 0; i < 4; ++i)
    if (t->ne[i] < 0) return false;
  return true;
}

hipError_t mul_mat(const weft_ggml_tensor* s0, const weft_ggml_tensor* s1, const weft_ggml_tensor* d,
                   void* wdata, size_t wsize) {
  if (s0 == nullptr || s1 == nullptr || d == nullptr) return fail(hipErrorInvalidValue);
  const TypeInfo* t0 = info(s0->type);
  const TypeInfo* t1 = info(s1->type);
  if (t0 == nullptr || t0->vec_dot < 0 || t1 == nullptr || d->type != WEFT_GGML_TYPE_F32)
    return fail(hipErrorNotSupported);
  const TypeInfo* vd = info(t0->vec_dot);
  if (s1->type != WEFT_GGML_TYPE_F32 && s1->type != t0->vec_dot) return fail(hipErrorNotSupported);
  if (!nonneg(s0) || !nonneg(s1) || !nonneg(d)) return fail(hipErrorInvalidValue);
  // an empty dst is skipped before the op runs (ggml_compute_forward,
  // ggml-cpu.c:1705)
  if (d->ne[0] == 0 || d->ne[1] == 0 || d->ne[2] == 0 || d->ne[3] == 0) return hipSuccess;
  // ggml_can_mul_mat (ggml.c:3234-3240) and the op's asserts (ggml-cpu.c:1266-1282)
  const int64_t K = s0->ne[0], N = s0->ne[1];
  if (s1->ne[0] != K || s0->ne[2] == 0 || s0->ne[3] == 0 || s1->ne[2] % s0->ne[2] != 0 ||
      s1->ne[3] % s0->ne[3] != 0 || d->ne[0] != N || d->ne[1] != s1->ne[1] ||
      d->ne[2] != s1->ne[2] || d->ne[3] != s1->ne[3] || K % t0->blck != 0 ||
      s0->nb[0] != t0->size || s1->nb[0] != t1->size || d->nb[0] != sizeof(float) ||
      d->nb[0] > d->nb[1] || d->nb[1] > d->nb[2] || d->nb[2] > d->nb[3])
    return fail(hipErrorInvalidValue);
  const int64_t M = s1->ne[1], ne12 = s1->ne[2], ne13 = s1->ne[3];
  if (K == 0 || N == 0 || M == 0 || ne12 == 0 || ne13 == 0) return hipSuccess;
  if (d->nb[1] % 4 != 0 || (s1->type == WEFT_GGML_TYPE_F32 && s1->nb[1] % 4 != 0))
    return fail(hipErrorInvalidValue);
  const bool quantize = s1->type == WEFT_GGML_TYPE_F32;
  const size_t nbw1 = row_size(vd, K);
  if (quantize) {
    if (wdata == nullptr || !aligned(wdata, 4) || wsize < nbw1 * (size_t)(M * ne12 * ne13))
      return fail(hipErrorInvalidValue);
  } else if (M > 1 && s1->nb[1] != nbw1) {
    return fail(hipErrorNotSupported);  // quantized src1 rows must be packed
  }
  const GgmlTables* tab = nullptr;
  if (s0->type == WEFT_GGML_TYPE_IQ2_XXS || s0->type == WEFT_GGML_TYPE_MXFP4 ||
      s0->type == WEFT_GGML_TYPE_NVFP4 || s0->type == WEFT_GGML_TYPE_IQ2_XS) {
    tab = device_tables();
    if (tab == nullptr) return fail(hipErrorInvalidDevice);
  }
  const int64_t r2 = ne12 / s0->ne[2], r3 = ne13 / s0->ne[3];
  const RowStrides st{s0->nb[1], quantize ? s1->nb[1] / 4 : (size_t)K, d->nb[1] / 4};

  // one call over all planes when src0 is one matrix and src1 / dst planes
  // continue their rows (the usual batched activation)
  int64_t mm = M, p2 = ne12, p3 = ne13;
  if (s0->ne[2] == 1 && s0->ne[3] == 1 && (!quantize || (s1->nb[2] == (size_t)M * s1->nb[1] &&
                                                         s1->nb[3] == (size_t)ne12 * s1->nb[2])) &&
      (quantize || (s1->nb[2] == (size_t)M * nbw1 && s1->nb[3] == (size_t)ne12 * s1->nb[2])) &&
      d->nb[2] == (size_t)M * d->nb[1] && d->nb[3] == (size_t)ne12 * d->nb[2]) {
    mm = M * ne12 * ne13;
    p2 = p3 = 1;
  }
  const size_t nbw2 = nbw1 * (size_t)M, nbw3 = nbw2 * (size_t)ne12;
  for (int64_t i13 = 0; i13 < p3; ++i13)
    for (int64_t i12 = 0; i12 < p2; ++i12) {
      const uint8_t* W = static_cast<const uint8_t*>(s0->data) + (size_t)(i12 / r2) * s0->nb[2] +
                         (size_t)(i13 / r3) * s0->nb[3];
      const uint8_t* src1 =
          static_cast<const uint8_t*>(s1->data) + (size_t)i12 * s1->nb[2] + (size_t)i13 * s1->nb[3];
      float* Y = reinterpret_cast<float*>(static_cast<uint8_t*>(d->data) + (size_t)i12 * d->nb[2] +
                                          (size_t)i13 * d->nb[3]);
      const size_t n = (size_t)N, k = (size_t)K, m = (size_t)mm;
      if (quantize) {
        const float* X = reinterpret_cast<const float*>(src1);
        uint8_t* Xq = static_cast<uint8_t*>(wdata) + (size_t)i12 * nbw2 + (size_t)i13 * nbw3;
        switch (s0->type) {
          case WEFT_GGML_TYPE_Q4_0: mul_mat_q4_0(W, X, Xq, Y, n, k, m, st); break;
          case WEFT_GGML_TYPE_Q4_K: mul_mat_q4k(W, X, Xq, Y, n, k, m, st); break;
          case WEFT_GGML_TYPE_Q6_K: mul_mat_q6k(W, X, Xq, Y, n, k, m, st); break;
          case WEFT_GGML_TYPE_Q5_K: mul_mat_q5k(W, X, Xq, Y, n, k, m, st); break;
          case WEFT_GGML_TYPE_NVFP4:
            mul_mat_nvfp4(W, X, Xq, tab->codebook, tab->ue4m3, Y, n, k, m, st);
            break;
          case WEFT_GGML_TYPE_IQ2_XXS:
            mul_mat_iq2_xxs(W, X, Xq, tab->grid, tab->signs, Y, n, k, m, st);
            break;
          case WEFT_GGML_TYPE_Q4_1: mul_mat_q4_1(W, X, Xq, Y, n, k, m, st); break;
          case WEFT_GGML_TYPE_IQ2_XS:
            mul_mat_iq2_xs(W, X, Xq, tab->grid_xs, tab->signs, Y, n, k, m, st);
            break;
          default: mul_mat_mxfp4(W, X, Xq, tab->codebook, tab->scale, Y, n, k, m, st); break;
        }
      } else {
        switch (s0->type) {
          case WEFT_GGML_TYPE_Q4_0: decode_quantized(0, W, src1, nullptr, nullptr, Y, n, k, m, st); break;
          case WEFT_GGML_TYPE_Q4_K: mul_mat_q4k_quantized(W, src1, Y, n, k, m, st); break;
          case WEFT_GGML_TYPE_Q6_K: mul_mat_q6k_quantized(W, src1, Y, n, k, m, st); break;
          case WEFT_GGML_TYPE_Q5_K: mul_mat_q5k_quantized(W, src1, Y, n, k, m, st); break;
          case WEFT_GGML_TYPE_NVFP4:
            decode_quantized(5, W, src1, tab->codebook, tab->ue4m3, Y, n, k, m, st);
            break;
          case WEFT_GGML_TYPE_IQ2_XXS:
            mul_mat_iq2_xxs_quantized(W, src1, tab->grid, tab->signs, Y, n, k, m, st);
            break;
          case WEFT_GGML_TYPE_Q4_1: decode_quantized(6, W, src1, nullptr, nullptr, Y, n, k, m, st); break;
          case WEFT_GGML_TYPE_IQ2_XS:
            mul_mat_iq2_xs_quantized(W, src1, tab->grid_xs, tab->signs, Y, n, k, m, st);
            break;
          default: decode_quantized(1, W, src1, tab->codebook, tab->scale, Y, n, k, m, st); break;
        }
      }
      if (pending_error() != hipSuccess) return pending_error();
    }
  return pending_error();
}

// GGML_OP_MUL_MAT_ID (ggml-cpu.c:1454-1698; shape rules of ggml_mul_mat_id,
// ggml.c:3293-3317): src0 holds n_as = ne02 expert matrices, ids (I32,
// n_ids x n_tokens) picks an expert per (slot, token), src1 row
// (s % ne11, t) meets it, dst row (s, t) receives the product.
hipError_t mul_mat_id(const weft_ggml_tensor* s0, const weft_ggml_tensor* s1,
                      const weft_ggml_tensor* ids, const weft_ggml_tensor* d, void* wdata,
                      size_t wsize) {
  if (s0 == nullptr || s1 == nullptr || ids == nullptr || d == nullptr) return fail(hipErrorInvalidValue);
  const TypeInfo* t0 = info(s0->type);
  if (t0 == nullptr || t0->vec_dot < 0 || d->type != WEFT_GGML_TYPE_F32 ||
      (s1->type != WEFT_GGML_TYPE_F32 && s1->type != t0->vec_dot))
    return fail(hipErrorNotSupported);
  if (ids->type != kGgmlTypeI32) return fail(hipErrorInvalidValue);
  const TypeInfo* t1 = info(s1->type);
  const TypeInfo* vd = info(t0->vec_dot);
  if (!nonneg(s0) || !nonneg(s1) || !nonneg(ids) || !nonneg(d)) return fail(hipErrorInvalidValue);
  const int64_t K = s0->ne[0], N = s0->ne[1], n_as = s0->ne[2];
  const int64_t ne11 = s1->ne[1], n_tok = s1->ne[2], n_ids = ids->ne[0];
  if (d->ne[0] == 0 || d->ne[1] == 0 || d->ne[2] == 0 || d->ne[3] == 0) return hipSuccess;
  if (s0->ne[3] != 1 || s1->ne[3] != 1 || ids->ne[2] != 1 || ids->ne[3] != 1 || ids->ne[1] != n_tok ||
      s1->ne[0] != K || ne11 == 0 || n_ids % ne11 != 0 || d->ne[0] != N || d->ne[1] != n_ids ||
      d->ne[2] != n_tok || d->ne[3] != 1 || K % t0->blck != 0 || s0->nb[0] != t0->size ||
      s1->nb[0] != t1->size || d->nb[0] != sizeof(float) || d->nb[0] > d->nb[1] ||
      d->nb[1] > d->nb[2] || d->nb[2] > d->nb[3] || d->nb[1] % 4 != 0 || d->nb[2] % 4 != 0 ||
      ids->nb[0] % 4 != 0 || ids->nb[1] % 4 != 0 || ids->data == nullptr ||
      !aligned(ids->data, 4) || n_as > INT32_MAX || n_ids > INT32_MAX ||
      n_ids * n_tok > INT32_MAX)
    return fail(hipErrorInvalidValue);
  if (K == 0 || N == 0) return hipSuccess;
  const bool quantize = s1->type == WEFT_GGML_TYPE_F32;
  const size_t nbw1 = row_size(vd, K);
  if (quantize) {
    if (s1->nb[1] % 4 != 0 || s1->nb[2] % 4 != 0 || wdata == nullptr || !aligned(wdata, 4) ||
        wsize < nbw1 * (size_t)(ne11 * n_tok))
      return fail(hipErrorInvalidValue);
  } else if ((ne11 > 1 && s1->nb[1] != nbw1) || (n_tok > 1 && s1->nb[2] != nbw1 * (size_t)ne11)) {
    return fail(hipErrorNotSupported);  // quantized src1 rows must be packed
  }
  const GgmlTables* tab = nullptr;
  if (s0->type == WEFT_GGML_TYPE_IQ2_XXS || s0->type == WEFT_GGML_TYPE_MXFP4 ||
      s0->type == WEFT_GGML_TYPE_NVFP4 || s0->type == WEFT_GGML_TYPE_IQ2_XS) {
    tab = device_tables();
    if (tab == nullptr) return fail(hipErrorInvalidDevice);
  }
  PairArgs pr{};
  pr.ids = static_cast<const int32_t*>(ids->data);
  pr.ids_s0 = (long long)(ids->nb[0] / 4);
  pr.ids_s1 = (long long)(ids->nb[1] / 4);
  pr.n_ids = (int)n_ids;
  pr.ne11 = (int)ne11;
  pr.n_as = (int)n_as;
  pr.w_es = (long long)s0->nb[2];
  pr.x_s1 = quantize ? (long long)(s1->nb[1] / 4) : 0;
  pr.x_s2 = quantize ? (long long)(s1->nb[2] / 4) : 0;
  pr.xq_row = (long long)nbw1;
  pr.y_s1 = (long long)(d->nb[1] / 4);
  pr.y_s2 = (long long)(d->nb[2] / 4);
  const int n_pairs = (int)(n_ids * n_tok);
  const RowStrides st{s0->nb[1], (size_t)K, (size_t)N};
  const uint8_t* W = static_cast<const uint8_t*>(s0->data);
  const float* X = quantize ? static_cast<const float*>(s1->data) : nullptr;
  const uint8_t* xq_in = quantize ? nullptr : static_cast<const uint8_t*>(s1->data);
  uint8_t* xq_out = quantize ? static_cast<uint8_t*>(wdata) : nullptr;
  float* Y = static_cast<float*>(d->data);
  // several pairs per expert on average, or rows the pair GEMV cannot hold
  // in LDS: group the pairs by expert on the device and run the grouped MFMA
  // GEMM (GGML's own order: quantize src1, group, multiply); the grouping
  // lives in the part of wdata GGML's plan reserves for its row mapping
  const int gemv_fmt = s0->type == WEFT_GGML_TYPE_Q4_0     ? 0
                       : s0->type == WEFT_GGML_TYPE_MXFP4   ? 1
                       : s0->type == WEFT_GGML_TYPE_IQ2_XXS ? 2
                       : s0->type == WEFT_GGML_TYPE_Q6_K    ? 3
                       : s0->type == WEFT_GGML_TYPE_Q5_K    ? 4
                       : s0->type == WEFT_GGML_TYPE_NVFP4   ? 5
                       : s0->type == WEFT_GGML_TYPE_Q4_1    ? 6
                                                            : 7;
  const bool pair_gemv_fits = s0->type == WEFT_GGML_TYPE_Q4_K ? q4k_gemv_fits((size_t)K)
                                                              : staged_gemv_fits(gemv_fmt, (size_t)K);
  if (((n_pairs >= 64 && n_pairs >= 4 * n_as) || !pair_gemv_fits) && wdata != nullptr) {
    const size_t xq_bytes = nbw1 * (size_t)(ne11 * n_tok);
    const size_t used = quantize ? (xq_bytes + 15) & ~(size_t)15 : 0;
    uint8_t* ws = static_cast<uint8_t*>(wdata) + used;
    const size_t ws_bytes = wsize >= used ? wsize - used : 0;
    const size_t n = (size_t)N, k = (size_t)K;
    // src1 rows (t, j) -> Q8_K records at (t * ne11 + j) * nbw1 of wdata
    auto quantize_q8k = [&]() {
      if (!quantize) return;
      if (ne11 == 1) {
        quantize_q8_k_rows(X, n_tok > 1 ? (size_t)pr.x_s2 : k, xq_out, (size_t)n_tok, k);
      } else if (n_tok == 1 || pr.x_s2 == (long long)ne11 * pr.x_s1) {
        quantize_q8_k_rows(X, (size_t)pr.x_s1, xq_out, (size_t)(ne11 * n_tok), k);
      } else {
        for (int64_t t = 0; t < n_tok; ++t)
          quantize_q8_k_rows(X + (size_t)t * pr.x_s2, (size_t)pr.x_s1, xq_out + (size_t)t * ne11 * nbw1,
                             (size_t)ne11, k);
      }
    };
    const uint8_t* xq = quantize ? xq_out : xq_in;
    switch (s0->type) {
      case WEFT_GGML_TYPE_Q4_K:
        if (mul_mat_id_q4k_grouped_ok(W, xq_bytes, Y, n, k, st, pr, n_pairs, ws, ws_bytes)) {
          quantize_q8k();
          mul_mat_id_q4k_grouped(W, xq, Y, n, k, st, pr, n_pairs, ws);
          return pending_error();
        }
        break;
      case WEFT_GGML_TYPE_IQ2_XXS:
      case WEFT_GGML_TYPE_IQ2_XS: {
        const bool xs = s0->type == WEFT_GGML_TYPE_IQ2_XS;
        const int8_t* grid = xs ? tab->grid_xs : tab->grid;
        if (mul_mat_id_iq2_grouped_ok(xs, W, xq_bytes, Y, grid, tab->signs, n, k, st, pr, n_pairs, ws,
                                      ws_bytes)) {
          quantize_q8k();
          mul_mat_id_iq2_grouped(xs, W, xq, grid, tab->signs, Y, n, k, st, pr, n_pairs, ws);
          return pending_error();
        }
        break;
      }
      case WEFT_GGML_TYPE_Q6_K:
      case WEFT_GGML_TYPE_Q5_K: {
        const bool q6 = s0->type == WEFT_GGML_TYPE_Q6_K;
        if (mul_mat_id_kq_grouped_ok(q6, W, xq_bytes, Y, n, k, st, pr, n_pairs, ws, ws_bytes)) {
          quantize_q8k();
          mul_mat_id_kq_grouped(q6, W, xq, Y, n, k, st, pr, n_pairs, ws);
          return pending_error();
        }
        break;
      }
      default: {  // Q4_0 / MXFP4 / NVFP4 / Q4_1: the GEMMs read a planar activation quantized from X
        const int fmt = s0->type == WEFT_GGML_TYPE_Q4_0    ? 0
                        : s0->type == WEFT_GGML_TYPE_MXFP4 ? 1
                        : s0->type == WEFT_GGML_TYPE_NVFP4 ? 2
                                                           : 3;
        const int8_t* cb = fmt == 1 || fmt == 2 ? tab->codebook : nullptr;
        const float* sc = fmt == 1 ? tab->scale : fmt == 2 ? tab->ue4m3 : nullptr;
        if (quantize && mul_mat_id_q80_grouped_ok(fmt, W, X, xq_out, Y, n, k, st, pr, n_pairs,
                                                  (int)n_tok, ws, ws_bytes, cb, sc)) {
          mul_mat_id_q80_grouped(fmt, W, X, xq_out, Y, n, k, st, pr, n_pairs, (int)n_tok, ws, cb, sc);
          return pending_error();
        }
        break;
      }
    }
  }
  switch (s0->type) {
    case WEFT_GGML_TYPE_Q4_K:
      decode_q4k_pairs(W, X, xq_in, xq_out, Y, (size_t)N, (size_t)K, st, pr, n_pairs);
      break;
    case WEFT_GGML_TYPE_Q4_0:
      decode_pairs(0, W, X, xq_in, xq_out, nullptr, nullptr, Y, (size_t)N, (size_t)K, st, pr, n_pairs);
      break;
    case WEFT_GGML_TYPE_Q6_K:
      decode_pairs(3, W, X, xq_in, xq_out, nullptr, nullptr, Y, (size_t)N, (size_t)K, st, pr, n_pairs);
      break;
    case WEFT_GGML_TYPE_Q5_K:
      decode_pairs(4, W, X, xq_in, xq_out, nullptr, nullptr, Y, (size_t)N, (size_t)K, st, pr, n_pairs);
      break;
    case WEFT_GGML_TYPE_NVFP4:
      decode_pairs(5, W, X, xq_in, xq_out, tab->codebook, tab->ue4m3, Y, (size_t)N, (size_t)K, st, pr,
                   n_pairs);
      break;
    case WEFT_GGML_TYPE_MXFP4:
      decode_pairs(1, W, X, xq_in, xq_out, tab->codebook, tab->scale, Y, (size_t)N, (size_t)K, st, pr,
                   n_pairs);
      break;
    case WEFT_GGML_TYPE_Q4_1:
      decode_pairs(6, W, X, xq_in, xq_out, nullptr, nullptr, Y, (size_t)N, (size_t)K, st, pr, n_pairs);
      break;
    case WEFT_GGML_TYPE_IQ2_XS:
      decode_pairs(7, W, X, xq_in, xq_out, tab->grid_xs, tab->signs, Y, (size_t)N, (size_t)K, st, pr,
                   n_pairs);
      break;
    default:
      decode_pairs(2, W, X, xq_in, xq_out, tab->grid, tab->signs, Y, (size_t)N, (size_t)K, st, pr, n_pairs);
      break;
  }
  return pending_error();
}

}  // namespace
}  // namespace weft

extern "C" {

size_t weft_ggml_type_size(int32_t type) {
  const weft::TypeInfo* t = weft::info(type);
  return t ? t->size : 0;
}

int64_t weft_ggml_blck_size(int32_t type) {
  const weft::TypeInfo* t = weft::info(type);
  return t ? t->blck : 0;
}

size_t weft_ggml_row_size(int32_t type, int64_t ne) {
  const weft::TypeInfo* t = weft::info(type);
  return t && ne >= 0 && ne % t->blck == 0 ? weft::row_size(t, ne) : 0;
}

int32_t weft_ggml_vec_dot_type(int32_t type) {
  const weft::TypeInfo* t = weft::info(type);
  return t ? t->vec_dot : -1;
}

size_t weft_ggml_mul_mat_id_work_size(const weft_ggml_tensor* src0, const weft_ggml_tensor* src1,
                                      const weft_ggml_tensor* ids) {
  // ggml_graph_plan's MUL_MAT_ID size (ggml-cpu.c:2827-2845, CACHE_LINE_SIZE 64)
  if (src0 == nullptr || src1 == nullptr || ids == nullptr) return 0;
  const weft::TypeInfo* t0 = weft::info(src0->type);
  if (t0 == nullptr || t0->vec_dot < 0) return 0;
  size_t cur = 0;
  if (src1->type != t0->vec_dot) {
    int64_t n = 1;
    for (int i = 0; i < 4; ++i) n *= src1->ne[i];
    cur += weft_ggml_row_size(t0->vec_dot, n) + sizeof(int64_t);
  }
  const size_t n_as = (size_t)src0->ne[2];
  cur += n_as * sizeof(int64_t) + sizeof(int64_t);
  cur += n_as * (size_t)ids->ne[0] * (size_t)ids->ne[1] * 2 * sizeof(int32_t) + sizeof(int64_t);
  cur += 64 * n_as + 64;
  return cur;
}

int weft_ggml_mul_mat_id(const weft_ggml_tensor* src0, const weft_ggml_tensor* src1,
                         const weft_ggml_tensor* ids, const weft_ggml_tensor* dst, void* wdata,
                         size_t wsize) {
  return (int)weft::mul_mat_id(src0, src1, ids, dst, wdata, wsize);
}

int weft_ggml_mul_mat_id_noalloc(const weft_ggml_tensor* src0, const weft_ggml_tensor* src1,
                                 const weft_ggml_tensor* ids, const weft_ggml_tensor* dst) {
  const size_t need = weft_ggml_mul_mat_id_work_size(src0, src1, ids);
  if (need > WEFT_GGML_NOALLOC_SCRATCH_BYTES) return (int)weft::fail(hipErrorOutOfMemory);
  uint8_t* ws = weft::noalloc_scratch();
  if (ws == nullptr) return (int)weft::pending_error();
  return (int)weft::mul_mat_id(src0, src1, ids, dst, ws, need);
}

size_t weft_ggml_mul_mat_work_size(const weft_ggml_tensor* src0, const weft_ggml_tensor* src1) {
  if (src0 == nullptr || src1 == nullptr) return 0;
  const weft::TypeInfo* t0 = weft::info(src0->type);
  if (t0 == nullptr || t0->vec_dot < 0 || src1->type == t0->vec_dot) return 0;
  int64_t n = 1;
  for (int i = 0; i < 4; ++i) n *= src1->ne[i];
  return weft_ggml_row_size(t0->vec_dot, n);
}

int weft_ggml_mul_mat(const weft_ggml_tensor* src0, const weft_ggml_tensor* src1,
                      const weft_ggml_tensor* dst, void* wdata, size_t wsize) {
  return (int)weft::mul_mat(src0, src1, dst, wdata, wsize);
}

}  // extern "C"
