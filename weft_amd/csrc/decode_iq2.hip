// Batch-1 decode GEMV for IQ2_XXS x Q8_K and IQ2_XS x Q8_K:
// production_mul_mat_iq2_xxs_decode / production_mul_mat_iq2_xs at M = 1
// (examples/kernels/mul_mat/iq2_xxs_decode.py, iq2_xs.py:26-56), rows of up
// to 4096 values.
//
// Semantics (GGML generic vec_dots, ggml-cpu/quants.c):
//   IQ2_XXS :855-895  y = 0.125 * sum_b (dw dx)_b * sum_g (2 s_g + 1) I_g
//   IQ2_XS  :897-946  the same with a 4-bit scale per 16-element half
//   I = sum_{8 elements of entry l} grid[idx_l][j] * sign_l[j] * q8       (exact)
//
// gfx950 mapping, as the Q4_0 / Q4_K batch-1 kernels: lane j of a row owns
// the 32-groups 2 (j % 4) and 2 (j % 4) + 1 of superblock j / 4 (64 values),
// their 16 record bytes loaded straight into VGPRs (five dwords from the
// aligned dword below them: a record is 2-byte aligned), the superblock's d
// and, for IQ2_XS, the two groups' scale bytes.  Its 64 activation values
// (the same for every row) are read from LDS into VGPRs once.  Grid rows and
// sign masks (the +-1 sign table turned into 0xff / 0x00 byte masks as it
// is staged) come from LDS tables; products run on v_dot4_i32_i8.  Tables
// outside the masks' precondition (a sign byte other than +-1, a grid byte
// of 0) are detected as they are staged and take the i8 byte product of
// grid and sign instead (weft_common.h).  A
// superblock's exact integer sum is the sum over its four lanes (DPP), then
// one fp32 term per superblock and a wave sum per row.  A wave walks its
// rows with one row of lookahead.  The activation is quantized in every
// workgroup (16 lanes per superblock, bit-exact with quantize_row_q8_K_ref);
// workgroup 0 writes Xq, so the mul_mat is one launch.
#include <algorithm>
#include <type_traits>

#include "activation.h"
#include "kernels.h"
#include "runtime.h"
#include "weft_common.h"
#include "weft_hip.h"

namespace weft {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / kWave;

struct Iq2Args {
  const uint8_t* W;
  const float* X;
  uint8_t* xq_out;
  const int8_t* grid;   // I8X8[256] (IQ2_XXS) or [512] (IQ2_XS)
  const int8_t* signs;  // I8X8[128], +-1
  float* Y;
  int N, K;
  int rows_per_wg;
  size_t ldw;
};

// four +-1 sign bytes -> byte masks (0xff where -1, bit 7 set), as the sign
// table is held in LDS
__device__ __forceinline__ uint32_t iq2_sign_mask(uint32_t s) { return ((s >> 7) & 0x01010101u) * 0xffu; }

// negate the bytes of g whose mask byte in m is 0xff: for a byte b != 0,
// (b ^ 0xff) + 1 = 256 - b never carries into the next byte (GGML's
// magnitudes are 8, 25 and 43; a table with a 0 byte takes mul8x4)
__device__ __forceinline__ int iq2_negate(uint32_t g, uint32_t m) {
  return (int)((g ^ m) + (m & 0x01010101u));
}

template <bool kXs>
__global__ void __launch_bounds__(kThreads) iq2_gemv_m1_kernel(Iq2Args a) {
  constexpr int kRec = kXs ? kIq2xsBytes : kIq2xxsBytes;  // 74 / 66
  constexpr int kGridBytes = kXs ? 4096 : 2048;
  extern __shared__ __align__(16) char lds[];
  char* tgrid = lds;
  char* tsign = lds + kGridBytes;         // sign rows as byte masks
  char* traw = lds + kGridBytes + 1024;   // sign rows as given
  char* act = lds + kGridBytes + 2048;    // Q8_K activation row
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int K = a.K;
  const int nsb = K >> 8;  // even, <= 16
  const bool live = lane < 4 * nsb;
  const int sb = min(lane >> 2, nsb - 1), g0 = 2 * (lane & 3);
  // the lane's 16 group bytes start 2 + 8 g0 into record sb
  const uint32_t doff = (uint32_t)(kRec * sb + 2 + 8 * g0);
  const uint32_t d_a = doff & ~3u, dsh = doff & 3u;  // 0 or 2
  const uint32_t hoff = (uint32_t)(kRec * sb) & ~3u;  // the dword holding d
  const uint32_t hsh = (uint32_t)(kRec * sb) & 3u;    // 0 or 2
  const uint32_t soff = (uint32_t)(kRec * sb + 66 + g0);  // IQ2_XS: the two groups' scale bytes
  const size_t rb = a.ldw;
  const int row_first = blockIdx.x * a.rows_per_wg + wave;
  const int row_end = min(a.N, blockIdx.x * a.rows_per_wg + a.rows_per_wg);
  const int nrows = row_first < row_end ? (row_end - row_first + kWaves - 1) / kWaves : 0;

  // activation loads first: waiting for them does not wait for the weights
  Q8KStager16<1> stager;
  stager.prefetch(a.X, (size_t)K, K, 0, 1);
  __builtin_amdgcn_sched_barrier(0);

  struct RowBuf {
    uint32_t w[5];
    uint32_t h, s;
  };
  auto issue = [&](RowBuf& buf, int k) {
    const int row = min(row_first + k * kWaves, a.N - 1);  // clamped: always a valid row
    const uint8_t* rp = a.W + (size_t)row * rb;
    const uint4 v = *reinterpret_cast<const uint4*>(rp + d_a);
    buf.w[0] = v.x, buf.w[1] = v.y, buf.w[2] = v.z, buf.w[3] = v.w;
    // the fifth dword only holds data at a 2-byte offset; otherwise dword 3
    // again (the last record's data ends at its row's end)
    buf.w[4] = *reinterpret_cast<const uint32_t*>(rp + d_a + (dsh ? 16 : 12));
    buf.h = *reinterpret_cast<const uint32_t*>(rp + hoff);
    if constexpr (kXs) buf.s = *reinterpret_cast<const uint16_t*>(rp + soff);
  };
  // the tables next, one dword per thread: they are needed with the
  // activation, so they do not queue behind the weight rows
  static_assert(kGridBytes / 4 <= kThreads, "one grid dword per thread");
  const int ti = threadIdx.x;
  uint32_t tg = 0, ts = 0;
  if (ti < kGridBytes / 4) tg = reinterpret_cast<const uint32_t*>(a.grid)[ti];
  if (ti < 256) ts = reinterpret_cast<const uint32_t*>(a.signs)[ti];
  __builtin_amdgcn_sched_barrier(0);

  RowBuf bufA, bufB;
  issue(bufA, 0);
  __builtin_amdgcn_sched_barrier(0);

  if (ti < kGridBytes / 4) reinterpret_cast<uint32_t*>(tgrid)[ti] = tg;
  if (ti < 256) {
    reinterpret_cast<uint32_t*>(tsign)[ti] = iq2_sign_mask(ts);
    reinterpret_cast<uint32_t*>(traw)[ti] = ts;
  }
  // the tables take the mask path when every workgroup thread's words meet
  // its precondition (the same answer in every workgroup)
  __shared__ uint32_t tflag[kWaves];
  iq2_flag_wave(tflag, (ti < kGridBytes / 4 && !iq2_grid_word_ok(tg)) || (ti < 256 && !iq2_sign_word_ok(ts)));
  stager.finish(a.X, (size_t)K, blockIdx.x == 0 ? a.xq_out : nullptr, K, 0, 1, act);
  __syncthreads();
  const bool canon = iq2_flags_clear(tflag, kWaves);

  // this lane's 64 activation values and its superblock's scale
  int4 xa[4];
  float dx;
  {
    const Q8KView v = q8k_view(act, K, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) xa[i] = *reinterpret_cast<const int4*>(v.qs + 256 * sb + 32 * g0 + 16 * i);
    dx = v.d[sb];
  }
  const uint2* grid = reinterpret_cast<const uint2*>(tgrid);

  // kGen: any int8 tables, each weight byte the i8 product grid * sign;
  // otherwise the sign masks' negate
  auto compute = [&](const RowBuf& buf, int k, auto gen) __attribute__((always_inline)) {
    constexpr bool kGen = decltype(gen)::value;
    const uint2* sgn = reinterpret_cast<const uint2*>(kGen ? traw : tsign);
    uint32_t q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = dsh ? __builtin_amdgcn_alignbyte(buf.w[i + 1], buf.w[i], 2) : buf.w[i];
    const float dw = fp16_to_fp32(hsh ? buf.h >> 16 : buf.h & 0xffffu);
    int sum = 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {  // group g0 + u: words q[2u], q[2u + 1]
      const int4 x0 = xa[2 * u], x1 = xa[2 * u + 1];
      const int xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      int part[2] = {0, 0};  // 16-element halves
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        uint2 gv, sv;
        if constexpr (kXs) {
          const uint32_t e = (q[2 * u + (l >> 1)] >> (16 * (l & 1))) & 0xffffu;
          gv = grid[e & 511u];
          sv = sgn[e >> 9];
        } else {
          gv = grid[(q[2 * u] >> (8 * l)) & 0xffu];
          sv = sgn[(q[2 * u + 1] >> (7 * l)) & 127u];
        }
        const int w0 = kGen ? (int)mul8x4(gv.x, sv.x) : iq2_negate(gv.x, sv.x);
        const int w1 = kGen ? (int)mul8x4(gv.y, sv.y) : iq2_negate(gv.y, sv.y);
        part[l >> 1] = dot4(w0, xv[2 * l], part[l >> 1]);
        part[l >> 1] = dot4(w1, xv[2 * l + 1], part[l >> 1]);
      }
      if constexpr (kXs) {
        const uint32_t sb8 = (buf.s >> (8 * u)) & 0xffu;
        sum += part[0] * (2 * (int)(sb8 & 15u) + 1) + part[1] * (2 * (int)(sb8 >> 4) + 1);
      } else {
        sum += (part[0] + part[1]) * (2 * (int)(q[2 * u + 1] >> 28) + 1);
      }
    }
    // the superblock's exact integer sum over its four lanes, then one fp32 term
    const int bsum = sum4(live ? sum : 0);
    const float t = (lane & 3) == 0 && live ? (dw * dx) * (float)bsum : 0.f;
    const float tot = wave_sum_f(t);
    if (lane == 0) a.Y[row_first + k * kWaves] = 0.125f * tot;
  };

  auto rows = [&](auto gen) __attribute__((always_inline)) {
    int k = 0;
    for (; k + 2 < nrows; k += 2) {
      issue(bufB, k + 1);
      compute(bufA, k, gen);
      issue(bufA, k + 2);
      compute(bufB, k + 1, gen);
    }
    if (nrows - k == 2) {
      issue(bufB, k + 1);
      compute(bufA, k, gen);
      compute(bufB, k + 1, gen);
    } else if (nrows - k == 1) {
      compute(bufA, k, gen);
    }
  };
  if (canon)
    rows(std::false_type{});
  else
    rows(std::true_type{});
}

}  // namespace

// Launches the kernel above when the call suits it: one activation row of
// K <= 4096 with an even number of superblocks (4-byte aligned rows), X and
// Xq 16- and 4-byte aligned, the tables 4-byte aligned.
bool decode_iq2_m1(bool xs, const uint8_t* W, const float* X, uint8_t* Xq, const int8_t* grid,
                   const int8_t* signs, float* Y, size_t N, size_t K, const RowStrides& st) {
  const size_t rb = K / 256 * (xs ? kIq2xsBytes : kIq2xxsBytes);
  const size_t ldw = N > 1 ? st.ldw : rb;
  if (N == 0 || K == 0 || K > 4096 || K % 512 != 0 || X == nullptr || Xq == nullptr || W == nullptr ||
      Y == nullptr || grid == nullptr || signs == nullptr || !aligned(X, 16) || !aligned(W, 4) ||
      ldw % 4 != 0 || !aligned(Y, 4) || !aligned(Xq, 4) || !aligned(grid, 4) || !aligned(signs, 4) ||
      N > (size_t)INT32_MAX || (N > 1 && ldw < rb) || ldw >= ((size_t)1 << 40))
    return false;
  const int cus = cu_count();
  const size_t wgs = std::max<size_t>(1, std::min<size_t>(2 * (size_t)cus, (N + kWaves - 1) / kWaves));
  Iq2Args a;
  a.W = W;
  a.X = X;
  a.xq_out = Xq;
  a.grid = grid;
  a.signs = signs;
  a.Y = Y;
  a.N = (int)N;
  a.K = (int)K;
  // a CompileOptions NC binding sets the weight rows per workgroup
  const int nc = tile_bindings().nc;
  a.rows_per_wg = nc > 0 ? (int)std::min<size_t>(N, (size_t)nc) : (int)((N + wgs - 1) / wgs);
  a.ldw = ldw;
  const int g = (int)((N + a.rows_per_wg - 1) / a.rows_per_wg);
  const size_t lds = (xs ? 4096 : 2048) + 2048 + q8k_lds_row_bytes((int)K);
  if (xs)
    iq2_gemv_m1_kernel<true><<<g, kThreads, lds, current_stream()>>>(a);
  else
    iq2_gemv_m1_kernel<false><<<g, kThreads, lds, current_stream()>>>(a);
  check_launch("iq2_gemv_m1_kernel");
  return true;
}

}  // namespace weft
