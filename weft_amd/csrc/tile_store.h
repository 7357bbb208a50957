// Output stage shared by the MFMA prefill GEMMs (prefill_q4k.hip,
// prefill_kq.hip, prefill_iq2.hip, prefill_q80.hip's int8 body), for their
// 64 x 128 tiles and the Q4_K GEMM's other tilings (32 or 64 rows, 64 or
// 128 columns).
//
// Each of the eight MFMA waves ends the K loop with the partial sums of one
// parity (superblocks, half superblocks or stages of that parity: w >> 2)
// for the tile's columns 32 (w & 3) .. + 31, in two 32 x 32 accumulators:
// register r of tile t holds row 32 t + 8 (r / 4) + 4 kg + r % 4 and column
// lane % 32 (kg = lane / 32).  Storing that layout straight to Y costs one
// 4-byte store instruction per register, 128 per workgroup, and the last
// stores of every workgroup meet in one burst at the end of the launch.
// Here both parities' partials go to LDS as two row-major 64 x 128 planes,
// then every MFMA wave adds them (even + odd, the order the kernels always
// used) and stores 16 contiguous bytes per lane: four rows per instruction,
// 32 store instructions per workgroup.
#pragma once

#include <cstdint>

#include <hip/hip_runtime.h>

namespace weft {

// floats per plane row: rows 4 apart (the kg halves of one register) start
// 32 banks apart, and rows stay 16-byte aligned
template <int kCols>
constexpr int tile_plane_ld() {
  return kCols + 8;
}
template <int kRows, int kCols>
constexpr int tile_plane_bytes() {
  return kRows * tile_plane_ld<kCols>() * 4;
}
constexpr int kTilePlaneLd = tile_plane_ld<128>();             // 136
constexpr int kTilePlaneBytes = tile_plane_bytes<64, 128>();   // 34,816

typedef float tile_v16f __attribute__((ext_vector_type(16)));

// Partials of T2 32 x 32 accumulators (tile rows 32 t ..) of column group
// wcol into a plane of kCols columns.  Every wave reading the K loop's LDS
// must have passed a barrier first.
template <int T2, int kCols>
__device__ inline void tile_partials_to_lds_t(const tile_v16f (&y)[T2], int wcol, int lane, float* plane) {
  constexpr int ld = tile_plane_ld<kCols>();
  const int col = 32 * wcol + (lane & 31), kg = lane >> 5;
#pragma unroll
  for (int t = 0; t < T2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 32 * t + 8 * (r >> 2) + 4 * kg + (r & 3);
      plane[row * ld + col] = y[t][r];
    }
}

// The 64 x 128 tile of eight waves: partials of this wave's parity into its
// plane (plane = the LDS plane of the wave's parity, 16-byte aligned,
// kTilePlaneBytes).
__device__ inline void tile_partials_to_lds(const tile_v16f (&y)[2], int wcol, int lane, float* plane) {
  tile_partials_to_lds_t<2, 128>(y, wcol, lane, plane);
}

// The tile row that lane `lane` of MFMA wave `wave` (of kWaves) stores in
// pass p (0 .. kRows / (4 kWaves) - 1) of tile_store_from_lds_t.
template <int kWaves>
__device__ inline int tile_store_row_t(int wave, int lane, int p) {
  return 4 * kWaves * p + 4 * wave + (lane >> 4);
}
__device__ inline int tile_store_row(int wave, int lane, int p) { return tile_store_row_t<8>(wave, lane, p); }

// After a barrier that follows every wave's partials: MFMA wave w (of
// kWaves) stores tile rows tile_store_row_t(w, lane, p), columns
// 4 (lane % 16) + 64 k, as fin(even, odd) per value.  Rows past mrows and
// columns past ncols are not written; row_ptr(rr) is the address of tile row
// rr's first column in Y.  A row segment that is not 16-byte aligned, or not
// wholly inside ncols, is stored value by value.
template <int kRows, int kCols, int kWaves, class RowPtr, class Fin>
__device__ inline void tile_store_from_lds_t(int wave, int lane, const float* even, const float* odd,
                                             int mrows, int ncols, RowPtr row_ptr, Fin fin) {
  static_assert(kRows % (4 * kWaves) == 0 && kCols % 64 == 0, "whole store passes");
  constexpr int ld = tile_plane_ld<kCols>();
  const int c0 = 4 * (lane & 15);
#pragma unroll
  for (int p = 0; p < kRows / (4 * kWaves); ++p) {
    const int rr = tile_store_row_t<kWaves>(wave, lane, p);
    if (rr >= mrows) continue;
    float* dst = row_ptr(rr);
#pragma unroll
    for (int k = 0; k < kCols / 64; ++k) {
      const int c = c0 + 64 * k;
      const float4 e = *reinterpret_cast<const float4*>(even + rr * ld + c);
      const float4 o = *reinterpret_cast<const float4*>(odd + rr * ld + c);
      const float4 v = make_float4(fin(e.x, o.x), fin(e.y, o.y), fin(e.z, o.z), fin(e.w, o.w));
      float* d = dst + c;
      if (c + 3 < ncols && (reinterpret_cast<uintptr_t>(d) & 15u) == 0) {
        *reinterpret_cast<float4*>(d) = v;
      } else {
        const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (c + i < ncols) d[i] = vv[i];
      }
    }
  }
}

// The 64 x 128 tile of eight waves.
template <class RowPtr, class Fin>
__device__ inline void tile_store_from_lds(int wave, int lane, const float* even, const float* odd,
                                           int mrows, int ncols, RowPtr row_ptr, Fin fin) {
  tile_store_from_lds_t<64, 128, 8>(wave, lane, even, odd, mrows, ncols, row_ptr, fin);
}

}  // namespace weft
