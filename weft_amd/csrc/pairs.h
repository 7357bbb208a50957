// MUL_MAT_ID pair mode of the GEMV kernels (GGML's mul_mat_id,
// ggml-cpu/ggml-cpu.c:1454-1698): one launch computes every (token t, expert
// slot s) pair, blockIdx.y + pair0 = t * n_ids + s.  The pair's expert
// e = ids[t, s] selects the weight matrix (src0 plane e), its activation is
// src1 row (t, s % ne11), its output dst row (t, s).  ids outside
// [0, n_as) (a GGML assert) leave the pair's dst row untouched.
#pragma once

#include "weft_common.h"

namespace weft {

// pairs per launch: gridDim.y is at most 65535
constexpr int kMaxGridY = 65535;

struct PairArgs {
  const int32_t* ids;        // null: a plain product, no pairs
  long long ids_s0, ids_s1;  // int32 elements between slots / between tokens
  int n_ids, ne11, n_as, pair0;
  long long w_es;            // bytes between expert matrices
  long long x_s1, x_s2;      // floats between src1 rows / src1 planes (tokens)
  long long xq_row;          // bytes of one quantized activation row
  long long y_s1, y_s2;      // floats between dst rows (slots) / planes (tokens)
};

// Point a GEMV launch's W / X / Xq / Y at this workgroup's pair.  The
// quantized activation row (t, r) is written by the pair with slot s = r
// (s < ne11), so every row is written once.  Returns false for an expert
// id outside [0, n_as): the workgroup then does nothing.
template <class A>
__device__ inline bool resolve_pair(A& a) {
  const PairArgs& p = a.pair;
  const int pair = p.pair0 + (int)blockIdx.y;
  const int t = pair / p.n_ids, s = pair - t * p.n_ids;
  const int e = __builtin_amdgcn_readfirstlane(p.ids[t * p.ids_s1 + s * p.ids_s0]);
  if (e < 0 || e >= p.n_as) return false;
  const int r = s % p.ne11;
  const long long xrow = (long long)t * p.ne11 + r;
  a.W += e * p.w_es;
  if (a.X != nullptr) {
    a.X += t * p.x_s2 + r * p.x_s1;
    a.xq_out = (a.xq_out != nullptr && s < p.ne11) ? a.xq_out + xrow * p.xq_row : nullptr;
  } else {
    a.xq_in += xrow * p.xq_row;
  }
  a.Y += t * p.y_s2 + s * p.y_s1;
  return true;
}

// Grouped (MUL_MAT_ID) mode of the MFMA GEMMs: the pairs grouped by expert
// into tiles of at most 64 (moe_group in moe.hip); a workgroup takes tile g
// (tiles past the device's count exit before any barrier), gathers its
// activation rows through the pair list and scatters its outputs.
struct GroupTiles {
  const int32_t* tiles;   // [tmax][3]: expert, first index into pairs, count
  const int32_t* ntiles;  // the tile count (device)
  const int32_t* pairs;   // p = token * n_ids + slot, grouped by expert
  int n_ids, ne11, tmax;
  long long w_es;         // bytes between expert matrices
  long long y_s1, y_s2;   // floats between dst rows (slots) / planes (tokens)
};

// Tile g of the table: false past the tile count; else its first pair index,
// its pair count and the byte offset of its expert's matrix.
__device__ inline bool group_tile(const GroupTiles& g, int tile, int& m0, int& mrows, long long& w_off) {
  if (tile >= __builtin_amdgcn_readfirstlane(*g.ntiles)) return false;
  w_off = (long long)__builtin_amdgcn_readfirstlane(g.tiles[3 * tile]) * g.w_es;
  m0 = __builtin_amdgcn_readfirstlane(g.tiles[3 * tile + 1]);
  mrows = __builtin_amdgcn_readfirstlane(g.tiles[3 * tile + 2]);
  return true;
}

// activation row (token * ne11 + slot % ne11) of the tile's row r
__device__ inline int group_act_row(const GroupTiles& g, int m0, int r) {
  const int p = g.pairs[m0 + r];
  const int t = p / g.n_ids, s = p - t * g.n_ids;
  return t * g.ne11 + s % g.ne11;
}

// float offset of the dst row of the tile's row r
__device__ inline long long group_dst_row(const GroupTiles& g, int m0, int r) {
  const int p = g.pairs[m0 + r];
  const int t = p / g.n_ids, s = p - t * g.n_ids;
  return t * g.y_s2 + s * g.y_s1;
}

}  // namespace weft
