// Device-side grouping of MUL_MAT_ID pairs by expert: the matrix_rows /
// matrix_row_counts step of ggml_compute_forward_mul_mat_id
// (ggml-cpu/ggml-cpu.c:1573-1590), done by one workgroup so the expert
// choices never leave the device.  Output, in the caller's work buffer:
//   int32 ntiles | pad to 16 B | tiles[tmax][3] = {expert, first, count} |
//   pairs[n_pairs] (pair p = token * n_ids + slot, grouped by expert)
// A tile holds at most 64 pairs of one expert, so the grouped GEMMs take one
// tile per workgroup row block.  Pairs whose id lies outside [0, n_as) (a
// GGML assert) are left out.  Within an expert the pair order depends on
// atomic timing; every output is computed from its own pair alone, so the
// results do not.
#include "kernels.h"
#include "runtime.h"
#include "weft_common.h"

namespace weft {
namespace {

constexpr int kGroupThreads = 1024;

struct GroupArgs {
  const int32_t* ids;
  long long s0, s1;  // int32 elements between slots / tokens
  int n_ids, n_pairs, n_as, tmax;
  int32_t* ntiles;
  int32_t* tiles;
  int32_t* pairs;
};

__global__ void __launch_bounds__(kGroupThreads) moe_group_kernel(GroupArgs g) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int start[kMaxExperts];
  __shared__ int fill[kMaxExperts];
  const int tid = threadIdx.x;
  for (int e = tid; e < g.n_as; e += kGroupThreads) {
    cnt[e] = 0;
    fill[e] = 0;
  }
  __syncthreads();
  for (int p = tid; p < g.n_pairs; p += kGroupThreads) {
    const int t = p / g.n_ids, s = p - t * g.n_ids;
    const int e = g.ids[t * g.s1 + s * g.s0];
    if (e >= 0 && e < g.n_as) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0, nt = 0;
    for (int e = 0; e < g.n_as; ++e) {
      start[e] = run;
      for (int j = 0; j < cnt[e] && nt < g.tmax; j += kMoeTileRows, ++nt) {
        g.tiles[3 * nt] = e;
        g.tiles[3 * nt + 1] = run + j;
        g.tiles[3 * nt + 2] = min(kMoeTileRows, cnt[e] - j);
      }
      run += cnt[e];
    }
    *g.ntiles = nt;
  }
  __syncthreads();
  for (int p = tid; p < g.n_pairs; p += kGroupThreads) {
    const int t = p / g.n_ids, s = p - t * g.n_ids;
    const int e = g.ids[t * g.s1 + s * g.s0];
    if (e >= 0 && e < g.n_as) g.pairs[start[e] + atomicAdd(&fill[e], 1)] = p;
  }
}

}  // namespace

int moe_tile_bound(int n_pairs, int n_as) { return (n_pairs + kMoeTileRows - 1) / kMoeTileRows + n_as; }

size_t moe_group_bytes(int n_pairs, int n_as) {
  return 16 + 12 * (size_t)moe_tile_bound(n_pairs, n_as) + 4 * (size_t)n_pairs;
}

MoeGroups moe_group(const PairArgs& pr, int n_pairs, void* ws) {
  MoeGroups m{};
  m.tmax = moe_tile_bound(n_pairs, pr.n_as);
  m.ntiles = static_cast<int32_t*>(ws);
  m.tiles = m.ntiles + 4;
  m.pairs = m.tiles + 3 * (size_t)m.tmax;
  GroupArgs g{pr.ids, pr.ids_s0, pr.ids_s1, pr.n_ids, n_pairs, pr.n_as, m.tmax, m.ntiles, m.tiles, m.pairs};
  moe_group_kernel<<<1, kGroupThreads, 0, current_stream()>>>(g);
  check_launch("moe_group_kernel");
  return m;
}

}  // namespace weft
