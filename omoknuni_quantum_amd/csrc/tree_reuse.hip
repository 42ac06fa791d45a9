// Subtree reuse: a node of each tree becomes the root, and its subtree is compacted to the
// front of the tree (gfx950).
//
// Reference: CSRTree.shift_root (python/mcts/gpu/csr_tree.py:1020-1229), reached through
// TreeOperations.apply_subtree_reuse (python/mcts/core/tree_operations.py:53-133) from
// MCTS.update_root (python/mcts/core/mcts.py:1205-1245).
//   - The kept nodes are numbered breadth-first from the new root, children in row order.
//   - N, W and P of every kept node are copied, and parents are remapped; the new root has
//     parent -1 and action -1.
//   - Every other node is dropped, and the edge arrays are rebuilt in the new node order.
// With breadth-first numbering, the children of every kept node are again consecutive, and
// the edge of child c is c-1. The implicit-column layout of this library
// (child of edge e = node e+1) therefore holds after the shift as it held before.
//
// One workgroup per tree walks the subtree level by level. A level is a contiguous range of
// new ids. A block-wide scan of the level's row lengths gives each node the new id of its
// first child, so a level costs one scan and one pass of writes. The new arrays are built in
// a workspace and then copied over the front of the tree. The workspace holds eight int32
// arrays of `capacity` entries per tree.
#include "omq_common.h"

namespace omq {

constexpr int kShiftThreads = 1024;
constexpr int kShiftWaves = kShiftThreads / kWave;

// exclusive scan of one value per thread over the workgroup; total through *total
__device__ inline int shift_block_scan(int v, int* s_wtot, int* total) {
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  int wt;
  const int wex = wave_excl_scan(v, &wt);
  if (lane_id() == 0) s_wtot[wave] = wt;
  __syncthreads();
  int base = 0, tot = 0;
  for (int i = 0; i < kShiftWaves; ++i) {
    const int x = s_wtot[i];
    if (i < wave) base += x;
    tot += x;
  }
  __syncthreads();  // s_wtot is reused by the next scan
  *total = tot;
  return base + wex;
}

__global__ __launch_bounds__(kShiftThreads) void shift_root_kernel(omq_forest f,
                                                                   const int32_t* new_roots,
                                                                   int32_t* ws) {
  __shared__ int s_wtot[kShiftWaves];
  const int t = blockIdx.x;
  const int tid = threadIdx.x;
  const int cap = f.capacity;
  const int64_t tb = (int64_t)t * cap;
  const int r = new_roots[t];
  const int n_old = f.num_nodes[t];
  if (r <= 0 || r >= n_old) return;  // tree unchanged (0: already the root; -1: no shift)

  int32_t* old_of_new = ws + (int64_t)t * cap * 8;
  int32_t* npar = old_of_new + cap;
  int32_t* nfirst = old_of_new + 2 * (int64_t)cap;
  int32_t* nnch = old_of_new + 3 * (int64_t)cap;
  int32_t* nN = old_of_new + 4 * (int64_t)cap;
  float* nW = reinterpret_cast<float*>(old_of_new + 5 * (int64_t)cap);
  float* nP = reinterpret_cast<float*>(old_of_new + 6 * (int64_t)cap);
  int32_t* nA = old_of_new + 7 * (int64_t)cap;

  if (tid == 0) {
    old_of_new[0] = r;
    npar[0] = -1;
  }
  __syncthreads();
  // breadth-first numbering: level [lo, hi) of new ids; its children get [hi, next).  A row
  // that leaves [0, num_nodes), or more kept nodes than num_nodes (a cycle), marks the tree
  // inconsistent: it is then left unchanged, and no access leaves the tree's arrays.
  int lo = 0, hi = 1, next = 1;
  bool bad = false;
  while (lo < hi && !bad) {
    for (int c0 = lo; c0 < hi; c0 += kShiftThreads) {
      const int i = c0 + tid;
      int k = 0, old = 0, of = 0;
      bool row_bad = false;
      if (i < hi) {
        old = old_of_new[i];
        k = f.num_children[tb + old];
        of = f.first_child[tb + old];
        if (k < 0 || (k > 0 && (of < 0 || (int64_t)of + k >= n_old))) {
          row_bad = true;
          k = 0;
        }
      }
      int tot;
      const int ex = shift_block_scan(k, s_wtot, &tot);
      if (__syncthreads_or(row_bad) || next + tot > n_old) {
        bad = true;
        break;
      }
      if (i < hi) {
        const int base = next + ex;
        nnch[i] = k;
        nfirst[i] = k > 0 ? base - 1 : -1;
        for (int j = 0; j < k; ++j) {
          old_of_new[base + j] = of + 1 + j;  // child of edge of+j is node of+j+1
          npar[base + j] = i;
        }
      }
      next += tot;
      __syncthreads();
    }
    lo = hi;
    hi = next;
  }
  if (bad) return;
  const int n_new = next;
  for (int i = tid; i < n_new; i += kShiftThreads) {
    const int64_t o = tb + old_of_new[i];
    nN[i] = f.visit_counts[o];
    nW[i] = f.value_sums[o];
    nP[i] = f.priors[o];
    nA[i] = i == 0 ? -1 : f.actions[o];
  }
  __syncthreads();
  for (int i = tid; i < n_new; i += kShiftThreads) {
    const int64_t d = tb + i;
    f.visit_counts[d] = nN[i];
    f.value_sums[d] = nW[i];
    f.priors[d] = nP[i];
    f.parents[d] = npar[i];
    f.first_child[d] = nfirst[i];
    f.num_children[d] = nnch[i];
    f.actions[d] = nA[i];
  }
  if (tid == 0) f.num_nodes[t] = n_new;
}

hipError_t launch_shift_root(const omq_forest& f, const int32_t* new_roots, int32_t* ws,
                             hipStream_t st) {
  hipLaunchKernelGGL(shift_root_kernel, dim3(f.num_trees), dim3(kShiftThreads), 0, st, f,
                     new_roots, ws);
  return hipGetLastError();
}

}  // namespace omq
