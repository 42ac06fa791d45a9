// Backup with virtual-loss revert (gfx950).
//
// Sequential definition: for every simulation s in order and every node x on its path,
//   N[x] = N[x] - VL + 1                      (cython_tree_optimized.pyx:222)
//   W[x] = W[x] + sign(x) * v(leaf of s)      (optimized_wave_search.py:472-483: leaf +v,
//                                              parent -v, ...; or root-positive, pyx:216-224)
// Ordered mode uses the group log of the selection: a node appears in exactly one group per
// wave, and the group's members are in simulation order, so folding the members' signed
// values into W[x] in that order gives the sequential result bit for bit, with no atomics.
// Small groups are folded by one lane each; groups with more than kBigGroup members by the
// whole wave (lanes load, one running sum through v_readlane).
#include "backup_groups.h"

namespace omq {

// signed value per simulation (sim_value_at)
__global__ void sim_value_kernel(omq_forest f, omq_wave w, int W, int sign_mode) {
  int bx = blockIdx.x, by = blockIdx.y;
  xcd_block(&bx, &by);  // one contiguous run of blocks (leaves of few trees) per XCD
  const int s = bx * blockDim.x + threadIdx.x;
  if (s >= W) return;
  sim_value_at(f, w, by, s, sign_mode);
}

template <bool FUSED>
__global__ __launch_bounds__(kBackupThreads) void backup_groups_kernel(omq_forest f, omq_wave w,
                                                                       int vli, int sign_mode) {
  int bx = blockIdx.x, by = blockIdx.y;
  xcd_block(&bx, &by);  // one contiguous run of blocks (leaves of few trees) per XCD
  backup_groups_block<FUSED>(f, w, vli, sign_mode, bx, by, (int)gridDim.x);
}

// atomic mode: one lane per simulation walks its path with float atomics (order not fixed)
__global__ void backup_atomic_kernel(omq_forest f, omq_wave w, int W, int vli) {
  const int t = blockIdx.y;
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= W) return;
  const int64_t tb = (int64_t)t * f.capacity;
  const int64_t wb = (int64_t)t * w.max_wave;
  const int L = w.path_len[wb + s];
  const float v = w.sim_value[wb + s];
  const int32_t* path = w.paths + (wb + s) * w.max_depth;
  for (int d = 0; d < L; ++d) {
    const int x = path[d];
    atomicAdd(&f.visit_counts[tb + x], 1 - vli);
    unsafeAtomicAdd(&f.value_sums[tb + x], (d & 1) ? -v : v);
  }
}

// reference-style backup over an explicit path matrix (vectorized_backup_kernel)
__global__ void paths_backup_kernel(omq_forest f, const int32_t* paths, const int32_t* plen,
                                    const int32_t* tree_of, const float* values, int batch,
                                    int max_depth, int sign_mode) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  const int t = tree_of ? tree_of[b] : 0;
  if (t < 0 || t >= f.num_trees) return;  // entries naming no tree are skipped
  const int64_t tb = (int64_t)t * f.capacity;
  // entries d < min(length, max_depth); the leaf-positive sign counts the distance from the
  // leaf by the length as given (vectorized_backup_kernel, mcts_kernels.cu:142-146), also for a
  // length past the row
  const int Lp = plen[b];
  const int L = min(Lp, max_depth);
  const float v = values[b];
  for (int d = 0; d < L; ++d) {
    const int x = paths[(int64_t)b * max_depth + d];
    if (x < 0 || x >= f.capacity) continue;  // -1 padding and out-of-range entries are skipped
    const int e = sign_mode == OMQ_SIGN_LEAF_POSITIVE ? (Lp - 1 - d) : d;
    atomicAdd(&f.visit_counts[tb + x], 1);
    unsafeAtomicAdd(&f.value_sums[tb + x], (e & 1) ? -v : v);
  }
}

__global__ void virtual_loss_kernel(omq_forest f, const int32_t* nodes, const int32_t* tree_of,
                                    int count, int delta) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  const int t = tree_of ? tree_of[i] : 0;
  const int x = nodes[i];
  if (x < 0 || x >= f.capacity || t < 0 || t >= f.num_trees) return;
  atomicAdd(&f.visit_counts[(int64_t)t * f.capacity + x], delta);
}

__global__ void reset_kernel(omq_forest f) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= f.num_trees) return;
  const int64_t r = (int64_t)t * f.capacity;
  f.visit_counts[r] = 1;
  f.value_sums[r] = 0.0f;
  f.priors[r] = 1.0f;
  f.parents[r] = -1;
  f.first_child[r] = -1;
  f.num_children[r] = 0;
  f.actions[r] = -1;
  f.num_nodes[t] = 1;
}

// ---------------------------------------------------------------------------------------
hipError_t launch_backup(const omq_forest& f, const omq_wave& w, int W, float virtual_loss,
                         int sign_mode, int w_mode, hipStream_t st) {
  const int vli = (int)virtual_loss;
  dim3 g1((W + 255) / 256, f.num_trees);
  const bool fused = w_mode != OMQ_WACC_ATOMIC && W <= kFuseMaxWave;
  if (!fused) {
    hipLaunchKernelGGL(sim_value_kernel, g1, dim3(256), 0, st, f, w, W, sign_mode);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (w_mode == OMQ_WACC_ATOMIC) {
    hipLaunchKernelGGL(backup_atomic_kernel, g1, dim3(256), 0, st, f, w, W, vli);
    return hipGetLastError();
  }
  // (the group count is on the device)
  const int blocks = backup_group_blocks(W);
  if (fused)
    hipLaunchKernelGGL(backup_groups_kernel<true>, dim3(blocks, f.num_trees),
                       dim3(kBackupThreads), 0, st, f, w, vli, sign_mode);
  else
    hipLaunchKernelGGL(backup_groups_kernel<false>, dim3(blocks, f.num_trees),
                       dim3(kBackupThreads), 0, st, f, w, vli, sign_mode);
  return hipGetLastError();
}

hipError_t launch_paths_backup(const omq_forest& f, const int32_t* paths, const int32_t* plen,
                               const int32_t* tree_of, const float* values, int batch,
                               int max_depth, int sign_mode, hipStream_t st) {
  hipLaunchKernelGGL(paths_backup_kernel, dim3((batch + 255) / 256), dim3(256), 0, st, f, paths,
                     plen, tree_of, values, batch, max_depth, sign_mode);
  return hipGetLastError();
}

hipError_t launch_virtual_loss(const omq_forest& f, const int32_t* nodes, const int32_t* tree_of,
                               int count, int delta, hipStream_t st) {
  hipLaunchKernelGGL(virtual_loss_kernel, dim3((count + 255) / 256), dim3(256), 0, st, f, nodes,
                     tree_of, count, delta);
  return hipGetLastError();
}

hipError_t launch_reset(const omq_forest& f, hipStream_t st) {
  hipLaunchKernelGGL(reset_kernel, dim3((f.num_trees + 255) / 256), dim3(256), 0, st, f);
  return hipGetLastError();
}

}  // namespace omq
