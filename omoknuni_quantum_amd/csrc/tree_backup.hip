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
#include "omq_common.h"

namespace omq {

constexpr int kBackupThreads = 256;
constexpr int kBigGroup = 32;
constexpr int kBigChunk = 8;  // member values per lane held per chunk of a big group

// signed value per simulation: v(leaf), negated when the leaf depth is odd in leaf-positive
// mode, so that the contribution at depth d is (d odd ? -sv : sv)
__global__ void sim_value_kernel(omq_forest f, omq_wave w, int W, int sign_mode) {
  int bx = blockIdx.x, by = blockIdx.y;
  xcd_block(&bx, &by);  // one contiguous run of blocks (leaves of few trees) per XCD
  const int t = by;
  const int s = bx * blockDim.x + threadIdx.x;
  if (s >= W) return;
  const int64_t wb = (int64_t)t * w.max_wave;
  const float v = w.values[wb + w.sim_uid[wb + s]];
  const int L = w.path_len[wb + s];
  const bool neg = sign_mode == OMQ_SIGN_LEAF_POSITIVE && ((L - 1) & 1);
  w.sim_value[wb + s] = neg ? -v : v;
}

// Groups are dealt to the lanes of all waves in a strided order (lane l of wave w takes groups
// w + (l + 64*i) * waves), so the few big groups of a level -- they are logged next to each
// other -- land in different waves.  A small group is folded by its lane after all of its
// member values have been fetched (the loads of a lane are issued together); a big group is
// folded by its wave: 64 member values at a time, one per lane, are read into scalar
// registers and added in order (the loads of the next 256 are in flight meanwhile).
//
// FUSED: the signed leaf value of a member is formed here from its unique leaf's value and its
// path length (as sim_value_kernel forms it), which saves that kernel's launch; used for waves
// of at most kFuseMaxWave simulations.  Larger waves have more groups per lane, and there the
// extra dependent load costs more than the launch (C3 and C4 backups were 6 % and 15 % slower).
constexpr int kFuseMaxWave = 512;

template <bool FUSED>
__global__ __launch_bounds__(kBackupThreads) void backup_groups_kernel(omq_forest f, omq_wave w,
                                                                       int vli, int sign_mode) {
  int bx = blockIdx.x, by = blockIdx.y;
  xcd_block(&bx, &by);  // one contiguous run of blocks (leaves of few trees) per XCD
  const int t = by;
  const int lane = lane_id();
  const int wib = threadIdx.x / kWave;
  const int64_t tb = (int64_t)t * f.capacity;
  const int64_t wb = (int64_t)t * w.max_wave;
  const int MW = w.max_wave, MD = w.max_depth;
  const int64_t gmax = (int64_t)MW * MD;
  const int G = w.gcount[t];
  const int waves_total = gridDim.x * (kBackupThreads / kWave);
  const int wave_global = bx * (kBackupThreads / kWave) + wib;
  const int32_t* uid = w.sim_uid + wb;
  const int32_t* plen = w.path_len + wb;
  const float* uval = w.values + wb;
  const float* svals = w.sim_value + wb;
  const bool leaf_pos = sign_mode == OMQ_SIGN_LEAF_POSITIVE;
  // signed leaf value of simulation s (sim_value_kernel's value)
  auto sv = [&](int s) {
    if (!FUSED) return svals[s];
    const float v = uval[uid[s]];
    return (leaf_pos && ((plen[s] - 1) & 1)) ? -v : v;
  };
  for (int i0 = 0; wave_global + i0 * waves_total < G; i0 += kWave) {
    const int g = wave_global + (i0 + lane) * waves_total;
    int p = 0, d = 0, seg = 0, m = 0;
    if (g < G) {
      const int4 rec = *reinterpret_cast<const int4*>(w.glog + ((int64_t)t * gmax + g) * 4);
      p = rec.x;
      d = rec.y;
      seg = rec.z;
      m = rec.w;
    }
    if (g < G && m <= kBigGroup) {
      const uint16_t* mem = w.gmembers + ((int64_t)t * MD + d) * MW + seg;
      float vals[kBigGroup];
#pragma unroll
      for (int i = 0; i < kBigGroup; ++i) vals[i] = i < m ? sv(mem[i]) : 0.0f;
      float acc = f.value_sums[tb + p];
      const bool odd = d & 1;
#pragma unroll
      for (int i = 0; i < kBigGroup; ++i)
        if (i < m) acc = acc + (odd ? -vals[i] : vals[i]);
      f.value_sums[tb + p] = acc;
      f.visit_counts[tb + p] += m - vli * m;
    }
    // big groups: the whole wave, one group at a time
    uint64_t big = __ballot(g < G && m > kBigGroup);
    while (big) {
      const int l = lowest_lane(big);
      big &= big - 1;
      const int bp = readlane_i(p, l), bd = readlane_i(d, l), bseg = readlane_i(seg, l),
                bm = readlane_i(m, l);
      const uint16_t* bmem = w.gmembers + ((int64_t)t * MD + bd) * MW + bseg;
      const bool odd = bd & 1;
      float acc = f.value_sums[tb + bp];
      // chunks of kBigChunk*64 members, software-pipelined over the two dependent loads: while
      // chunk c is folded in order, the values of chunk c+1 (from member ids loaded one chunk
      // earlier) and the member ids of chunk c+2 are in flight
      constexpr int kCh = kBigChunk * kWave;
      float xa[kBigChunk], xb[kBigChunk];
      int ib[kBigChunk];
#pragma unroll
      for (int u = 0; u < kBigChunk; ++u) {
        const int c = u * kWave + lane;
        xa[u] = c < bm ? sv(bmem[c]) : 0.0f;
        const int c1 = kCh + c;
        ib[u] = c1 < bm ? (int)bmem[c1] : 0;
      }
      for (int c0 = 0; c0 < bm; c0 += kCh) {
        const int cn = c0 + kCh;
#pragma unroll
        for (int u = 0; u < kBigChunk; ++u) {
          const int c = cn + u * kWave + lane;
          xb[u] = c < bm ? sv(ib[u]) : 0.0f;
          const int c2 = cn + kCh + u * kWave + lane;
          ib[u] = c2 < bm ? (int)bmem[c2] : 0;
        }
#pragma unroll
        for (int u = 0; u < kBigChunk; ++u) {
          const int cb = c0 + u * kWave;
          if (cb >= bm) break;
          // lanes 0..63 hold members cb..cb+63: add them in order from scalar registers (the
          // reads are independent, only the adds form a chain)
          const float x = odd ? -xa[u] : xa[u];
          if (bm - cb >= kWave) {
#pragma unroll
            for (int l = 0; l < kWave; ++l) acc = acc + readlane_f(x, l);
          } else {
            for (int l = 0; l < bm - cb; ++l) acc = acc + readlane_f(x, l);
          }
        }
#pragma unroll
        for (int u = 0; u < kBigChunk; ++u) xa[u] = xb[u];
      }
      if (lane == 0) {
        f.value_sums[tb + bp] = acc;
        f.visit_counts[tb + bp] += bm - vli * bm;
      }
    }
  }
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
  // group count is on the device; size the grid for a typical wave (groups ~ W * depth),
  // the kernel strides over the rest
  const int est_groups = W * 8;
  int blocks = (est_groups + kBackupThreads - 1) / kBackupThreads;
  if (blocks < 1) blocks = 1;
  if (blocks > 1024) blocks = 1024;
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
