// The reference's fused UCB selection operator over explicit CSR edges (gfx950).
//
// Reference: fused_ucb_selection_adapter_kernel (python/mcts/gpu/mcts_kernels.cu:1466-1512),
// registered as mcts::fused_ucb_selection (python/mcts/gpu/torch_custom_ops.py:108-193).  For
// parent p = node_indices[b], row [children_start[p], children_end[p]):
//     sqrt_parent = sqrtf((float)visit_counts[p])
//     ucb_i = (visit_counts[c_i] > 0 ? q_values[c_i] : 0) + c*P_i*sqrt_parent / (1 + n_i)
// (float32; c*P_i*sqrt_parent evaluated left to right), and the result is the row position of
// the first maximum above -1e10 (strict '>'), or -1 for an empty row.  Unlike the tree
// selection of omq_select, an unvisited child has no priority here: its q is 0.
//
// One wavefront per query: lanes stride the row, each keeping its first maximum; the wave then
// takes the largest score (order-preserving keys) and, among the lanes that hold it, the lowest
// row position.
#include "omq_common.h"

namespace omq {

constexpr int kUcbWavesPerBlock = 4;

__global__ void fused_ucb_kernel(const int32_t* node_indices, int batch,
                                 const int32_t* children_start, const int32_t* children_end,
                                 const int32_t* children, const float* q_values,
                                 const int32_t* visit_counts, const float* priors, float c_puct,
                                 int32_t* selected) {
  const int lane = lane_id();
  const int b = blockIdx.x * kUcbWavesPerBlock + (int)threadIdx.x / kWave;
  if (b >= batch) return;
  const int p = node_indices[b];
  const int start = children_start[p];
  const int end = children_end[p];
  if (start >= end) {
    if (lane == 0) selected[b] = -1;
    return;
  }
  const float sqrt_parent = sqrtf((float)visit_counts[p]);
  // lane-local first maximum above -1e10 (positions ascend within a lane)
  uint32_t best_key = 0u;
  int best_pos = 0x7FFFFFFF;
  float best = -1e10f;
  for (int i = start + lane; i < end; i += kWave) {
    const int child = children[i];
    const int n = visit_counts[child];
    const float q = n > 0 ? q_values[child] : 0.0f;
    const float exploration = c_puct * priors[i] * sqrt_parent / (1.0f + (float)n);
    const float ucb = q + exploration;
    if (ucb > best) {
      best = ucb;
      best_pos = i - start;
    }
  }
  if (best_pos != 0x7FFFFFFF) best_key = fkey(best + 0.0f);  // -0 -> +0
  const uint32_t top = wave_max_u32(best_key);
  int pos = -1;
  if (top != 0u) {
    const int mine = best_key == top ? best_pos : 0x7FFFFFFF;
    pos = (int)~wave_max_u32(~(uint32_t)mine);  // wave minimum
  }
  if (lane == 0) selected[b] = pos;
}

hipError_t launch_fused_ucb(const int32_t* node_indices, int batch, const int32_t* starts,
                            const int32_t* ends, const int32_t* children, const float* q,
                            const int32_t* visits, const float* priors, float c_puct,
                            int32_t* selected, hipStream_t st) {
  if (batch <= 0) return hipSuccess;
  const int blocks = (batch + kUcbWavesPerBlock - 1) / kUcbWavesPerBlock;
  hipLaunchKernelGGL(fused_ucb_kernel, dim3(blocks), dim3(kUcbWavesPerBlock * kWave), 0, st,
                     node_indices, batch, starts, ends, children, q, visits, priors, c_puct,
                     selected);
  return hipGetLastError();
}

}  // namespace omq

// ===========================================================================================
// The reference accelerator's remaining operators (MCTSGPUAccelerator,
// python/mcts/gpu/mcts_gpu_accelerator.py:81-207; kernels in python/mcts/gpu/mcts_kernels.cu).
// Their trees are the reference's GPU variant: a dense children table [num_nodes, max_children]
// whose rows end at the first negative entry, per-node arrays indexed by node, and CSR edges.
// Every sequential "first maximum by strict '>'" of the reference is taken here by one wave:
// lanes own row positions i = 64 k + lane, keep their first maximum, and the wave takes the
// largest key (order-preserving, -0 folded onto +0) and, among the lanes holding it, the
// lowest position -- the same element the sequential scan keeps.
// ===========================================================================================
namespace omq {

namespace {

constexpr int kRowWaves = 4;  // waves per block of the wave-per-item kernels

// The row position of the wave's first maximum: key = fkey(best + 0) of the lane's first
// maximum (0 when the lane has none), pos its position.  -1 when no lane has one.
__device__ inline int wave_first_max_pos(uint32_t key, int pos) {
  const uint32_t top = wave_max_u32(key);
  if (top == 0u) return -1;
  const int mine = (key == top) ? pos : 0x7FFFFFFF;
  return (int)~wave_max_u32(~(uint32_t)mine);  // wave minimum
}

// One child row of the dense table scanned by the wave up to its end (the first entry < 0 or
// >= num_nodes, or max_children); score(i, c) gives the score of position i, child c.  Returns
// the winning position (-1 without a score above -inf) and, through *child, its child; *end
// receives the number of positions in the row.
template <class Score>
__device__ inline int row_first_max(const int32_t* row, int max_children, int num_nodes,
                                    Score score, int* child, int* end) {
  const int lane = lane_id();
  float best = -INFINITY;
  int best_pos = 0x7FFFFFFF;
  int best_child = -1;
  int n = max_children;
  for (int base = 0; base < max_children; base += kWave) {
    const int i = base + lane;
    const int c = i < max_children ? row[i] : -1;
    const uint64_t stop = __ballot(i < max_children && (c < 0 || c >= num_nodes));
    const int lim = stop ? lowest_lane(stop) : kWave;
    if (lane < lim && i < max_children) {
      const float s = score(i, c);
      if (s > best) {
        best = s;
        best_pos = i;
        best_child = c;
      }
    }
    if (stop) {
      n = base + lim;
      break;
    }
  }
  *end = n;
  const uint32_t key = best_pos != 0x7FFFFFFF ? fkey(best + 0.0f) : 0u;
  const int pos = wave_first_max_pos(key, best_pos);
  *child = pos >= 0 ? readlane_i(best_child, pos & (kWave - 1)) : -1;
  return pos;
}

// ---- find_expansion_nodes ----------------------------------------------------------------
// Pass 1, one wave per path: flag[s] = the path's node when it needs expansion, else -1
// (written into out_nodes, which pass 2 compacts in place).
__global__ void expansion_flag_kernel(const int32_t* current_nodes, const uint8_t* valid_mask,
                                      int wave_size, const int32_t* children, int max_children,
                                      const int32_t* visit_counts, int num_nodes,
                                      int32_t* flag) {
  const int s = blockIdx.x * kRowWaves + (int)threadIdx.x / kWave;
  if (s >= wave_size) return;
  const int lane = lane_id();
  int out = -1;
  const int node = current_nodes[s];
  if (valid_mask[s] && node >= 0 && node < num_nodes && visit_counts[node] == 0) {
    const int32_t* row = children + (int64_t)node * max_children;
    bool any = false;
    for (int base = 0; base < max_children && !any; base += kWave) {
      const int i = base + lane;
      any = __ballot(i < max_children && row[i] >= 0) != 0ull;
    }
    if (!any) out = node;
  }
  if (lane == 0) flag[s] = out;
}

// Pass 2, one block: order-preserving compaction of the flags, in place, chunk by chunk (a
// chunk's entries are all read before any of its writes, and writes land at or below the
// entry they come from).
constexpr int kScanThreads = 1024;

template <class T>
__device__ inline T block_excl_scan(T v, T* wave_tot, T* total) {
  const int wid = (int)threadIdx.x / kWave, lane = lane_id();
  T x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const T y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  if (lane == kWave - 1) wave_tot[wid] = x;
  __syncthreads();
  T off = 0, tot = 0;
  for (int k = 0; k < kScanThreads / kWave; ++k) {
    const T t = wave_tot[k];
    off += k < wid ? t : 0;
    tot += t;
  }
  __syncthreads();  // wave_tot is reused by the next call
  *total = tot;
  return off + x - v;
}

__global__ void __launch_bounds__(kScanThreads)
expansion_compact_kernel(int32_t* nodes, int wave_size, int32_t* count) {
  __shared__ int wave_tot[kScanThreads / kWave];
  int done = 0;
  for (int base = 0; base < wave_size; base += kScanThreads) {
    const int s = base + (int)threadIdx.x;
    const int v = s < wave_size ? nodes[s] : -1;
    int tot;
    const int at = block_excl_scan<int>(v >= 0 ? 1 : 0, wave_tot, &tot);  // barriers inside
    if (v >= 0) nodes[done + at] = v;
    done += tot;
    __syncthreads();
  }
  if (threadIdx.x == 0) count[0] = done;
}

// ---- batched_ucb_selection ---------------------------------------------------------------
__global__ void batched_ucb_kernel(const float* q_values, const int32_t* visit_counts,
                                   int num_children, const int32_t* parent_visits,
                                   const float* priors, const int32_t* row_ptr,
                                   const int32_t* col_indices, int batch, float c_puct,
                                   int32_t* selected, float* scores) {
  const int b = blockIdx.x * kRowWaves + (int)threadIdx.x / kWave;
  if (b >= batch) return;
  const int lane = lane_id();
  const int start = row_ptr[b];
  const int end = row_ptr[b + 1];
  if (start < 0 || end <= start) {
    if (lane == 0) {
      selected[b] = (start >= 0 && end == start) ? -1 : 0;
      if (scores) scores[b] = 0.0f;
    }
    return;
  }
  const float sqrt_parent = sqrtf((float)parent_visits[b] + 1.0f);
  float best = -1e10f;
  int best_pos = 0x7FFFFFFF;
  const int hi = min(end, num_children);
  for (int i = start + lane; i < hi; i += kWave) {
    const int c = col_indices[i];
    if (c < 0 || c >= num_children) continue;
    const float n = (float)visit_counts[c];
    const float q = n > 0.0f ? q_values[c] : 0.0f;
    const float exploration = c_puct * priors[i] * sqrt_parent / (1.0f + n);
    const float ucb = q + exploration;
    if (ucb > best) {
      best = ucb;
      best_pos = i - start;
    }
  }
  const uint32_t key = best_pos != 0x7FFFFFFF ? fkey(best + 0.0f) : 0u;
  const int pos = wave_first_max_pos(key, best_pos);
  if (pos < 0) {
    if (lane == 0) {
      selected[b] = 0;
      if (scores) scores[b] = -1e10f;
    }
  } else if (best_pos == pos) {  // the one lane holding the winner
    selected[b] = pos;
    if (scores) scores[b] = best;
  }
}

// ---- fused_select_expand -------------------------------------------------------------------
__global__ void fused_select_expand_kernel(const int32_t* roots, int num_paths,
                                           const int32_t* children, int num_nodes,
                                           int max_children, const int32_t* visit_counts,
                                           const float* q_values, const float* prior_probs,
                                           const uint8_t* is_expanded, int max_depth,
                                           float c_puct, int32_t* paths, int32_t* path_lengths,
                                           int32_t* expand_nodes, uint8_t* needs_expansion) {
  const int w = blockIdx.x * kRowWaves + (int)threadIdx.x / kWave;
  if (w >= num_paths) return;
  const int lane = lane_id();
  int32_t* path = paths + (int64_t)w * max_depth;
  int node = roots[w];
  if (lane == 0) path[0] = node;
  int depth = 0;
  bool leaf = false;
  if (node < 0 || node >= num_nodes) {
    leaf = true;
  } else {
    while (depth < max_depth - 1) {
      int next = -1;
      if (is_expanded[node]) {
        const float sqrt_parent = sqrtf((float)visit_counts[node]);
        int end;
        row_first_max(children + (int64_t)node * max_children, max_children, num_nodes,
                      [&](int, int c) {
                        const int n = visit_counts[c];
                        if (n == 0) return INFINITY;
                        return q_values[c] + c_puct * prior_probs[c] * sqrt_parent /
                                                 (1.0f + (float)n);
                      },
                      &next, &end);
      }
      if (next < 0) {
        leaf = true;
        break;
      }
      node = next;
      ++depth;
      if (lane == 0) path[depth] = node;
    }
  }
  for (int i = depth + 1 + lane; i < max_depth; i += kWave) path[i] = -1;
  if (lane == 0) {
    path_lengths[w] = leaf ? depth + 1 : 0;
    expand_nodes[w] = leaf ? node : 0;
    needs_expansion[w] = leaf ? 1 : 0;
  }
}

// sqrt_parent of the second form: 1 / sqrt(r), r = 1 / (float)(pv + 1) in float32, with the
// square root and its reciprocal in float64, rounded once to float32.
__device__ inline float rsqrt_of_rcp(int pv) {
  const float r = 1.0f / (float)(pv + 1);
  return (float)(1.0 / sqrt((double)r));
}

__global__ void fused_select_expand_opt_kernel(const int32_t* roots, int num_paths,
                                               const int32_t* children, int num_nodes,
                                               int max_children, const int32_t* visit_counts,
                                               const float* value_sums, const float* priors,
                                               int max_depth, float c_puct, float* ucb_scores,
                                               int32_t* paths, int32_t* path_lengths) {
  const int w = blockIdx.x * kRowWaves + (int)threadIdx.x / kWave;
  if (w >= num_paths) return;
  const int lane = lane_id();
  int32_t* path = paths + (int64_t)w * max_depth;
  float* ucb_row = ucb_scores + (int64_t)w * max_children;
  int node = roots[w];
  if (lane == 0) path[0] = node;
  int depth = 0;
  int scored = 0;  // positions of the root's row that received a score
  if (node >= 0 && node < num_nodes) {
    while (depth < max_depth - 1 && depth < 32) {
      const int pv = visit_counts[node];
      if (pv == 0) break;
      const float sqrt_parent = rsqrt_of_rcp(pv);
      const bool root = depth == 0;
      int next, end;
      row_first_max(children + (int64_t)node * max_children, max_children, num_nodes,
                    [&](int i, int c) {
                      const int n = visit_counts[c];
                      const float q = n > 0 ? value_sums[c] * (1.0f / ((float)n + 1e-8f))
                                            : 0.0f;
                      const float expl = c_puct * priors[c] * sqrt_parent *
                                         (1.0f / (1.0f + (float)n));
                      const float u = q + expl;
                      if (root) ucb_row[i] = u;
                      return u;
                    },
                    &next, &end);
      if (root) scored = end;
      if (next < 0) break;
      node = next;
      ++depth;
      if (lane == 0) path[depth] = node;
    }
  }
  for (int i = scored + lane; i < max_children; i += kWave) ucb_row[i] = 0.0f;
  for (int i = depth + 1 + lane; i < max_depth; i += kWave) path[i] = -1;
  if (lane == 0) path_lengths[w] = depth + 1;
}

// ---- batched_add_children ------------------------------------------------------------------
// Pass 1, one block: the batch-order exclusive scan of the child counts of the parents that
// take nodes.  For item b it stores the item's first node, or -1 when nothing is written for
// it (invalid parent, no child, or past capacity), in child_indices[b * max_children] (pass 2
// reads it back before it writes that row), and advances both counters by the total.
__global__ void __launch_bounds__(kScanThreads)
add_children_alloc_kernel(const int32_t* parent_indices, const int32_t* num_children,
                          int batch, int32_t* node_counter, int32_t* edge_counter,
                          int max_nodes, int max_children, int max_edges,
                          int32_t* child_indices) {
  __shared__ int64_t wave_tot[kScanThreads / kWave];
  const int64_t node0 = node_counter[0], edge0 = edge_counter[0];
  int64_t done = 0;
  for (int base = 0; base < batch; base += kScanThreads) {
    const int b = base + (int)threadIdx.x;
    int64_t n = 0;
    if (b < batch) {
      const int p = parent_indices[b];
      const int k = num_children[b];
      n = (p >= 0 && p < max_nodes && k > 0) ? k : 0;
    }
    int64_t tot;
    const int64_t at = block_excl_scan<int64_t>(n, wave_tot, &tot);  // barriers inside
    if (b < batch) {
      const int64_t nd = node0 + done + at, ed = edge0 + done + at;
      const bool fits = n > 0 && nd >= 0 && ed >= 0 && nd + n <= max_nodes && ed + n <= max_edges;
      child_indices[(int64_t)b * max_children] = fits ? (int32_t)nd : -1;
    }
    done += tot;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    node_counter[0] = (int32_t)(uint32_t)((uint64_t)node0 + (uint64_t)done);
    edge_counter[0] = (int32_t)(uint32_t)((uint64_t)edge0 + (uint64_t)done);
  }
}

// Pass 2, one wave per item: the writes of the item's children (positions i < min(n,
// max_children)), and its row of child_indices (-1 where nothing is written).  The item's
// first node comes from pass 1; its first edge is first node + (edge counter - node counter),
// both counters having advanced by the same total (modulo 2^32, as int32 atomics wrap).  Two
// items with the same parent write the same children-table slots; which one lands last is not
// specified, as in the reference.
__global__ void add_children_write_kernel(
    const int32_t* parent_indices, int batch, const int32_t* actions, const float* priors,
    const int32_t* num_children, const int32_t* node_counter, const int32_t* edge_counter,
    int32_t* children, int32_t* parent_indices_out, int32_t* parent_actions_out,
    float* node_priors_out, int32_t* visit_counts_out, float* value_sums_out,
    int32_t* col_indices, int32_t* edge_actions, float* edge_priors, int max_children,
    int32_t* child_indices) {
  const int b = blockIdx.x * kRowWaves + (int)threadIdx.x / kWave;
  if (b >= batch) return;
  const int lane = lane_id();
  const int64_t rb = (int64_t)b * max_children;
  int32_t* crow = child_indices + rb;
  const int32_t first = crow[0];  // every store below depends on this load
  if (first < 0) {
    for (int i = lane; i < max_children; i += kWave) crow[i] = -1;
    return;
  }
  const int p = parent_indices[b];
  const int n = min(num_children[b], max_children);
  const uint32_t delta = (uint32_t)edge_counter[0] - (uint32_t)node_counter[0];
  for (int i = lane; i < max_children; i += kWave) {
    if (i < n) {
      const int32_t c = first + i;
      const int32_t e = (int32_t)((uint32_t)c + delta);
      const int32_t a = actions[rb + i];
      const float pr = priors[rb + i];
      parent_indices_out[c] = p;
      parent_actions_out[c] = a;
      node_priors_out[c] = pr;
      visit_counts_out[c] = 0;
      value_sums_out[c] = 0.0f;
      children[(int64_t)p * max_children + i] = c;  // p < max_nodes, i < max_children
      col_indices[e] = c;
      edge_actions[e] = a;
      edge_priors[e] = pr;
      crow[i] = c;
    } else {
      crow[i] = -1;
    }
  }
}

inline int row_blocks(int items) { return (items + kRowWaves - 1) / kRowWaves; }

// ---- parallel_select_with_virtual_loss -------------------------------------------------------
// One wave per simulation over its parent's row of the dense table (every position up to
// max_children; negative entries and entries past the node arrays are skipped, the row does
// not end at them).  Effective visits n = N + VLc and value W + VLc * vl (float), Q = W / n
// for n > 0, else 0; the parent's sqrt(N + 1) takes no virtual loss; with the legal filter,
// a non-root parent's child whose action is illegal for the simulation is skipped.  The first
// maximum above -inf (strict '>', lowest position on ties) gives the child, else -1.
__global__ void parallel_select_vl_kernel(const int32_t* parent_nodes, int num_sims,
                                          const int32_t* children, int num_rows,
                                          int max_children, int children_stride,
                                          const int32_t* visit_counts, const int32_t* vl_counts,
                                          const float* value_sums, int num_nodes,
                                          const float* priors, int priors_stride,
                                          const uint8_t* legal_masks, int action_space,
                                          const int32_t* child_actions, float c_puct,
                                          float vl_value, int32_t* selected) {
  const int s = blockIdx.x * kRowWaves + (int)threadIdx.x / kWave;
  if (s >= num_sims) return;
  const int lane = lane_id();
  const int p = parent_nodes[s];
  if (p < 0 || p >= num_rows || p >= num_nodes) {
    if (lane == 0) selected[s] = -1;
    return;
  }
  const float sqrt_parent = sqrtf((float)(visit_counts[p] + 1));
  const bool filter = legal_masks != nullptr && p != 0;
  const uint8_t* legal = filter ? legal_masks + (int64_t)s * action_space : nullptr;
  const int32_t* row = children + (int64_t)p * children_stride;
  float best = -INFINITY;
  int best_pos = 0x7FFFFFFF, best_child = -1;
  for (int i = lane; i < max_children; i += kWave) {
    const int c = row[i];
    if (c < 0 || c >= num_nodes) continue;
    if (filter) {
      const int a = child_actions[c];
      if (a >= 0 && a < action_space && !legal[a]) continue;
    }
    float prior;
    if (priors_stride > 0) {  // per-simulation priors [num_sims, priors_stride]
      if (c >= priors_stride) continue;
      prior = priors[(int64_t)s * priors_stride + c];
    } else {
      prior = priors[c];
    }
    const int vc = vl_counts[c];
    const int n = visit_counts[c] + vc;
    const float w = value_sums[c] + (float)vc * vl_value;
    const float q = n > 0 ? w / (float)n : 0.0f;
    const float ucb = q + c_puct * prior * sqrt_parent / (1.0f + (float)n);
    if (ucb > best) {
      best = ucb;
      best_pos = i;
      best_child = c;
    }
  }
  const uint32_t key = best_pos != 0x7FFFFFFF ? fkey(best + 0.0f) : 0u;
  const int pos = wave_first_max_pos(key, best_pos);
  const int child = pos >= 0 ? readlane_i(best_child, pos & (kWave - 1)) : -1;
  if (lane == 0) selected[s] = child;
}

// ---- fused_ucb_with_noise ------------------------------------------------------------------
// One wave per simulation over the shared row of num_children: prior (1 - eps) P + eps * noise
// of the simulation, ucb = q + c * prior' * sqrt_parent / (1 + N), the first maximum above
// -1e10 (strict '>'), or position 0 when none is above it.
__global__ void fused_ucb_noise_kernel(const float* q_values, const int32_t* visit_counts,
                                       const float* priors, int num_children,
                                       const float* noise, int num_sims,
                                       float parent_visits_sqrt, float c_puct, float epsilon,
                                       int32_t* selected) {
  const int s = blockIdx.x * kRowWaves + (int)threadIdx.x / kWave;
  if (s >= num_sims) return;
  const int lane = lane_id();
  const float* nz = noise + (int64_t)s * num_children;
  const float keep = 1.0f - epsilon;
  float best = -1e10f;
  int best_pos = 0x7FFFFFFF;
  for (int c = lane; c < num_children; c += kWave) {
    const float mixed = keep * priors[c] + epsilon * nz[c];
    const float ucb = q_values[c] + c_puct * mixed * parent_visits_sqrt /
                                        (1.0f + (float)visit_counts[c]);
    if (ucb > best) {
      best = ucb;
      best_pos = c;
    }
  }
  const uint32_t key = best_pos != 0x7FFFFFFF ? fkey(best + 0.0f) : 0u;
  const int pos = wave_first_max_pos(key, best_pos);
  if (lane == 0) selected[s] = pos >= 0 ? pos : 0;
}

// ---- batched_ucb_selection_dense ---------------------------------------------------------
// One wave per batch item over its slots: a slot counts when valid_mask is set and its child
// lies in [0, num_valid_children); value = child_values when the child is visited, else 0;
// ucb = value + c * P_slot * sqrt(pv + 1) / (1 + N).  The child of the first maximum above
// -1e10 (strict '>'), or -1.
__global__ void batched_ucb_dense_kernel(const int32_t* batch_children, const float* batch_priors,
                                         const int32_t* parent_visits, const uint8_t* valid_mask,
                                         int batch, int max_children, const int32_t* child_visits,
                                         const float* child_values, int num_valid,
                                         float c_puct, int32_t* selected) {
  const int b = blockIdx.x * kRowWaves + (int)threadIdx.x / kWave;
  if (b >= batch) return;
  const int lane = lane_id();
  const int64_t rb = (int64_t)b * max_children;
  const float sqrt_parent = sqrtf((float)parent_visits[b] + 1.0f);
  float best = -1e10f;
  int best_pos = 0x7FFFFFFF, best_child = -1;
  for (int i = lane; i < max_children; i += kWave) {
    if (!valid_mask[rb + i]) continue;
    const int c = batch_children[rb + i];
    if (c < 0 || c >= num_valid) continue;
    const int n = child_visits[c];
    const float v = n > 0 ? child_values[c] : 0.0f;
    const float ucb = v + c_puct * batch_priors[rb + i] * sqrt_parent / (1.0f + (float)n);
    if (ucb > best) {
      best = ucb;
      best_pos = i;
      best_child = c;
    }
  }
  const uint32_t key = best_pos != 0x7FFFFFFF ? fkey(best + 0.0f) : 0u;
  const int pos = wave_first_max_pos(key, best_pos);
  const int child = pos >= 0 ? readlane_i(best_child, pos & (kWave - 1)) : -1;
  if (lane == 0) selected[b] = child;
}

}  // namespace

hipError_t launch_find_expansion_nodes(const int32_t* current_nodes, const uint8_t* valid_mask,
                                       int wave_size, const int32_t* children, int max_children,
                                       const int32_t* visit_counts, int num_nodes,
                                       int32_t* out_nodes, int32_t* out_count, hipStream_t st) {
  if (wave_size > 0)
    hipLaunchKernelGGL(expansion_flag_kernel, dim3(row_blocks(wave_size)),
                       dim3(kRowWaves * kWave), 0, st, current_nodes, valid_mask, wave_size,
                       children, max_children, visit_counts, num_nodes, out_nodes);
  hipLaunchKernelGGL(expansion_compact_kernel, dim3(1), dim3(kScanThreads), 0, st, out_nodes,
                     wave_size, out_count);
  return hipGetLastError();
}

hipError_t launch_batched_ucb(const float* q_values, const int32_t* visit_counts,
                              int num_children, const int32_t* parent_visits,
                              const float* priors, const int32_t* row_ptr,
                              const int32_t* col_indices, int batch, float c_puct,
                              int32_t* selected, float* scores, hipStream_t st) {
  if (batch <= 0) return hipSuccess;
  hipLaunchKernelGGL(batched_ucb_kernel, dim3(row_blocks(batch)), dim3(kRowWaves * kWave), 0,
                     st, q_values, visit_counts, num_children, parent_visits, priors, row_ptr,
                     col_indices, batch, c_puct, selected, scores);
  return hipGetLastError();
}

hipError_t launch_fused_select_expand(const int32_t* roots, int num_paths,
                                      const int32_t* children, int num_nodes, int max_children,
                                      const int32_t* visit_counts, const float* q_values,
                                      const float* prior_probs, const uint8_t* is_expanded,
                                      int max_depth, float c_puct, int32_t* paths,
                                      int32_t* path_lengths, int32_t* expand_nodes,
                                      uint8_t* needs_expansion, hipStream_t st) {
  if (num_paths <= 0) return hipSuccess;
  hipLaunchKernelGGL(fused_select_expand_kernel, dim3(row_blocks(num_paths)),
                     dim3(kRowWaves * kWave), 0, st, roots, num_paths, children, num_nodes,
                     max_children, visit_counts, q_values, prior_probs, is_expanded, max_depth,
                     c_puct, paths, path_lengths, expand_nodes, needs_expansion);
  return hipGetLastError();
}

hipError_t launch_fused_select_expand_opt(const int32_t* roots, int num_paths,
                                          const int32_t* children, int num_nodes,
                                          int max_children, const int32_t* visit_counts,
                                          const float* value_sums, const float* priors,
                                          int max_depth, float c_puct, float* ucb_scores,
                                          int32_t* paths, int32_t* path_lengths,
                                          hipStream_t st) {
  if (num_paths <= 0) return hipSuccess;
  hipLaunchKernelGGL(fused_select_expand_opt_kernel, dim3(row_blocks(num_paths)),
                     dim3(kRowWaves * kWave), 0, st, roots, num_paths, children, num_nodes,
                     max_children, visit_counts, value_sums, priors, max_depth, c_puct,
                     ucb_scores, paths, path_lengths);
  return hipGetLastError();
}

hipError_t launch_batched_add_children(
    const int32_t* parent_indices, int batch, const int32_t* actions, const float* priors,
    const int32_t* num_children, int32_t* node_counter, int32_t* edge_counter,
    int32_t* children, int32_t* parent_indices_out, int32_t* parent_actions_out,
    float* node_priors_out, int32_t* visit_counts_out, float* value_sums_out,
    int32_t* col_indices, int32_t* edge_actions, float* edge_priors, int max_nodes,
    int max_children, int max_edges, int32_t* child_indices, hipStream_t st) {
  if (batch <= 0) return hipSuccess;
  hipLaunchKernelGGL(add_children_alloc_kernel, dim3(1), dim3(kScanThreads), 0, st,
                     parent_indices, num_children, batch, node_counter, edge_counter, max_nodes,
                     max_children, max_edges, child_indices);
  hipLaunchKernelGGL(add_children_write_kernel, dim3(row_blocks(batch)),
                     dim3(kRowWaves * kWave), 0, st, parent_indices, batch, actions, priors,
                     num_children, node_counter, edge_counter, children, parent_indices_out,
                     parent_actions_out, node_priors_out, visit_counts_out, value_sums_out,
                     col_indices, edge_actions, edge_priors, max_children, child_indices);
  return hipGetLastError();
}

hipError_t launch_parallel_select_vl(const int32_t* parent_nodes, int num_sims,
                                     const int32_t* children, int num_rows, int max_children,
                                     int children_stride, const int32_t* visit_counts,
                                     const int32_t* vl_counts, const float* value_sums,
                                     int num_nodes, const float* priors, int priors_stride,
                                     const uint8_t* legal_masks, int action_space,
                                     const int32_t* child_actions, float c_puct, float vl_value,
                                     int32_t* selected, hipStream_t st) {
  if (num_sims <= 0) return hipSuccess;
  hipLaunchKernelGGL(parallel_select_vl_kernel, dim3(row_blocks(num_sims)),
                     dim3(kRowWaves * kWave), 0, st, parent_nodes, num_sims, children, num_rows,
                     max_children, children_stride, visit_counts, vl_counts, value_sums,
                     num_nodes, priors, priors_stride, legal_masks, action_space, child_actions,
                     c_puct, vl_value, selected);
  return hipGetLastError();
}

hipError_t launch_fused_ucb_noise(const float* q_values, const int32_t* visit_counts,
                                  const float* priors, int num_children, const float* noise,
                                  int num_sims, float parent_visits_sqrt, float c_puct,
                                  float epsilon, int32_t* selected, hipStream_t st) {
  if (num_sims <= 0) return hipSuccess;
  hipLaunchKernelGGL(fused_ucb_noise_kernel, dim3(row_blocks(num_sims)), dim3(kRowWaves * kWave),
                     0, st, q_values, visit_counts, priors, num_children, noise, num_sims,
                     parent_visits_sqrt, c_puct, epsilon, selected);
  return hipGetLastError();
}

hipError_t launch_batched_ucb_dense(const int32_t* batch_children, const float* batch_priors,
                                    const int32_t* parent_visits, const uint8_t* valid_mask,
                                    int batch, int max_children, const int32_t* child_visits,
                                    const float* child_values, int num_valid, float c_puct,
                                    int32_t* selected, hipStream_t st) {
  if (batch <= 0) return hipSuccess;
  hipLaunchKernelGGL(batched_ucb_dense_kernel, dim3(row_blocks(batch)), dim3(kRowWaves * kWave), 0,
                     st, batch_children, batch_priors, parent_visits, valid_mask, batch,
                     max_children, child_visits, child_values, num_valid, c_puct, selected);
  return hipGetLastError();
}

}  // namespace omq
