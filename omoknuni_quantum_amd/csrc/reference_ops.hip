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
