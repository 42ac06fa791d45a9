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
// first child, and all threads then write the level's children together. Two grid-wide
// kernels follow: one gathers the kept nodes' fields into a workspace, the other writes them
// over the front of the tree. The workspace holds eight int32 arrays of `capacity` entries
// per tree.
#include <mutex>

#include "omq_common.h"

namespace omq {

constexpr int kShiftThreads = 1024;
constexpr int kShiftWaves = kShiftThreads / kWave;

// Workgroup barrier that orders LDS only: global loads in flight stay in flight across it
// (__syncthreads also waits for them).
__device__ inline void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Exclusive scans of two values per thread over the workgroup, together (one pair of
// barriers); totals through *ta, *tb.  s_wtot holds 2 * kShiftWaves ints.
__device__ inline void shift_block_scan2(int a, int b, int* s_wtot, int* ea, int* eb, int* ta,
                                         int* tb) {
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  int wa, wb;
  const int xa = wave_excl_scan(a, &wa);
  const int xb = wave_excl_scan(b, &wb);
  if (lane_id() == 0) {
    s_wtot[wave] = wa;
    s_wtot[kShiftWaves + wave] = wb;
  }
  lds_barrier();
  int ba = 0, bb = 0, sa = 0, sb = 0;
  for (int i = 0; i < kShiftWaves; ++i) {
    const int x = s_wtot[i], y = s_wtot[kShiftWaves + i];
    if (i < wave) {
      ba += x;
      bb += y;
    }
    sa += x;
    sb += y;
  }
  lds_barrier();  // s_wtot is reused by the next scan
  *ea = ba + xa;
  *eb = bb + xb;
  *ta = sa;
  *tb = sb;
}

// Breadth-first numbering of tree t's kept nodes (one workgroup per tree).  Writes, for new
// id i: old_of_new[i], npar[i], nfirst[i], nnch[i]; then num_nodes[t] = kept count.  npar[0]
// is -1 for a tree to move and -2 for a tree left unchanged (no shift, or an inconsistent row:
// a row that leaves [0, num_nodes), or more kept nodes than num_nodes, as from a cycle).
// A level is taken in chunks of kShiftPer consecutive nodes per thread, so that the row loads
// of a chunk are in flight together.  The chunk's children are written in tiles of 64
// consecutive new ids, one tile per wave at a time: the chunk's nodes with children are
// compacted (their first child's offset strictly increasing), the tile's first node is found
// by a two-level search over that list (64 samples, then 64 entries: two LDS reads per lane),
// and each lane walks forward from it to the node of its own id.
constexpr int kShiftPer = 4;
constexpr int kShiftChunk = kShiftThreads * kShiftPer;

__global__ __launch_bounds__(kShiftThreads) void shift_order_kernel(omq_forest f,
                                                                    const int32_t* new_roots,
                                                                    int32_t* ws) {
  __shared__ int s_wtot[2 * kShiftWaves];
  __shared__ int s_cex[kShiftChunk];  // compacted nodes with children: first child's offset
  __shared__ int s_cof[kShiftChunk];  //   their old row offset
  __shared__ int s_cid[kShiftChunk];  //   their position in the chunk
  __shared__ int s_bad;               // a row of the chunk is inconsistent
  const int t = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int cap = f.capacity;
  const int64_t tb = (int64_t)t * cap;
  int32_t* old_of_new = ws + (int64_t)t * cap * 8;
  int32_t* npar = old_of_new + cap;
  int32_t* nfirst = old_of_new + 2 * (int64_t)cap;
  int32_t* nnch = old_of_new + 3 * (int64_t)cap;
  const int r = new_roots[t];
  const int n_old = f.num_nodes[t];
  if (r <= 0 || r >= n_old) {  // 0: already the root; -1: no shift
    if (tid == 0) npar[0] = -2;
    return;
  }
  if (tid == 0) {
    old_of_new[0] = r;
    s_bad = 0;
  }
  __syncthreads();
  // level [lo, hi) of new ids; its children get [hi, next)
  int lo = 0, hi = 1, next = 1;
  bool bad = false;
  // The rows of a level's next chunk are loaded while the current chunk is processed: a
  // level's new-to-old ids were all written before the level began, and the barriers inside a
  // chunk order LDS only, so the loads stay in flight until the chunk's end.
  int pk[kShiftPer], pof[kShiftPer];
  auto load_rows = [&](int c0) {
    const int i0 = c0 + tid * kShiftPer;
#pragma unroll
    for (int e = 0; e < kShiftPer; ++e) {
      pk[e] = 0;
      pof[e] = 0;
      if (i0 + e < hi) {
        const int old = old_of_new[i0 + e];
        pk[e] = f.num_children[tb + old];
        pof[e] = f.first_child[tb + old];
      }
    }
  };
  while (lo < hi && !bad) {
    load_rows(lo);
    for (int c0 = lo; c0 < hi; c0 += kShiftChunk) {
      const int i0 = c0 + tid * kShiftPer;  // this thread's nodes: i0 .. i0+kShiftPer-1
      int k[kShiftPer], of[kShiftPer];
#pragma unroll
      for (int e = 0; e < kShiftPer; ++e) {
        k[e] = pk[e];
        of[e] = pof[e];
      }
      if (c0 + kShiftChunk < hi) load_rows(c0 + kShiftChunk);
      bool row_bad = false;
      int mine = 0, nzm = 0;
#pragma unroll
      for (int e = 0; e < kShiftPer; ++e) {
        if (i0 + e < hi && (k[e] < 0 || (k[e] > 0 && (of[e] < 0 || (int64_t)of[e] + k[e] >= n_old)))) {
          row_bad = true;
          k[e] = 0;
        }
        mine += k[e];
        nzm += k[e] > 0 ? 1 : 0;
      }
      if (row_bad) s_bad = 1;  // (read after the scan's barriers)
      int tot, nz, ex, zx;
      shift_block_scan2(mine, nzm, s_wtot, &ex, &zx, &tot, &nz);
      const bool any_bad = s_bad != 0;
      if (any_bad || next + tot > n_old) {
        bad = true;
        break;
      }
#pragma unroll
      for (int e = 0; e < kShiftPer; ++e) {
        const int i = i0 + e;
        if (i < hi) {
          nnch[i] = k[e];
          nfirst[i] = k[e] > 0 ? next + ex - 1 : -1;
        }
        if (k[e] > 0) {
          s_cex[zx] = ex;
          s_cof[zx] = of[e];
          s_cid[zx] = tid * kShiftPer + e;
          ++zx;
        }
        ex += k[e];
      }
      lds_barrier();
      // the chunk's children, tile by tile: output q belongs to the last listed node j with
      // s_cex[j] <= q, as its child q - s_cex[j]
      for (int q0 = wave * kWave; q0 < tot; q0 += kShiftThreads) {
        // the tile's first node: a sample every 64 entries, then the entries after the sample
        const int si = lane * kWave;
        const uint64_t b1 = __ballot(si < nz && s_cex[si] <= q0);  // lane 0 always qualifies
        const int L = kWave - 1 - __clzll(b1);
        const int sj = L * kWave + lane;
        const uint64_t b2 = __ballot(sj < nz && s_cex[sj] <= q0);
        int j = L * kWave + (kWave - 1 - __clzll(b2));
        const int q = q0 + lane;
        if (q < tot) {
          // forward to the last node starting at or before q (at most nz - 1 - j steps)
          while (j + 1 < nz && s_cex[j + 1] <= q) ++j;
          old_of_new[next + q] = s_cof[j] + 1 + (q - s_cex[j]);  // child of edge of+x is node of+x+1
          npar[next + q] = c0 + s_cid[j];
        }
      }
      next += tot;
      __syncthreads();
    }
    lo = hi;
    hi = next;
  }
  if (tid == 0) {
    npar[0] = bad ? -2 : -1;
    if (!bad) f.num_nodes[t] = next;
  }
}

// Gathers the kept nodes' N, W, P and action into the workspace (grid-stride over new ids).
__global__ void shift_gather_kernel(omq_forest f, int32_t* ws) {
  const int t = blockIdx.y;
  const int cap = f.capacity;
  const int64_t tb = (int64_t)t * cap;
  const int32_t* old_of_new = ws + (int64_t)t * cap * 8;
  const int32_t* npar = old_of_new + cap;
  if (npar[0] != -1) return;
  int32_t* nN = const_cast<int32_t*>(old_of_new) + 4 * (int64_t)cap;
  float* nW = reinterpret_cast<float*>(nN + cap);
  float* nP = reinterpret_cast<float*>(nN + 2 * (int64_t)cap);
  int32_t* nA = nN + 3 * (int64_t)cap;
  const int n_new = f.num_nodes[t];
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n_new; i += gridDim.x * blockDim.x) {
    const int64_t o = tb + old_of_new[i];
    nN[i] = f.visit_counts[o];
    nW[i] = f.value_sums[o];
    nP[i] = f.priors[o];
    nA[i] = i == 0 ? -1 : f.actions[o];
  }
}

// Writes the compacted tree over the front of the tree's arrays.
__global__ void shift_write_kernel(omq_forest f, const int32_t* ws) {
  const int t = blockIdx.y;
  const int cap = f.capacity;
  const int64_t tb = (int64_t)t * cap;
  const int32_t* base = ws + (int64_t)t * cap * 8;
  const int32_t* npar = base + cap;
  if (npar[0] != -1) return;
  const int32_t* nfirst = base + 2 * (int64_t)cap;
  const int32_t* nnch = base + 3 * (int64_t)cap;
  const int32_t* nN = base + 4 * (int64_t)cap;
  const float* nW = reinterpret_cast<const float*>(nN + cap);
  const float* nP = reinterpret_cast<const float*>(nN + 2 * (int64_t)cap);
  const int32_t* nA = nN + 3 * (int64_t)cap;
  const int n_new = f.num_nodes[t];
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n_new; i += gridDim.x * blockDim.x) {
    const int64_t d = tb + i;
    f.visit_counts[d] = nN[i];
    f.value_sums[d] = nW[i];
    f.priors[d] = nP[i];
    f.parents[d] = npar[i];
    f.first_child[d] = nfirst[i];
    f.num_children[d] = nnch[i];
    f.actions[d] = nA[i];
  }
}

// ---- the workspace of omq_shift_root_noalloc ----------------------------------------------
// A file-scope device array, one copy per GPU the library runs on, held until the process
// ends.  Its address on a device is looked up once per device, with that device current
// (hipGetSymbolAddress); host code never passes the array's name to a kernel.  Every entry the
// shift kernels read is written earlier in the same call, so nothing has to start at zero.
// Calls that overlap on one GPU share the array and race.
static __device__ __align__(256) int32_t scratch[OMQ_NOALLOC_SHIFT_INTS];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
int32_t* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

// The address of this device's scratch (looked up on the first call on the device).
hipError_t shift_scratch(int32_t** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = static_cast<int32_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

hipError_t launch_shift_root(const omq_forest& f, const int32_t* new_roots, int32_t* ws,
                             hipStream_t st) {
  hipLaunchKernelGGL(shift_order_kernel, dim3(f.num_trees), dim3(kShiftThreads), 0, st, f,
                     new_roots, ws);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int blocks = (int)std::min<int64_t>(64, ((int64_t)f.capacity + 255) / 256);
  hipLaunchKernelGGL(shift_gather_kernel, dim3(blocks, f.num_trees), dim3(256), 0, st, f, ws);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(shift_write_kernel, dim3(blocks, f.num_trees), dim3(256), 0, st, f, ws);
  return hipGetLastError();
}

}  // namespace omq

// ===========================================================================================
// The reference's two-step subtree API: parallel_bfs_subtree and extract_subtree_edges
// (python/mcts/gpu/mcts_kernels.cu:2095-2337, bound at :2396-2408), over a CSR graph
// (row_ptr [max_nodes + 1], col_indices [num_edges]).  Their callers are
// python/mcts/gpu/gpu_bfs.py:49,149 and python/mcts/gpu/compact_subtree.py:220.
//   - BFS: breadth-first from root_idx, each level's nodes in order and each row's children in
//     row order; a child not yet in the subtree gets the next new index at its first
//     occurrence (the order of the reference's fallback, gpu_bfs.py:70-127, and of a FIFO
//     queue).  Children outside [0, max_nodes) are skipped.  The reference kernel numbers
//     children in the order its atomics land and marks a bool array through 32-bit CAS at the
//     child's index (touching the three bytes after it and reading past the array): its order
//     is one of the orders that can arise, and no other.
//   - Edges: for every node of the subtree in ascending old index, the edges of its row (in
//     row order) whose child lies in the subtree, as (new parent, new child, action); the
//     reference appends them in atomic order, of which this is one.
// ===========================================================================================
namespace omq {

constexpr int kBfsThreads = 1024;
constexpr int kBfsWaves = kBfsThreads / kWave;

// exclusive scan of one int64 per thread over the workgroup; total through *tot
__device__ inline int64_t bfs_block_scan(int64_t v, int64_t* s_wtot, int64_t* tot) {
  const int wave = (int)threadIdx.x / kWave, lane = lane_id();
  int64_t x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int64_t y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  if (lane == kWave - 1) s_wtot[wave] = x;
  __syncthreads();
  int64_t before = 0, all = 0;
  for (int i = 0; i < kBfsWaves; ++i) {
    const int64_t t = s_wtot[i];
    before += i < wave ? t : 0;
    all += t;
  }
  __syncthreads();  // s_wtot is reused by the next scan
  *tot = all;
  return before + x - v;
}

// row [a, b) of node, clamped to the edge array
__device__ inline void bfs_row(const int32_t* row_ptr, int num_edges, int node, int* a, int* b) {
  int lo = row_ptr[node], hi = row_ptr[node + 1];
  lo = lo < 0 ? 0 : (lo > num_edges ? num_edges : lo);
  hi = hi < lo ? lo : (hi > num_edges ? num_edges : hi);
  *a = lo;
  *b = hi;
}

// candidate k of the level: the level position q with off[q] <= k < off[q + 1] (binary search
// over off[0..L]), and its child
__device__ inline int bfs_candidate(const int32_t* row_ptr, const int32_t* col, int num_edges,
                                    const int32_t* level, const int32_t* off, int L, int k) {
  int lo = 0, hi = L - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (off[mid] <= k) lo = mid; else hi = mid - 1;
  }
  int a, b;
  bfs_row(row_ptr, num_edges, level[lo], &a, &b);
  return col[a + (k - off[lo])];
}

// One workgroup.  Workspace: queue [max_nodes], claim [max_nodes], off [max_nodes + 1].
__global__ __launch_bounds__(kBfsThreads) void bfs_subtree_kernel(
    const int32_t* row_ptr, const int32_t* col, int num_edges, int root, int max_nodes,
    uint8_t* in_subtree, int32_t* remap, int32_t* count_out, int32_t* queue, int32_t* claim,
    int32_t* off) {
  __shared__ int64_t s_wtot[kBfsWaves];
  const int tid = threadIdx.x;
  for (int i = tid; i < max_nodes; i += kBfsThreads) {
    in_subtree[i] = 0;
    remap[i] = -1;
    claim[i] = 0x7FFFFFFF;
  }
  __syncthreads();
  if (tid == 0) {
    in_subtree[root] = 1;
    remap[root] = 0;
    queue[0] = root;
  }
  __syncthreads();
  int start = 0, end = 1;  // the current level: queue[start, end)
  bool overflow = false;
  while (start < end) {
    const int L = end - start;
    const int32_t* level = queue + start;
    // offsets of the level's rows in its list of candidates (level order, then row order)
    int64_t run = 0;
    for (int c0 = 0; c0 < L; c0 += kBfsThreads) {
      const int q = c0 + tid;
      int64_t len = 0;
      if (q < L) {
        int a, b;
        bfs_row(row_ptr, num_edges, level[q], &a, &b);
        len = b - a;
      }
      int64_t tot;
      const int64_t ex = bfs_block_scan(len, s_wtot, &tot);
      if (q < L) off[q] = (int32_t)min(run + ex, (int64_t)0x7FFFFFFF);
      run += tot;
    }
    if (run > 0x7FFFFFFF) {  // more candidates than int32 keys (rows that overlap)
      overflow = true;
      break;
    }
    const int total = (int)run;
    if (tid == 0) off[L] = total;
    __syncthreads();
    // every candidate outside the subtree claims its child with its key (the earliest wins)
    for (int k = tid; k < total; k += kBfsThreads) {
      const int c = bfs_candidate(row_ptr, col, num_edges, level, off, L, k);
      if (c >= 0 && c < max_nodes && !in_subtree[c]) atomicMin(&claim[c], k);
    }
    __syncthreads();
    // the winners, numbered in key order
    int added = 0;
    for (int k0 = 0; k0 < total; k0 += kBfsThreads) {
      const int k = k0 + tid;
      int c = -1;
      bool win = false;
      if (k < total) {
        c = bfs_candidate(row_ptr, col, num_edges, level, off, L, k);
        win = c >= 0 && c < max_nodes && !in_subtree[c] && claim[c] == k;
      }
      int64_t tot;
      const int ex = (int)bfs_block_scan(win ? 1 : 0, s_wtot, &tot);
      if (win) {
        remap[c] = end + added + ex;
        queue[end + added + ex] = c;
      }
      added += (int)tot;
    }
    __syncthreads();
    for (int i = tid; i < added; i += kBfsThreads) in_subtree[queue[end + i]] = 1;
    __syncthreads();
    start = end;
    end += added;
  }
  if (tid == 0) count_out[0] = overflow ? -1 : end;
}

// Edge extraction: count per node and block scan (pass 1), scan of the block totals (pass 2),
// writes (pass 3).  Workspace: local [num_nodes], block totals [blocks + 1].
constexpr int kEdgeThreads = 1024;

__device__ inline int edges_kept(const int32_t* row_ptr, const int32_t* col, int num_edges,
                                 const uint8_t* in_subtree, int num_nodes, int node) {
  if (!in_subtree[node]) return 0;
  int a, b;
  bfs_row(row_ptr, num_edges, node, &a, &b);
  int n = 0;
  for (int e = a; e < b; ++e) {
    const int c = col[e];
    n += (c >= 0 && c < num_nodes && in_subtree[c]) ? 1 : 0;
  }
  return n;
}

__global__ __launch_bounds__(kEdgeThreads) void edges_count_kernel(
    const int32_t* row_ptr, const int32_t* col, int num_edges, const uint8_t* in_subtree,
    int num_nodes, int32_t* local, int32_t* block_tot) {
  __shared__ int64_t s_wtot[kEdgeThreads / kWave];
  const int i = blockIdx.x * kEdgeThreads + threadIdx.x;
  const int n = i < num_nodes ? edges_kept(row_ptr, col, num_edges, in_subtree, num_nodes, i) : 0;
  int64_t tot;
  const int64_t ex = bfs_block_scan(n, s_wtot, &tot);
  if (i < num_nodes) local[i] = (int32_t)ex;
  if (threadIdx.x == 0) block_tot[blockIdx.x] = (int32_t)tot;
}

__global__ __launch_bounds__(kEdgeThreads) void edges_scan_kernel(int32_t* block_tot, int blocks,
                                                                  int32_t* edge_count) {
  __shared__ int64_t s_wtot[kEdgeThreads / kWave];
  int64_t run = 0;
  for (int b0 = 0; b0 < blocks; b0 += kEdgeThreads) {
    const int b = b0 + (int)threadIdx.x;
    const int64_t v = b < blocks ? block_tot[b] : 0;
    int64_t tot;
    const int64_t ex = bfs_block_scan(v, s_wtot, &tot);
    __syncthreads();  // every block total of the chunk is read before any is overwritten
    if (b < blocks) block_tot[b] = (int32_t)(run + ex);
    run += tot;
  }
  if (threadIdx.x == 0) edge_count[0] = (int32_t)min(run, (int64_t)0x7FFFFFFF);
}

__global__ __launch_bounds__(kEdgeThreads) void edges_write_kernel(
    const int32_t* row_ptr, const int32_t* col, const int16_t* actions, int num_edges,
    const uint8_t* in_subtree, const int32_t* remap, int num_nodes, int max_edges,
    const int32_t* local, const int32_t* block_off, int32_t* out_parent, int32_t* out_child,
    int16_t* out_action) {
  const int i = blockIdx.x * kEdgeThreads + threadIdx.x;
  if (i >= num_nodes || !in_subtree[i]) return;
  int a, b;
  bfs_row(row_ptr, num_edges, i, &a, &b);
  int64_t pos = (int64_t)block_off[blockIdx.x] + local[i];
  const int np = remap[i];
  for (int e = a; e < b && pos < max_edges; ++e) {
    const int c = col[e];
    if (c < 0 || c >= num_nodes || !in_subtree[c]) continue;
    out_parent[pos] = np;
    out_child[pos] = remap[c];
    out_action[pos] = actions != nullptr ? actions[e] : (int16_t)0;
    ++pos;
  }
}

hipError_t launch_bfs_subtree(const int32_t* row_ptr, const int32_t* col, int num_edges,
                              int root, int max_nodes, uint8_t* in_subtree, int32_t* remap,
                              int32_t* count, int32_t* ws, hipStream_t st) {
  int32_t* queue = ws;
  int32_t* claim = ws + max_nodes;
  int32_t* off = ws + 2 * (int64_t)max_nodes;
  hipLaunchKernelGGL(bfs_subtree_kernel, dim3(1), dim3(kBfsThreads), 0, st, row_ptr, col,
                     num_edges, root, max_nodes, in_subtree, remap, count, queue, claim, off);
  return hipGetLastError();
}

int edges_blocks(int num_nodes) { return (num_nodes + kEdgeThreads - 1) / kEdgeThreads; }

hipError_t launch_extract_edges(const int32_t* row_ptr, const int32_t* col, const int16_t* actions,
                                int num_edges, const uint8_t* in_subtree, const int32_t* remap,
                                int num_nodes, int max_edges, int32_t* out_parent,
                                int32_t* out_child, int16_t* out_action, int32_t* edge_count,
                                int32_t* ws, hipStream_t st) {
  const int blocks = edges_blocks(num_nodes);
  int32_t* local = ws;
  int32_t* block_tot = ws + num_nodes;
  if (blocks == 0) {
    hipLaunchKernelGGL(edges_scan_kernel, dim3(1), dim3(kEdgeThreads), 0, st, block_tot, 0,
                       edge_count);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(edges_count_kernel, dim3(blocks), dim3(kEdgeThreads), 0, st, row_ptr, col,
                     num_edges, in_subtree, num_nodes, local, block_tot);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(edges_scan_kernel, dim3(1), dim3(kEdgeThreads), 0, st, block_tot, blocks,
                     edge_count);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(edges_write_kernel, dim3(blocks), dim3(kEdgeThreads), 0, st, row_ptr, col,
                     actions, num_edges, in_subtree, remap, num_nodes, max_edges, local,
                     block_tot, out_parent, out_child, out_action);
  return hipGetLastError();
}

}  // namespace omq
