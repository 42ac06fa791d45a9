// Leaf bookkeeping, synthetic evaluator and expansion (gfx950).
//
// Expansion follows the reference CPU driver (python/mcts/cpu/optimized_wave_search.py:367-438)
// and CythonLockFreeTree.expand_node (python/mcts/cpu/cython_tree_optimized.pyx:232-277):
// unique leaves in first-occurrence order; legal priors renormalised by their sum; Dirichlet
// mixing at the root; children bumped contiguously for nodes and edges; a leaf whose children
// do not fit is skipped (and later leaves may still fit).  The prior sum uses the canonical
// wave order (wave_sum_canonical) in place of numpy's pairwise order.
//
// Kernels per wave:
//   leaf_info_kernel    thread per unique leaf: hash key (fold over path actions), legal count
//                       (waves of more than OMQ_SELECT_RECORDS_MAX_WAVE; select forms them for
//                       smaller waves)
//   synth_eval_kernel   wave per unique leaf: synthetic priors/value (evaluator stand-in)
//   expand_plan_kernel  workgroup per tree: children counts, scan, capacity rule, row headers
//   expand_write_kernel wave per expanded leaf: priors, children N/W/P/parent/action/row
//   plan_values_kernel, write_backup_kernel: the plan and the writes side by side with the
//                       signed leaf values and the group backup (omq_expand_backup)
#include "backup_groups.h"
#include "omq_common.h"

namespace omq {

// wave-private LDS carve-up used by the per-leaf kernels
struct LeafLds {
  uint32_t* mask;  // legal_words: board legal mask
  uint32_t* bits;  // ceil(list_cap/32): chosen flags of progressive widening
  int* list;       // list_cap: legal actions, ascending
  double* val;     // list_cap: priors of the legal actions
};

__host__ __device__ inline int list_cap(const omq_forest& f) {
  return f.game == OMQ_GAME_SPARSE ? f.max_legal : f.num_actions;
}

__host__ __device__ inline size_t leaf_lds_per_wave(const omq_forest& f) {
  const size_t lc = (size_t)list_cap(f);
  size_t b = (size_t)f.legal_words * 4 + ((lc + 31) / 32) * 4 + lc * 4;
  b = (b + 7) & ~(size_t)7;
  return b + lc * 8;
}

// Board games with at most kStageMaxA actions: the expansion stages the leaf's policy row in
// LDS (loaded coalesced at the kernel's start), behind the wave's LeafLds region.
constexpr int kStageMaxA = 6 * kWave;

__host__ __device__ inline bool stage_policy(const omq_forest& f) {
  return f.game != OMQ_GAME_SPARSE && f.num_actions <= kStageMaxA;
}

__host__ __device__ inline size_t expand_lds_per_wave(const omq_forest& f) {
  return leaf_lds_per_wave(f) + (stage_policy(f) ? (size_t)f.num_actions * 4 : 0);
}

__device__ inline LeafLds carve(const omq_forest& f, unsigned char* base, int wave,
                                size_t stride) {
  const size_t lc = (size_t)list_cap(f);
  unsigned char* p = base + stride * wave;
  LeafLds l;
  l.mask = reinterpret_cast<uint32_t*>(p);
  l.bits = l.mask + f.legal_words;
  l.list = reinterpret_cast<int*>(l.bits + (lc + 31) / 32);
  size_t off = (size_t)f.legal_words * 4 + ((lc + 31) / 32) * 4 + lc * 4;
  off = (off + 7) & ~(size_t)7;
  l.val = reinterpret_cast<double*>(p + off);
  return l;
}

// ---------------------------------------------------------------------------------------
// One thread per unique leaf: its path is read once (the entries of its first simulation, then
// the action of each path node), the key is folded over the actions, and the legal count of a
// board leaf is the root's count less the path's moves (a pass stays legal).  Every legal list
// excludes the moves on its path, so those moves are distinct and legal at the root: the count
// equals that of the root mask with the path's cells cleared.  Consecutive threads write
// consecutive keys and counts.  The block also adds its leaves' path entries to the tree's
// OMQ_ST_ULEAFPATH counter (one atomic per block).
constexpr int kLeafInfoThreads = 256;

__global__ __launch_bounds__(kLeafInfoThreads) void leaf_info_kernel(omq_forest f, omq_wave w) {
  __shared__ int s_part[kLeafInfoThreads / kWave];
  int bx = blockIdx.x, by = blockIdx.y;
  xcd_block(&bx, &by);  // one contiguous run of blocks (leaves of few trees) per XCD
  const int t = by;
  const int u = bx * kLeafInfoThreads + threadIdx.x;
  const int64_t wb = (int64_t)t * w.max_wave;
  const int nu = w.ucount[t];
  int L = 0;
  if (u < nu) {
    uint64_t key;
    int count;
    const int rc = f.game != OMQ_GAME_SPARSE ? root_legal_count(f, t) : 0;
    L = leaf_key_count(f, w, t, w.ufirst[wb + u], rc, &key, &count);
    w.ukey[wb + u] = key;
    w.ulegal[wb + u] = count;
  }
  const int part = wave_sum_i(L);
  if (lane_id() == 0) s_part[threadIdx.x / kWave] = part;
  __syncthreads();
  if (threadIdx.x == 0) {
    int sum = 0;
    for (int i = 0; i < kLeafInfoThreads / kWave; ++i) sum += s_part[i];
    if (sum > 0)
      atomicAdd(reinterpret_cast<unsigned long long*>(&w.stats[(int64_t)t * OMQ_NSTATS +
                                                               OMQ_ST_ULEAFPATH]),
                (unsigned long long)sum);
  }
}

// ---------------------------------------------------------------------------------------
__global__ void synth_eval_kernel(omq_forest f, omq_wave w, float scale) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int t = blockIdx.y;
  const int wave = threadIdx.x / kWave;
  const int u = blockIdx.x * (blockDim.x / kWave) + wave;
  const int lane = lane_id();
  const int64_t wb = (int64_t)t * w.max_wave;
  if (u >= w.ucount[t]) return;
  LeafLds l = carve(f, smem, wave, leaf_lds_per_wave(f));
  const uint64_t key = w.ukey[wb + u];
  const int n = leaf_legal_list(f, w, t, u, l.mask, l.list);
  float* row = w.policy + (wb + u) * (int64_t)f.num_actions;
  // the scaled logits are kept in the wave's LDS (exactly, as doubles) for the second pass
  float mx = -__builtin_inff();
  for (int i = lane; i < n; i += kWave) {
    const float z = scale * key_normal(key, l.list[i]);
    l.val[i] = (double)z;
    mx = fmaxf(mx, z);
  }
  mx = wave_max_f32(mx);
  float part = 0.0f;
  for (int i = lane; i < n; i += kWave) {
    const float e = exp_cw((float)l.val[i] - mx);
    l.val[i] = (double)e;
    part = part + e;
  }
  const float S = wave_sum_canonical(part);
  for (int i = lane; i < n; i += kWave) row[l.list[i]] = (float)l.val[i] / S;
  if (lane == 0) w.values[wb + u] = key_value(key);
}

// ---------------------------------------------------------------------------------------
// progressive widening of the reference CPU driver (optimized_wave_search.py:394-415 and
// MAX_CHILDREN of cython_tree_optimized.pyx:31,239):
//   root:     mc = max(5, min(min(L, int(10*sqrt(N0)) + 1), 15)); the chosen set is the top-mc
//             (if L > mc, renormalised) or all L; the first min(8, |chosen|) become children
//   non-root: the top-3 (if L > 3, renormalised) or all L
__device__ inline int pw_root_mc(int L, int N0) {
  const int m1 = min(L, (int)(10.0 * sqrt((double)N0)) + 1);
  return max(5, min(m1, 15));
}

struct ExpCfg {
  int W;
  int vli;
  int policy;   // OMQ_EXPAND_*
  const double* noise;
  double eps;
};

constexpr int kPlanThreads = 1024;

// The plan of tree t, by a workgroup of kPlanThreads threads; want is its LDS array of
// max_wave ints.
__device__ inline void expand_plan_block(const omq_forest& f, const omq_wave& w, const ExpCfg& c,
                                         int t, int* want) {
  __shared__ int s_wtot[kPlanThreads / kWave];
  __shared__ int s_total;
  __shared__ unsigned long long s_exp, s_new, s_fail;
  const int tid = threadIdx.x;
  const int64_t tb = (int64_t)t * f.capacity;
  const int64_t wb = (int64_t)t * w.max_wave;
  const int U = w.ucount[t];
  if (tid == 0) {
    s_exp = 0;
    s_new = 0;
    s_fail = 0;
  }
  // four leaves per thread at a time, so that their two dependent loads (the leaf, then its
  // row length) are in flight together
  constexpr int kPlanBatch = 4;
  for (int u0 = tid; u0 < U; u0 += kPlanBatch * kPlanThreads) {
    int leafv[kPlanBatch], Lv[kPlanBatch], nchv[kPlanBatch];
#pragma unroll
    for (int j = 0; j < kPlanBatch; ++j) {
      const int u = u0 + j * kPlanThreads;
      leafv[j] = u < U ? w.uleaf[wb + u] : 0;
      Lv[j] = u < U ? w.ulegal[wb + u] : 0;
    }
#pragma unroll
    for (int j = 0; j < kPlanBatch; ++j) {
      const int u = u0 + j * kPlanThreads;
      nchv[j] = u < U ? f.num_children[tb + leafv[j]] : 1;
    }
#pragma unroll
    for (int j = 0; j < kPlanBatch; ++j) {
      const int u = u0 + j * kPlanThreads;
      if (u >= U) break;
      const int leaf = leafv[j];
      const int L = Lv[j];
      int k = 0;
      if (nchv[j] == 0 && L > 0) {
        if (c.policy == OMQ_EXPAND_FULL) {
          k = L;
        } else if (leaf == 0) {
          const int N0 = f.visit_counts[tb] - c.vli * c.W;
          const int mc = pw_root_mc(L, N0);
          k = min(L > mc ? mc : L, 8);
        } else {
          k = min(L, 3);
        }
      }
      if (k > OMQ_MAX_ROW) {  // a selection row must fit the register tile
        atomicOr(&w.status[0], OMQ_STATUS_ROWLIMIT);
        k = 0;
      }
      want[u] = k;
    }
  }
  __syncthreads();
  // exclusive scan over contiguous chunks
  const int per = (U + kPlanThreads - 1) / kPlanThreads;
  const int lo = tid * per, hi = min(lo + per, U);
  int sum = 0;
  for (int i = lo; i < hi; ++i) sum += want[i];
  int wt;
  const int wex = wave_excl_scan(sum, &wt);
  if (lane_id() == 0) s_wtot[tid / kWave] = wt;
  __syncthreads();
  int wbase = 0, total = 0;
  for (int i = 0; i < kPlanThreads / kWave; ++i) {
    if (i < tid / kWave) wbase += s_wtot[i];
    total += s_wtot[i];
  }
  const int base = f.num_nodes[t];
  const bool all_fit = (int64_t)base + total <= (int64_t)f.capacity;
  // excl offsets into a second pass; want[] keeps k, offsets go to uedge directly
  int run = wbase + wex;
  if (all_fit) {
    int n_exp = 0;  // (the thread's leaves expanded; their children are its chunk's sum)
    for (int i = lo; i < hi; ++i) {
      const int k = want[i];
      w.uedge[wb + i] = k > 0 ? base + run - 1 : -1;
      w.unew[wb + i] = k;
      if (k > 0) {
        const int leaf = w.uleaf[wb + i];
        f.first_child[tb + leaf] = base + run - 1;
        f.num_children[tb + leaf] = k;
        ++n_exp;
      }
      run += k;
    }
    // one atomic per wave (the per-leaf atomics on one address serialized)
    const int we = wave_sum_i(n_exp);
    if (lane_id() == 0 && we > 0) {
      atomicAdd(&s_exp, (unsigned long long)we);
      atomicAdd(&s_new, (unsigned long long)wt);
    }
    if (tid == 0) s_total = total;
  } else if (tid < kWave) {
    // Capacity boundary: first-fit in leaf order (expand_node refuses a leaf whose children do
    // not fit; later, smaller leaves may still fit), decided by one wave, 64 leaves at a time.
    // Leaf i fits when cur_i + k_i <= capacity, cur_i = base + the children of the leaves
    // before it that fit.  Within a chunk each round first drops the leaves that cannot fit
    // even now (cur only grows, so they never will), then lets every remaining leaf fit up to
    // the first one whose running sum overflows; that one is dropped by the next round.  Each
    // round settles at least one leaf.
    const int lane = tid;
    const int64_t cap = f.capacity;
    int64_t cur = base;
    unsigned long long n_exp = 0, n_new = 0, n_fail = 0;
    for (int c0 = 0; c0 < U; c0 += kWave) {
      const int i = c0 + lane;
      const int k = i < U ? want[i] : 0;
      bool pend = k > 0;
      bool fits = false;
      int64_t at = -1;  // node id of the first child, when the leaf fits
      for (int round = 0; round <= kWave && __ballot(pend) != 0; ++round) {
        pend = pend && !(cur + k > cap);
        int tot;
        const int ex = wave_excl_scan(pend ? k : 0, &tot);
        const uint64_t over = __ballot(pend && cur + ex + k > cap);
        const int f0 = over != 0 ? lowest_lane(over) : kWave;
        if (pend && lane < f0) {
          fits = true;
          at = cur + ex;
          pend = false;
        }
        // the children of the leaves that fit this round: those before f0 (all when f0 = 64)
        cur += f0 < kWave ? readlane_i(ex, f0) : tot;
      }
      if (i < U) {
        if (fits) {
          w.uedge[wb + i] = (int)at - 1;
          w.unew[wb + i] = k;
          const int leaf = w.uleaf[wb + i];
          f.first_child[tb + leaf] = (int)at - 1;
          f.num_children[tb + leaf] = k;
        } else {
          w.uedge[wb + i] = -1;
          w.unew[wb + i] = 0;
        }
      }
      n_exp += __popcll(__ballot(fits));
      n_new += (unsigned long long)wave_sum_i(fits ? k : 0);
      n_fail += __popcll(__ballot(k > 0 && !fits));
    }
    if (lane == 0) {
      s_exp = n_exp;
      s_new = n_new;
      s_fail = n_fail;
      s_total = (int)(cur - base);
    }
  }
  __syncthreads();
  if (tid == 0) {
    f.num_nodes[t] = base + s_total;
    int64_t* st = w.stats + (int64_t)t * OMQ_NSTATS;
    atomicAdd(reinterpret_cast<unsigned long long*>(&st[OMQ_ST_EXPANDED]), s_exp);
    atomicAdd(reinterpret_cast<unsigned long long*>(&st[OMQ_ST_NEWCHILD]), s_new);
    atomicAdd(reinterpret_cast<unsigned long long*>(&st[OMQ_ST_CAPFAIL]), s_fail);
  }
}

// four int32 as a vector of the compiler's own (what __builtin_nontemporal_store takes)
typedef int IntX4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kPlanThreads) void expand_plan_kernel(omq_forest f, omq_wave w,
                                                                   ExpCfg c) {
  extern __shared__ __align__(16) int want[];  // [max_wave] (ucount <= max_wave)
  expand_plan_block(f, w, c, (int)blockIdx.x, want);
}

// ---------------------------------------------------------------------------------------
// Block bx of tree t's expansion writes (one wave per expanded leaf), with the block's
// dynamic LDS smem.
__device__ inline void expand_write_block(const omq_forest& f, const omq_wave& w,
                                          const ExpCfg& c, int bx, int t, unsigned char* smem) {
  const int wave = threadIdx.x / kWave;
  const int u = bx * (blockDim.x / kWave) + wave;
  const int lane = lane_id();
  const int64_t tb = (int64_t)t * f.capacity;
  const int64_t wb = (int64_t)t * w.max_wave;
  if (u >= c.W) return;
  // The leaf's records, and (staged boards) its policy row, are loaded together before the
  // checks below, so that their latencies overlap.  (For a slot past the wave's unique leaves
  // they are stale and unused.)
  const int ucnt = w.ucount[t];
  const int k = w.unew[wb + u];
  const int leaf = w.uleaf[wb + u];
  const int cbase = w.uedge[wb + u] + 1;  // node id of the first child
  const int s0 = w.ufirst[wb + u];
  const uint64_t ukey = f.game == OMQ_GAME_SPARSE ? w.ukey[wb + u] : 0ull;
  const float* pol = w.policy + (wb + u) * (int64_t)f.num_actions;
  const bool staged = stage_policy(f);
  float prow[kStageMaxA / kWave];
#pragma unroll
  for (int j = 0; j < kStageMaxA / kWave; ++j) {
    const int a = j * kWave + lane;
    prow[j] = (staged && a < f.num_actions) ? pol[a] : 0.0f;
  }
  if (u >= ucnt || k <= 0) return;
  LeafLds l = carve(f, smem, wave, expand_lds_per_wave(f));
  float* spol = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(l.mask) +
                                         leaf_lds_per_wave(f));
  if (staged) {
#pragma unroll
    for (int j = 0; j < kStageMaxA / kWave; ++j) {
      const int a = j * kWave + lane;
      if (a < f.num_actions) spol[a] = prow[j];
    }
  }
  int n;
  if (f.game == OMQ_GAME_SPARSE) {
    n = sparse_legal_list(f, ukey, l.list, l.mask);
  } else if (w.umask != nullptr) {
    leaf_umask(f, w, t, u, l.mask);  // (its barrier also orders spol)
    n = board_legal_list(f, l.mask, l.list);
  } else {
    int a_lo, a_hi;
    const int L = load_path_actions(f, w, t, s0, &a_lo, &a_hi);
    board_legal_mask(f, t, L, a_lo, a_hi, l.mask);  // (its barriers also order spol)
    n = board_legal_list(f, l.mask, l.list);
  }
  if (staged) pol = spol;

  // legal priors renormalised by their sum (optimized_wave_search.py:384-385)
  float part = 0.0f;
  for (int i = lane; i < n; i += kWave) part = part + pol[l.list[i]];
  const float S = wave_sum_canonical(part);
  // root Dirichlet mixing (optimized_wave_search.py:388-392): numpy keeps
  // (1-eps)*float32 in float32 and promotes the sum with the float64 noise to float64
  const bool noisy = (leaf == 0) && c.noise != nullptr && c.eps > 0.0;
  const float w32 = (float)(1.0 - c.eps);
  for (int i = lane; i < n; i += kWave) {
    const float p = pol[l.list[i]] / S;
    if (noisy)
      l.val[i] = (double)(w32 * p) + c.eps * c.noise[(int64_t)t * f.num_actions + i];
    else
      l.val[i] = (double)p;
  }
  wave_sync();

  int nch = n;
  if (c.policy == OMQ_EXPAND_REFERENCE_PW) {
    const int sel = (leaf == 0) ? pw_root_mc(n, f.visit_counts[tb] - c.vli * c.W) : 3;
    if (n > sel) {
      // top-sel by (prior desc, action asc), kept in ascending action order, renormalised
      const int nwords = (n + 31) / 32;
      for (int i = lane; i < nwords; i += kWave) l.bits[i] = 0u;
      wave_sync();
      for (int it = 0; it < sel; ++it) {
        double bv = -__builtin_inf();
        int bi = 0x7FFFFFFF;
        for (int i = lane; i < n; i += kWave) {
          const bool taken = (l.bits[i >> 5] >> (i & 31)) & 1u;
          if (!taken && (l.val[i] > bv || (l.val[i] == bv && i < bi))) {
            bv = l.val[i];
            bi = i;
          }
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
          const double ov = __shfl_xor(bv, off, 64);
          const int oi = __shfl_xor(bi, off, 64);
          if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
          }
        }
        if (lane == 0 && bi < n) l.bits[bi >> 5] |= 1u << (bi & 31);
        wave_sync();
      }
      // the chosen entries compacted in order, 64 at a time: a chunk's entries are read before
      // any is written, and its writes land below the next chunk's entries (j <= i)
      int j0 = 0;
      for (int c0 = 0; c0 < n; c0 += kWave) {
        const int i = c0 + lane;
        const bool keep = i < n && ((l.bits[i >> 5] >> (i & 31)) & 1u);
        const double v = keep ? l.val[i] : 0.0;
        const int a = keep ? l.list[i] : 0;
        const uint64_t b = __ballot(keep);
        wave_sync();
        if (keep) {
          const int j = j0 + (int)__builtin_amdgcn_mbcnt_hi(
                                 (uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
          l.val[j] = v;
          l.list[j] = a;
        }
        j0 += __popcll(b);
        wave_sync();
      }
      nch = sel;
      if (noisy) {
        double dpart = 0.0;
        for (int j = lane; j < nch; j += kWave) dpart = dpart + l.val[j];
        const double Sd = wave_sum_canonical_d(dpart);
        wave_sync();
        for (int j = lane; j < nch; j += kWave) l.val[j] = l.val[j] / Sd;
      } else {
        float fpart = 0.0f;
        for (int j = lane; j < nch; j += kWave) fpart = fpart + (float)l.val[j];
        const float Sf = wave_sum_canonical(fpart);
        wave_sync();
        for (int j = lane; j < nch; j += kWave) l.val[j] = (double)((float)l.val[j] / Sf);
      }
      wave_sync();
    }
  }
  if (k > nch) {
    if (lane == 0) atomicOr(&w.status[0], OMQ_STATUS_ROWLIMIT);
    return;
  }
  // children: the first k chosen actions, ascending.  Rows of at least 4 * 64 children are
  // written 16 bytes per lane (four children) from the first node index that is a multiple of
  // 4, the children before it and after the last whole quad one per lane; shorter rows one per
  // lane (C3 expand_write 48.8 -> 47.6 us; quads on rows of 20-45 children, C4, cost 7 %).
  // The quads of parents and actions, which no kernel of the next waves reads (only subtree
  // reuse and the leaves' records, along paths), are stored non-temporally, so that they take
  // no L2 lines from the rows and counts that selection and backup read (C3 101.1 -> 102.2 M
  // sims/s).  The other five arrays stored so cost the expansion more than they saved
  // elsewhere, and so did the one-per-lane stores of the head, the tail and short rows (C2's
  // expansion 28.4 -> 32.5 us).
  const int64_t node0 = tb + cbase;
  auto put1 = [&](int j) {
    const int64_t node = node0 + j;
    f.visit_counts[node] = 0;
    f.value_sums[node] = 0.0f;
    f.priors[node] = (float)l.val[j];
    f.parents[node] = leaf;
    f.actions[node] = l.list[j];
    f.first_child[node] = -1;
    f.num_children[node] = 0;
  };
  if (k < 4 * kWave) {
    for (int j = lane; j < k; j += kWave) put1(j);
    return;
  }
  const int hd = (int)((4 - (node0 & 3)) & 3);  // (< 4 <= k)
  if (lane < hd) put1(lane);
  const int nq = (k - hd) >> 2;
  for (int q = lane; q < nq; q += kWave) {
    const int j = hd + 4 * q;
    const int64_t node = node0 + j;
    const float4 pr = make_float4((float)l.val[j], (float)l.val[j + 1], (float)l.val[j + 2],
                                  (float)l.val[j + 3]);
    const int4 ac = make_int4(l.list[j], l.list[j + 1], l.list[j + 2], l.list[j + 3]);
    *reinterpret_cast<int4*>(f.visit_counts + node) = make_int4(0, 0, 0, 0);
    *reinterpret_cast<float4*>(f.value_sums + node) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    *reinterpret_cast<float4*>(f.priors + node) = pr;
    __builtin_nontemporal_store((IntX4){leaf, leaf, leaf, leaf},
                                reinterpret_cast<IntX4*>(f.parents + node));
    __builtin_nontemporal_store((IntX4){ac.x, ac.y, ac.z, ac.w},
                                reinterpret_cast<IntX4*>(f.actions + node));
    *reinterpret_cast<int4*>(f.first_child + node) = make_int4(-1, -1, -1, -1);
    *reinterpret_cast<int4*>(f.num_children + node) = make_int4(0, 0, 0, 0);
  }
  const int tl = hd + 4 * nq;
  if (lane < k - tl) put1(tl + lane);
}

__global__ void expand_write_kernel(omq_forest f, omq_wave w, ExpCfg c) {
  extern __shared__ __align__(16) unsigned char smem[];
  int bx = blockIdx.x, by = blockIdx.y;
  xcd_block(&bx, &by);  // one contiguous run of blocks (leaves of few trees) per XCD
  expand_write_block(f, w, c, bx, by, smem);
}

// ---------------------------------------------------------------------------------------
// A wave's expansion and group backup in two launches instead of four.  The expansion writes
// the expanded leaves' row headers and their new children, the backup N and W of the path
// nodes: no address is written by both, and neither reads what the other writes (the new
// children lie past every path node, and the backup reads no row header).  Under the
// reference_pw rule the expansion reads the root's count, which the backup changes; there the
// two run one after the other (omq_expand_backup).  So the plan runs beside the signed leaf
// values, and the child writes beside the group backup.

// Plan of tree blockIdx.y (block 0 of each tree), beside the signed leaf values of its
// simulations (blocks 1 on, kPlanThreads simulations each).
__global__ __launch_bounds__(kPlanThreads) void plan_values_kernel(omq_forest f, omq_wave w,
                                                                   ExpCfg c, int sign_mode) {
  extern __shared__ __align__(16) int want[];  // [max_wave] (ucount <= max_wave)
  const int t = blockIdx.y;
  if (blockIdx.x == 0) {
    expand_plan_block(f, w, c, t, want);
    return;
  }
  const int s = ((int)blockIdx.x - 1) * kPlanThreads + (int)threadIdx.x;
  if (s < c.W) sim_value_at(f, w, t, s, sign_mode);
}

// Blocks [0, nbb) of a tree: backup_groups_block; the rest: expand_write_block (kBackupThreads
// / 64 leaves each), nbe of them.  The backup's blocks come first, so that their dependent
// loads start with the first writes instead of after the last (C3's expansion-and-backup phase
// 68.2 -> 63.1 us, C4's 68.0 -> 61.5 us, C2's 33.6 -> 31.6 us against the writes first).
template <bool FUSED>
__global__ __launch_bounds__(kBackupThreads) void write_backup_kernel(omq_forest f, omq_wave w,
                                                                      ExpCfg c, int sign_mode,
                                                                      int nbe, int nbb) {
  extern __shared__ __align__(16) unsigned char smem[];
  int bx = blockIdx.x, by = blockIdx.y;
  xcd_block(&bx, &by);  // one contiguous run of blocks (leaves of few trees) per XCD
  if (bx < nbb)
    backup_groups_block<FUSED>(f, w, c.vli, sign_mode, bx, by, nbb);
  else
    expand_write_block(f, w, c, bx - nbb, by, smem);
}

// ---------------------------------------------------------------------------------------
size_t leaf_lds_per_wave_host(const omq_forest& f) { return leaf_lds_per_wave(f); }

static int leaf_waves_per_block(const omq_forest& f) {
  const size_t per = leaf_lds_per_wave_host(f);
  int wpb = 4;
  while (wpb > 1 && per * wpb > 64 * 1024) wpb >>= 1;
  return wpb;
}

hipError_t launch_leaf_info(const omq_forest& f, const omq_wave& w, int W, hipStream_t st) {
  dim3 grid((W + kLeafInfoThreads - 1) / kLeafInfoThreads, f.num_trees);
  hipLaunchKernelGGL(leaf_info_kernel, grid, dim3(kLeafInfoThreads), 0, st, f, w);
  return hipGetLastError();
}

hipError_t launch_synth_eval(const omq_forest& f, const omq_wave& w, int W, float scale,
                             hipStream_t st) {
  const int wpb = leaf_waves_per_block(f);
  const size_t lds = leaf_lds_per_wave_host(f) * wpb;
  dim3 grid((W + wpb - 1) / wpb, f.num_trees);
  hipLaunchKernelGGL(synth_eval_kernel, grid, dim3(wpb * kWave), lds, st, f, w, scale);
  return hipGetLastError();
}

hipError_t launch_expand(const omq_forest& f, const omq_wave& w, int W, float virtual_loss,
                         int policy, const double* noise, double eps, hipStream_t st) {
  ExpCfg c;
  c.W = W;
  c.vli = (int)virtual_loss;
  c.policy = policy;
  c.noise = noise;
  c.eps = eps;
  hipLaunchKernelGGL(expand_plan_kernel, dim3(f.num_trees), dim3(kPlanThreads),
                     (size_t)w.max_wave * sizeof(int), st, f, w, c);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t per = expand_lds_per_wave(f);
  int wpb = 4;
  while (wpb > 1 && per * wpb > 64 * 1024) wpb >>= 1;
  dim3 grid((W + wpb - 1) / wpb, f.num_trees);
  hipLaunchKernelGGL(expand_write_kernel, grid, dim3(wpb * kWave), per * wpb, st, f, w, c);
  return hipGetLastError();
}

bool expand_backup_fusable(const omq_forest& f, int policy, int w_mode) {
  return policy == OMQ_EXPAND_FULL && w_mode == OMQ_WACC_ORDERED &&
         expand_lds_per_wave(f) * (kBackupThreads / kWave) <= 64 * 1024;
}

hipError_t launch_expand_backup(const omq_forest& f, const omq_wave& w, int W,
                                float virtual_loss, const double* noise, double eps,
                                int sign_mode, hipStream_t st) {
  ExpCfg c;
  c.W = W;
  c.vli = (int)virtual_loss;
  c.policy = OMQ_EXPAND_FULL;
  c.noise = noise;
  c.eps = eps;
  // the signed leaf values: formed by the group backup itself for the waves it fuses them in
  const bool fused_values = W <= kFuseMaxWave;
  const int nvb = fused_values ? 0 : (W + kPlanThreads - 1) / kPlanThreads;
  hipLaunchKernelGGL(plan_values_kernel, dim3(1 + nvb, f.num_trees), dim3(kPlanThreads),
                     (size_t)w.max_wave * sizeof(int), st, f, w, c, sign_mode);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  constexpr int wpb = kBackupThreads / kWave;
  const size_t lds = expand_lds_per_wave(f) * wpb;
  const int nbe = (W + wpb - 1) / wpb;
  const int nbb = backup_group_blocks(W);
  const dim3 grid(nbe + nbb, f.num_trees);
  if (fused_values)
    hipLaunchKernelGGL(write_backup_kernel<true>, grid, dim3(kBackupThreads), lds, st, f, w, c,
                       sign_mode, nbe, nbb);
  else
    hipLaunchKernelGGL(write_backup_kernel<false>, grid, dim3(kBackupThreads), lds, st, f, w, c,
                       sign_mode, nbe, nbb);
  return hipGetLastError();
}

}  // namespace omq
