// Wave selection with virtual loss (gfx950).
//
// Sequential definition (python/mcts/cpu/cython_tree_optimized.pyx:177-202 select_path and
// :421-464 select_best_child_nogil): simulations s = 0..W-1 descend one after another; on
// arrival at a node its visit count grows by VL = (int)virtual_loss; at an expanded node the
// child with the first N==0 wins, otherwise the argmax of
//     W/((float)N + VLf) + ((c*P)*sqrt((float)Np)) / (float)(1+N)
// with strict '>' (lowest index on ties) and -1e9 as the initial best.
//
// Parallel schedule, same result: the simulations that are at the same node p at depth d
// form a group.  A decision at p reads only N of p and of p's children; during a wave those
// change only through simulations that pass through p, and all of them are in p's group.  So
// the group is processed as a chain in simulation order, the r-th member (1-based) seeing
// Np = N[p] + VL*r and each child c with N[c] + VL*(members before it that chose c).  Groups
// are independent of each other.  A workgroup per tree takes the groups level by level, one
// wavefront per group; the chain keeps the row (N, W, c*P, Q) in registers, lane l holding
// children [l*R, l*R+R), so the winning lane order is the index order.  The members of a
// group are kept in simulation order in LDS and partitioned among the chosen children by a
// counting scatter, which yields the groups of the next level.
//
// Virtual loss is materialised once per group (N[p] += VL*m, p is owned by one group per
// wave), or with one atomic per path entry when vl_atomic is set.

#include "omq_common.h"

namespace omq {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / kWave;
constexpr uint32_t kNoChild = 0xFFFFFFFFu;

struct SelCfg {
  int W;          // simulations per tree in this wave
  float c_puct;
  float vlf;      // virtual loss as float
  int vli;        // (int)virtual loss
  int max_depth;  // forced leaf at depth max_depth-1
  int vl_atomic;
};

// Serial chain of row-argmaxes for one group (whole wave).  ch[r] receives, for the r-th
// member, (child index << 16) | rank among the members that chose the same child, or
// kNoChild.  Child counts are left in cnt_s[0..k).  Returns the first rank without a child
// (or -1).
template <int R>
__device__ int run_chain(const omq_forest& f, int64_t tb, int first, int k, int Np0, int m,
                         const SelCfg& c, uint32_t* ch, uint16_t* cnt_s) {
  const int lane = lane_id();
  int n[R], cnt[R];
  float wv[R], q[R], cp[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int i = lane * R + j;
    cnt[j] = 0;
    n[j] = 0;
    wv[j] = 0.0f;
    cp[j] = 0.0f;
    if (i < k) {
      const int64_t node = tb + first + 1 + i;  // child of edge first+i is node first+i+1
      n[j] = f.visit_counts[node];
      wv[j] = f.value_sums[node];
      cp[j] = c.c_puct * f.priors[node];
    }
    q[j] = wv[j] / ((float)n[j] + c.vlf);
  }
  int first_end = -1;
  for (int r = 0; r < m; ++r) {
    const int Np = Np0 + c.vli * (r + 1);
    int win = -1;
    if (Np != 0) {
      const float s = sqrtf((float)Np);
      int uv = -1, bi = -1;
      float bs = 0.0f;
#pragma unroll
      for (int j = 0; j < R; ++j) {
        const int i = lane * R + j;
        if (i < k) {
          if (n[j] == 0) {
            if (uv < 0) uv = i;
          } else {
            float sc = q[j] + (cp[j] * s) / (float)(1 + n[j]);
            sc = sc + 0.0f;  // -0 -> +0, so that equal scores compare equal below
            if (sc > -1e9f && (bi < 0 || sc > bs)) {
              bs = sc;
              bi = i;
            }
          }
        }
      }
      const uint64_t um = __ballot(uv >= 0);
      if (um) {
        win = readlane_i(uv, lowest_lane(um));
      } else {
        const float mx = wave_max_f32(bi >= 0 ? bs : -__builtin_inff());
        const uint64_t bm = __ballot(bi >= 0 && bs == mx);
        if (bm) win = readlane_i(bi, lowest_lane(bm));
      }
    }
    if (win >= 0) {
      const int owner = win / R;
      const int jj = win - owner * R;
      if (lane == owner) {
#pragma unroll
        for (int j = 0; j < R; ++j) {
          if (j == jj) {
            ch[r] = ((uint32_t)win << 16) | (uint32_t)cnt[j];
            cnt[j] += 1;
            n[j] += c.vli;
            q[j] = wv[j] / ((float)n[j] + c.vlf);
          }
        }
      }
    } else {
      if (lane == 0) ch[r] = kNoChild;
      if (first_end < 0) first_end = r;
    }
  }
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int i = lane * R + j;
    if (i < k) cnt_s[i] = (uint16_t)cnt[j];
  }
  wave_sync();
  return first_end;
}

__device__ inline int dispatch_chain(const omq_forest& f, int64_t tb, int first, int k, int Np0,
                                     int m, const SelCfg& c, uint32_t* ch, uint16_t* cnt_s) {
  if (k <= 64) return run_chain<1>(f, tb, first, k, Np0, m, c, ch, cnt_s);
  if (k <= 128) return run_chain<2>(f, tb, first, k, Np0, m, c, ch, cnt_s);
  if (k <= 256) return run_chain<4>(f, tb, first, k, Np0, m, c, ch, cnt_s);
  return run_chain<8>(f, tb, first, k, Np0, m, c, ch, cnt_s);  // k <= OMQ_MAX_ROW = 512
}

// Block-wide exclusive scan of a[0..n) in place (n <= 4 * kSelThreads); returns the total.
__device__ int block_excl_scan(int32_t* a, int n, int* s_wtot) {
  const int tid = threadIdx.x;
  const int per = (n + kSelThreads - 1) / kSelThreads;
  const int lo = tid * per;
  const int hi = min(lo + per, n);
  int sum = 0;
  for (int i = lo; i < hi; ++i) sum += a[i];
  int wtotal;
  const int wex = wave_excl_scan(sum, &wtotal);
  const int wave = tid / kWave;
  if (lane_id() == 0) s_wtot[wave] = wtotal;
  __syncthreads();
  int wbase = 0, total = 0;
  for (int i = 0; i < kSelWaves; ++i) {
    const int v = s_wtot[i];
    if (i < wave) wbase += v;
    total += v;
  }
  int run = wbase + wex;
  for (int i = lo; i < hi; ++i) {
    const int v = a[i];
    a[i] = run;
    run += v;
  }
  __syncthreads();
  return total;
}

__global__ __launch_bounds__(kSelThreads) void select_kernel(omq_forest f, omq_wave w,
                                                             SelCfg c) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int W = c.W;
  uint32_t* choice = reinterpret_cast<uint32_t*>(smem);       // [W]
  int32_t* lflag = reinterpret_cast<int32_t*>(choice + W);    // [W] leaf-first flags, then scan
  uint32_t* gnode = reinterpret_cast<uint32_t*>(lflag + W);   // [2W] group node per level
  uint32_t* gsl = gnode + 2 * W;                              // [2W] seg | len << 16
  uint16_t* buf = reinterpret_cast<uint16_t*>(gsl + 2 * W);   // [2W] members by position
  uint16_t* lfs = buf + 2 * W;                                // [W] first sim of own leaf group
  uint16_t* cnt_all = lfs + W;                                // [kSelWaves * OMQ_MAX_ROW]

  __shared__ int s_gcount[2];
  __shared__ int s_glog;
  __shared__ int s_wtot[kSelWaves];
  __shared__ unsigned long long s_st[OMQ_NSTATS];

  const int t = blockIdx.x;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = lane_id();
  const int64_t tb = (int64_t)t * f.capacity;
  const int MW = w.max_wave, MD = w.max_depth;
  const int64_t gmax = (int64_t)MW * MD;
  int32_t* N = f.visit_counts;
  uint16_t* cnt_s = cnt_all + wave * OMQ_MAX_ROW;

  for (int s = tid; s < W; s += kSelThreads) {
    buf[s] = (uint16_t)s;
    lflag[s] = 0;
  }
  if (tid < OMQ_NSTATS) s_st[tid] = 0;
  if (tid == 0) {
    gnode[0] = 0;
    gsl[0] = 0u | ((uint32_t)W << 16);
    s_gcount[0] = 1;
    s_gcount[1] = 0;
    s_glog = 0;
  }
  __syncthreads();

  for (int d = 0; d < c.max_depth; ++d) {
    const int cur = d & 1, nxt = cur ^ 1;
    const int ng = s_gcount[cur];
    if (ng == 0) break;
    for (int gi = wave; gi < ng; gi += kSelWaves) {
      const int p = (int)gnode[cur * W + gi];
      const uint32_t sl = gsl[cur * W + gi];
      const int seg = (int)(sl & 0xFFFFu);
      const int m = (int)(sl >> 16);
      const uint16_t* mem = buf + cur * W + seg;

      // log the group and record the path entries
      int gid = 0;
      if (lane == 0) gid = atomicAdd(&s_glog, 1);
      gid = readlane_i(gid, 0);
      if (lane < 4) {
        const int v = lane == 0 ? p : lane == 1 ? d : lane == 2 ? seg : m;
        w.glog[((int64_t)t * gmax + gid) * 4 + lane] = v;
      }
      for (int r = lane; r < m; r += kWave) {
        const int s = mem[r];
        w.paths[((int64_t)t * MW + s) * MD + d] = p;
        w.gmembers[((int64_t)t * MD + d) * MW + seg + r] = (uint16_t)s;
      }

      const int Np0 = N[tb + p];
      const int k = f.num_children[tb + p];
      const int first = f.first_child[tb + p];
      if (c.vl_atomic) {
        for (int r = lane; r < m; r += kWave) atomicAdd(&N[tb + p], c.vli);
      } else if (lane == 0) {
        N[tb + p] = Np0 + c.vli * m;
      }
      if (lane == 0) atomicAdd(&s_st[OMQ_ST_PATHNODES], 1ull);

      bool leaf = (k <= 0) || (first < 0) || (d == c.max_depth - 1);
      if (!leaf && k > OMQ_MAX_ROW) {
        if (lane == 0) atomicOr(&w.status[0], OMQ_STATUS_ROWLIMIT);
        leaf = true;
      }
      if (leaf) {
        const int s0 = mem[0];
        for (int r = lane; r < m; r += kWave) {
          const int s = mem[r];
          w.path_len[(int64_t)t * MW + s] = d + 1;
          w.leaves[(int64_t)t * MW + s] = p;
          lfs[s] = (uint16_t)s0;
        }
        if (lane == 0) {
          lflag[s0] = 1;
          atomicAdd(&s_st[OMQ_ST_PATHENTRIES], (unsigned long long)m * (d + 1));
        }
        continue;
      }

      uint32_t* ch = choice + seg;
      const int fe = dispatch_chain(f, tb, first, k, Np0, m, c, ch, cnt_s);
      if (lane == 0) {
        atomicAdd(&s_st[OMQ_ST_INTERNAL], 1ull);
        atomicAdd(&s_st[OMQ_ST_ROWSUM], (unsigned long long)k);
        atomicAdd(&s_st[OMQ_ST_STEPS], (unsigned long long)m);
      }

      // exclusive scan of the child counts (blocks of B children per lane) -> offsets, and
      // the groups of the next level
      const int B = (k + kWave - 1) / kWave;
      const int lo = lane * B, hi = min(lo + B, k);
      int sum = 0, nz = 0;
      for (int i = lo; i < hi; ++i) {
        const int v = cnt_s[i];
        sum += v;
        nz += v > 0;
      }
      int tot_sum, tot_nz;
      int run = wave_excl_scan(sum, &tot_sum);
      int gpos = wave_excl_scan(nz, &tot_nz);
      int gbase = 0;
      if (lane == 0 && tot_nz > 0) gbase = atomicAdd(&s_gcount[nxt], tot_nz);
      gbase = readlane_i(gbase, 0);
      for (int i = lo; i < hi; ++i) {
        const int v = cnt_s[i];
        if (v > 0) {
          const int g = gbase + gpos++;
          gnode[nxt * W + g] = (uint32_t)(first + 1 + i);
          gsl[nxt * W + g] = (uint32_t)(seg + run) | ((uint32_t)v << 16);
        }
        cnt_s[i] = (uint16_t)run;
        run += v;
      }
      wave_sync();

      // scatter the members to their child's segment (rank keeps simulation order)
      const int s_end = fe >= 0 ? (int)mem[fe] : -1;
      for (int r = lane; r < m; r += kWave) {
        const int s = mem[r];
        const uint32_t cv = ch[r];
        if (cv == kNoChild) {
          w.path_len[(int64_t)t * MW + s] = d + 1;
          w.leaves[(int64_t)t * MW + s] = p;
          lfs[s] = (uint16_t)s_end;
          atomicAdd(&s_st[OMQ_ST_PATHENTRIES], (unsigned long long)(d + 1));
        } else {
          const int i = (int)(cv >> 16);
          const int rk = (int)(cv & 0xFFFFu);
          buf[nxt * W + seg + cnt_s[i] + rk] = (uint16_t)s;
        }
      }
      if (fe >= 0 && lane == 0) {
        lflag[s_end] = 1;
        atomicOr(&w.status[0], OMQ_STATUS_NOCHILD);
      }
      wave_sync();
    }
    __syncthreads();
    if (tid == 0) s_gcount[cur] = 0;
    __syncthreads();
  }

  // unique leaves in order of first occurrence
  const int nu = block_excl_scan(lflag, W, s_wtot);
  for (int s = tid; s < W; s += kSelThreads) {
    const int s0 = lfs[s];
    const int uid = lflag[s0];
    w.sim_uid[(int64_t)t * MW + s] = uid;
    if (s0 == s) {
      w.uleaf[(int64_t)t * MW + uid] = w.leaves[(int64_t)t * MW + s];
      w.ufirst[(int64_t)t * MW + uid] = s;
    }
  }
  if (tid == 0) {
    w.ucount[t] = nu;
    w.gcount[t] = s_glog;
    s_st[OMQ_ST_ULEAVES] += (unsigned long long)nu;
    s_st[OMQ_ST_SIMS] += (unsigned long long)W;
  }
  __syncthreads();
  if (tid < OMQ_NSTATS && s_st[tid] != 0)
    atomicAdd(reinterpret_cast<unsigned long long*>(&w.stats[(int64_t)t * OMQ_NSTATS + tid]),
              s_st[tid]);
}

}  // namespace omq

// ---- host launcher (C++ linkage; the C ABI wrappers live in capi.hip) ----
namespace omq {

size_t select_lds_bytes(int W) {
  return (size_t)W * (4 + 4 + 8 + 8) + (size_t)W * (4 + 2) +
         (size_t)kSelWaves * OMQ_MAX_ROW * 2;
}

hipError_t launch_select(const omq_forest& f, const omq_wave& w, int W, float c_puct,
                         float virtual_loss, int max_depth, int vl_atomic, hipStream_t stream) {
  SelCfg c;
  c.W = W;
  c.c_puct = c_puct;
  c.vlf = virtual_loss;
  c.vli = (int)virtual_loss;
  c.max_depth = max_depth;
  c.vl_atomic = vl_atomic;
  const size_t lds = select_lds_bytes(W);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)select_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)select_lds_bytes(OMQ_MAX_WAVE));
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL(select_kernel, dim3(f.num_trees), dim3(kSelThreads), lds, stream, f, w, c);
  return hipGetLastError();
}

}  // namespace omq
