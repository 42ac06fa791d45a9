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

#ifndef OMQ_SEL_THREADS
#define OMQ_SEL_THREADS 1024
#endif
constexpr int kSelThreads = OMQ_SEL_THREADS;
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

// The arrays the selection touches (a compact kernel argument block: passing both full
// structures costs more scalar registers than the kernel has).
struct SelArgs {
  int32_t* N;
  const float* W;
  const float* P;
  const int32_t* first;
  const int32_t* nchild;
  int32_t* paths;
  int32_t* path_len;
  int32_t* leaves;
  int32_t* sim_uid;
  int32_t* uleaf;
  int32_t* ufirst;
  int32_t* ucount;
  int32_t* glog;
  int32_t* gcount;
  uint16_t* gmembers;
  int64_t* stats;
  int32_t* status;
  int capacity;
  int max_wave;
  int max_depth_buf;
};

// Max of a uint32 over the 64 lanes, made uniform: DPP row shifts 1,2,4,8 (each a single
// v_max_u32_dpp; a lane whose DPP source lies outside its row reads 0, the identity) leave
// each row's maximum in its last lane; the four row maxima are read into scalar registers
// and combined there.
__device__ inline uint32_t wave_max_rows(uint32_t x) {
  int v = (int)x;
  v = (int)max((uint32_t)v, (uint32_t)__builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true));
  v = (int)max((uint32_t)v, (uint32_t)__builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true));
  v = (int)max((uint32_t)v, (uint32_t)__builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true));
  v = (int)max((uint32_t)v, (uint32_t)__builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true));
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane(v, 15);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane(v, 31);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane(v, 47);
  const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane(v, 63);
  return max(max(r0, r1), max(r2, r3));
}

// Max of a float over the 64 lanes, made uniform: DPP row shifts 1,2,4,8 then row broadcasts
// of lanes 15 and 31 (a lane whose DPP source is invalid keeps its value), read from lane 63.
// NaN lanes are ignored unless every lane is NaN.
__device__ inline float wave_max_bcast(float x) {
  int v = __float_as_int(x);
  v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(__builtin_amdgcn_update_dpp(v, v, 0x111, 0xF, 0xF, false))));
  v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(__builtin_amdgcn_update_dpp(v, v, 0x112, 0xF, 0xF, false))));
  v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(__builtin_amdgcn_update_dpp(v, v, 0x114, 0xF, 0xF, false))));
  v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(__builtin_amdgcn_update_dpp(v, v, 0x118, 0xF, 0xF, false))));
  v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(__builtin_amdgcn_update_dpp(v, v, 0x142, 0xA, 0xF, false))));
  v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(__builtin_amdgcn_update_dpp(v, v, 0x143, 0xC, 0xF, false))));
  return __int_as_float(__builtin_amdgcn_readlane(v, 63));
}

// Serial chain of row-argmaxes for one group (whole wave).  ch[r] receives, for the r-th
// member, (child index << 16) | rank among the members that chose the same child, or
// kNoChild.  Child counts are left in cnt_s[0..k).  Returns the first rank without a child
// (or -1).
//
// Exact score (the reference's fp32 expression):
//     sc = Q + ((c*P)*s)/d,   Q = W/((float)N + VL),  d = (float)(1+N),  s = sqrt((float)Np)
// Lane l holds children l, l+64, ... (slot j holds child j*64 + l).  Each lane keeps, per child,
// qa = W*r' and a = (c*P)*r, with r and r' Newton-refined reciprocals of d and of (float)N + VL
// (|r*d - 1| <= 2^-24(1+eps)), and each step ranks the children by ap = fma(s, a, qa).  With
// U = s*(c*P)/d: |qa - Q| <= |Q|*2^-22.4, |ap - (Q + U)| <= U*2^-23 + |Q|*2^-22.4 + |ap|*2^-24
// and |sc - (Q + U)| <= U*2^-23 + |sc|*2^-24; since U <= |ap| + |Q| + tiny,
// |ap - sc| <= (|ap| + QB) * 2^-21 with QB >= max |Q|.  Let A = max ap and
// E = (|A| + QB) * 2^-20.5.  The child with ap = A has exact score >= A - E; a child w whose
// exact score reaches the maximum then has ap_w >= A - 2E (|ap_w| <= |A| + 2E keeps e_w <= E).
// So the exact argmax is among the candidates ap >= T = A - (|A| + QB) * 2^-19 (a further
// factor 2^0.5 of margin).  A single candidate is the exact argmax (A is checked above -1e8,
// so its exact score is above the -1e9 start value); otherwise the candidates are scored
// exactly (two correctly rounded divisions each) and compared in scalar registers.  No
// candidate (NaN or infinite scores) or a negative c*P scores every child exactly.
//
// QB is fixed for the whole chain: W does not change during selection and N only grows, so
// |Q| = |W|/((float)N + VL) of every later state is at most its value at the start (the
// approximation error of qa, 2^-22.4 relative, is absorbed by the 2^0.5 margin above).
//
// An unvisited child i (N == 0) carries qa = (1024 - i) * 2^90 and a = 0: it dominates every
// visited child, and a lower index dominates a higher one by a factor >= 1 + 2^-10, so the
// lowest-index unvisited child is the single candidate, as the reference's first-unvisited
// rule requires.  A padding child (index >= k) carries qa = -inf, a = 0.  Every child's state
// after its next pick is kept too, so a pick is a register select; the state after the
// following pick is computed at the start of the next step, off the pick's dependency chain.
// Ranks are counted per child in registers.  The parent's sqrt for ranks r0..r0+63 is computed
// once per 64 steps (lane l holds rank r0+l); the 64 records of a block are kept one per lane
// and stored together.
__device__ inline float refined_rcp(float d) {
  const float r = __builtin_amdgcn_rcpf(d);
  return __builtin_fmaf(r, __builtin_fmaf(-d, r, 1.0f), r);
}

// approximate selection state of a child with denominator d = (float)(1+N): (qa, a), computed
// without branches; returns whether the child is visited
__device__ inline bool child_state(float d, float w, float cp, int i, float vlf, float* qa,
                                   float* a) {
  const bool vis = d != 1.0f;
  const float qv = w * refined_rcp((d - 1.0f) + vlf);
  const float av = cp * refined_rcp(d);
  *qa = vis ? qv : __builtin_ldexpf((float)(1024 - i), 90);
  *a = vis ? av : 0.0f;
  return vis;
}

// Exact argmax of the step among the candidate children (all children when `all`), or -1 when
// no child scores above -1e9: exact scores as order-preserving keys, compared in scalar
// registers, lowest index on ties; an unvisited child ranks above every visited one, lower
// index first.
template <int R>
__device__ inline int exact_pick(const float* den, const float* wv,
                                                    const float* cp, uint32_t bits, bool all,
                                                    int k, float s, float vlf) {
  const int lane = lane_id();
  uint32_t kx[R];
  uint64_t cj[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int i = j * kWave + lane;
    const bool cand = all ? (i < k) : (((bits >> j) & 1u) != 0);
    cj[j] = __ballot(cand);
    kx[j] = 0u;
    if (cand) {
      if (den[j] == 1.0f) {
        kx[j] = 0xFFFF0000u | (uint32_t)(0xFFFF - i);
      } else {
        const float qe = wv[j] / ((den[j] - 1.0f) + vlf);
        float sc = qe + (cp[j] * s) / den[j];
        sc = sc + 0.0f;  // -0 -> +0, so that equal scores compare equal
        kx[j] = (sc > -1e9f) ? fkey(sc) : 0u;
      }
    }
  }
  uint32_t bk = 0u;
  int bidx = 0x7FFFFFFF;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    uint64_t rest = cj[j];
    while (rest) {
      const int l = lowest_lane(rest);
      rest &= rest - 1;
      const uint32_t kv = (uint32_t)readlane_i((int)kx[j], l);
      const int idx = j * kWave + l;
      if (kv > bk || (kv == bk && kv != 0u && idx < bidx)) {
        bk = kv;
        bidx = idx;
      }
    }
  }
  return bk != 0u ? bidx : -1;
}

template <int R>
__device__ int run_chain(const SelArgs& f, int64_t tb, int first, int k, int Np0, int m,
                         const SelCfg& c, uint32_t* ch, uint16_t* cnt_s) {
  const int lane = lane_id();
  const float vlf = c.vlf;
  const float fvl = (float)c.vli;
  float wv[R], cp[R], den[R], q[R], ar[R], qn[R], arn[R];
  float qbl = 0.0f;
  bool negcp = false;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int i = j * kWave + lane;
    if (i < k) cnt_s[i] = 0;
    if (i < k) {
      const int64_t node = tb + first + 1 + i;  // child of edge first+i is node first+i+1
      const int n = f.N[node];
      wv[j] = f.W[node];
      cp[j] = c.c_puct * f.P[node];
      den[j] = (float)(1 + n);
      negcp = negcp || !(cp[j] >= 0.0f);
      if (child_state(den[j], wv[j], cp[j], i, vlf, &q[j], &ar[j]))
        qbl = fmaxf(qbl, __builtin_fabsf(q[j]));
      child_state(den[j] + fvl, wv[j], cp[j], i, vlf, &qn[j], &arn[j]);
    } else {
      wv[j] = 0.0f;
      cp[j] = 0.0f;
      den[j] = 2.0f;
      q[j] = qn[j] = -__builtin_inff();
      ar[j] = arn[j] = 0.0f;
    }
  }
  const uint32_t QBb = wave_max_rows(__float_as_uint(qbl));  // bits of QB (non-negative)
  const float qbt = __uint_as_float(QBb) * (-1.0f / 524288.0f);
  const bool exact_only = __ballot(negcp) != 0;
  if (Np0 == 0 && c.vli == 0) {
    // N is never negative: Np = 0 at every step, the reference returns no child
    for (int r = lane; r < m; r += kWave) ch[r] = kNoChild;
    for (int i = lane; i < k; i += kWave) cnt_s[i] = 0;
    wave_sync();
    return m > 0 ? 0 : -1;
  }
  int first_end = -1;
  int powner = -1, pjj = 0;  // the previous step's pick, whose next state is pending
  for (int r0 = 0; r0 < m; r0 += kWave) {
    const int Npl = Np0 + c.vli * (r0 + lane + 1);
    const float svec = sqrtf((float)Npl);
    const int rend = min(kWave, m - r0);
    uint32_t rec = kNoChild;
    for (int rr = 0; rr < rend; ++rr) {
      // state after the next pick of the child picked in the previous step
      {
        float dw = den[0], ww = wv[0], cw = cp[0];
#pragma unroll
        for (int j = 1; j < R; ++j) {
          const bool sel = j == pjj;
          dw = sel ? den[j] : dw;
          ww = sel ? wv[j] : ww;
          cw = sel ? cp[j] : cw;
        }
        float qx, ax;
        child_state(dw + fvl, ww, cw, pjj * kWave + lane, vlf, &qx, &ax);
        const bool mine = lane == powner;
#pragma unroll
        for (int j = 0; j < R; ++j) {
          const bool hit = mine && j == pjj;
          qn[j] = hit ? qx : qn[j];
          arn[j] = hit ? ax : arn[j];
        }
      }
      const float s = readlane_f(svec, rr);
      float ap[R];
#pragma unroll
      for (int j = 0; j < R; ++j) ap[j] = __builtin_fmaf(s, ar[j], q[j]);
      float lm;
      if (R == 1) {
        lm = ap[0];
      } else {
        float t[R];
#pragma unroll
        for (int j = 0; j < R; ++j) t[j] = ap[j];
#pragma unroll
        for (int w = 1; w < R; w <<= 1)
#pragma unroll
          for (int j = 0; j + w < R; j += 2 * w) t[j] = fmaxf(t[j], t[j + w]);
        lm = t[0];
      }
#if defined(OMQ_STEP_V4)
      const uint32_t Ak = wave_max_u32(fkey(lm));
      const float A = funkey(Ak);
      const float T = __builtin_fmaf(__builtin_fabsf(A), -1.0f / 524288.0f, A) + qbt;
      const bool aok = Ak > 0x334143DFu;
#elif defined(OMQ_STEP_V3)
      const float A = wave_max_bcast(lm);
      // T = A - |A| * 2^-19 - QB * 2^-19
      const float T = __builtin_fmaf(__builtin_fabsf(A), -1.0f / 524288.0f, A) + qbt;
      // A > -1e8 keeps the exact score of a single candidate above -1e9; as bits: every
      // non-negative A and every negative A of magnitude below 1e8 lies below bits(-1e8)
      const bool aok = __float_as_uint(A) < 0xCCBEBC20u;
#else
      const uint32_t Ak = wave_max_rows(fkey(lm));
      const float A = funkey(Ak);
      // T = A - (|A| + QB) * 2^-19 = A * (1 -+ 2^-19) - QB * 2^-19 (key MSB set: A >= 0)
      const float T = __builtin_fmaf(A, (Ak & 0x80000000u) ? 0.99999809265136719f
                                                           : 1.0000019073486328f, qbt);
      const bool aok = Ak > 0x334143DFu;
#endif
      uint32_t bits = 0;
#pragma unroll
      for (int j = 0; j < R; ++j) bits |= (ap[j] >= T) ? (1u << j) : 0u;
      const uint64_t cm = __ballot(bits != 0);
      // A > -1e8 (key 0x334143DF) keeps the exact score of a single candidate above -1e9
      bool single = !exact_only && __popcll(cm) == 1 && aok;
      if (R > 1) single = single && __ballot((bits & (bits - 1)) != 0) == 0ull;
      int win;
      if (single) {
        const int l = lowest_lane(cm);
        win = (R == 1) ? l : (__ffs((unsigned)readlane_i((int)bits, l)) - 1) * kWave + l;
      } else {
        win = exact_pick<R>(den, wv, cp, bits, exact_only || cm == 0, k, s, vlf);
        win = __builtin_amdgcn_readfirstlane(win);
        if (win < 0 && first_end < 0) first_end = r0 + rr;
      }
      if (win >= 0) {
        const int owner = win & (kWave - 1);
        const int jj = win / kWave;
        const bool mine = lane == owner;
#pragma unroll
        for (int j = 0; j < R; ++j) {
          const bool hit = mine && j == jj;
          q[j] = hit ? qn[j] : q[j];
          ar[j] = hit ? arn[j] : ar[j];
          den[j] = hit ? den[j] + fvl : den[j];
        }
        powner = owner;
        pjj = jj;
      } else {
        powner = -1;
      }
      rec = (lane == rr) ? (uint32_t)win : rec;
    }
    // ranks of the block's picks: count of the child before the block (cnt_s) plus the number
    // of earlier picks of the same child within the block
    const bool valid = lane < rend && rec != kNoChild;
    const uint32_t key = valid ? rec : 0u;
    const uint32_t base = valid ? (uint32_t)cnt_s[key] : 0u;
    uint64_t pend = __ballot(valid);
    uint32_t inb = 0;
    bool last = false;
    while (pend) {
      const uint32_t kk = (uint32_t)readlane_i((int)key, lowest_lane(pend));
      const bool eq = valid && key == kk;
      const uint64_t same = __ballot(eq);
      if (eq) {
        inb = __builtin_amdgcn_mbcnt_hi((uint32_t)(same >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)same, 0u));
        last = (same >> lane) == 1ull;
      }
      pend &= ~same;
    }
    if (valid && last) cnt_s[key] = (uint16_t)(base + inb + 1);
    if (lane < rend) ch[r0 + lane] = valid ? ((key << 16) | (base + inb)) : kNoChild;
    wave_sync();
  }
  return first_end;
}

__device__ inline int dispatch_chain(const SelArgs& f, int64_t tb, int first, int k, int Np0,
                                     int m, const SelCfg& c, uint32_t* ch, uint16_t* cnt_s) {
  switch ((k + kWave - 1) / kWave) {  // k <= OMQ_MAX_ROW = 512
    case 1: return run_chain<1>(f, tb, first, k, Np0, m, c, ch, cnt_s);
    case 2: return run_chain<2>(f, tb, first, k, Np0, m, c, ch, cnt_s);
    case 3: return run_chain<3>(f, tb, first, k, Np0, m, c, ch, cnt_s);
    case 4: return run_chain<4>(f, tb, first, k, Np0, m, c, ch, cnt_s);
    case 5: return run_chain<5>(f, tb, first, k, Np0, m, c, ch, cnt_s);
    case 6: return run_chain<6>(f, tb, first, k, Np0, m, c, ch, cnt_s);
    case 7: return run_chain<7>(f, tb, first, k, Np0, m, c, ch, cnt_s);
    default: return run_chain<8>(f, tb, first, k, Np0, m, c, ch, cnt_s);
  }
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

__global__ __launch_bounds__(kSelThreads) void select_kernel(SelArgs f, SelCfg c) {
  SelArgs& w = f;
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
  const int MW = w.max_wave, MD = w.max_depth_buf;
  const int64_t gmax = (int64_t)MW * MD;
  int32_t* N = f.N;
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
      const int k = f.nchild[tb + p];
      const int first = f.first[tb + p];
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
  SelArgs a;
  a.N = f.visit_counts;
  a.W = f.value_sums;
  a.P = f.priors;
  a.first = f.first_child;
  a.nchild = f.num_children;
  a.paths = w.paths;
  a.path_len = w.path_len;
  a.leaves = w.leaves;
  a.sim_uid = w.sim_uid;
  a.uleaf = w.uleaf;
  a.ufirst = w.ufirst;
  a.ucount = w.ucount;
  a.glog = w.glog;
  a.gcount = w.gcount;
  a.gmembers = w.gmembers;
  a.stats = w.stats;
  a.status = w.status;
  a.capacity = f.capacity;
  a.max_wave = w.max_wave;
  a.max_depth_buf = w.max_depth;
  hipLaunchKernelGGL(select_kernel, dim3(f.num_trees), dim3(kSelThreads), lds, stream, a, c);
  return hipGetLastError();
}

}  // namespace omq
