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
// wavefront per group; the chain keeps the row's selection state in registers, slot j of lane
// l holding child j*64 + l.  In the kernels for rows of at most 192 children, groups of one
// member are taken one per lane instead (small_groups); in those for 256 and 384, their leaves
// are finished by all threads at once (leaf_pass).  The members of a group are kept in
// simulation order in LDS and partitioned among the chosen children by a counting scatter,
// which yields the groups of the next level.  In the kernels for rows of at most 192 children,
// the level-1 chains run during the root chain, block by block (the level overlap below).
//
// Virtual loss is materialised once per group (N[p] += VL*m, p is owned by one group per
// wave), or with one atomic per path entry when vl_atomic is set.

#include <algorithm>
#include <atomic>

#include "omq_common.h"

namespace omq {

constexpr uint32_t kNoChild = 0xFFFFFFFFu;

struct SelCfg {
  int W;           // simulations per tree in this wave
  float c_puct;
  float vlf;       // virtual loss as float
  int vli;         // (int)virtual loss
  int max_depth;   // forced leaf at depth max_depth-1
  int vl_atomic;
  int spin_limit;  // polls of a follower's bounded wait for the root chain
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
  int num_trees;
  // selection scratch (omq_wave::sel_scratch)
  int32_t* lflag;  // [T*max_wave] 1 for the first simulation of a leaf group
  int32_t* lfs;    // [T*max_wave] first simulation of a simulation's leaf group
};

// What the select kernel reads and writes for the unique leaves' records (waves of at most
// OMQ_SELECT_RECORDS_MAX_WAVE simulations): a kernel argument of its own, after SelArgs and
// SelCfg, whose places in the argument block it leaves as they were.
struct RecordArgs {
  const int32_t* actions;
  const uint64_t* root_keys;
  const uint32_t* root_legal;
  uint64_t* ukey;
  int32_t* ulegal;
  int game;
  int num_actions;
  int legal_words;
  int min_legal;
  int max_legal;
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

// One step of a wave max over order-preserving keys: the DPP source of an out-of-row or
// masked lane reads 0, the identity of the max, so each step is one fused v_max_u32_dpp.
#define OMQ_DPP_MAX(v, ctrl, rmask)                                                        \
  v = (int)max((uint32_t)(v),                                                             \
               (uint32_t)__builtin_amdgcn_update_dpp(0, (v), (ctrl), (rmask), 0xF, true))
// Keeps the instruction scheduler from moving instructions across this point (used to
// interleave two independent dependency chains by hand).
#define OMQ_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)
// Materialises a value at this point (an empty asm that reads and rewrites the register), so
// that the compiler cannot sink its computation towards its later use.
#define OMQ_PIN(x) asm volatile("" : "+v"(x))

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
// factor 2^0.5 of margin).  (That is the test of the steps over a whole row, whose states all
// use refined reciprocals; the steps over one child per lane use raised keys instead, with the
// argument at raised_key, which also covers states formed with the hardware reciprocal.)  A single candidate is the exact argmax; otherwise the candidates
// are scored exactly (two correctly rounded divisions each) and compared in scalar registers.
// No candidate (NaN or infinite scores), a negative c*P or QB >= 1e8 scores every child
// exactly.
//
// QB is fixed for the whole chain: W does not change during selection and N only grows, so
// |Q| = |W|/((float)N + VL) of every later state is at most its value at the start (the
// approximation error of qa, 2^-22.4 relative, is absorbed by the 2^0.5 margin above).  With
// QB < 1e8, c*P >= 0 and s >= 0 every real child has ap >= -QB > -1e8, so the exact score of a
// single candidate is above the reference's -1e9 start value.
//
// An unvisited child i (N == 0) carries qa = (1024 - i) * 2^90 and a = 0: it dominates every
// visited child, and a lower index dominates a higher one by a factor >= 1 + 2^-10, so the
// lowest-index unvisited child is the single candidate, as the reference's first-unvisited
// rule requires.  A padding child (index >= k) carries qa = -inf, a = 0.  Every child's state
// after its next pick is kept too, so a pick is a register select; each step forms every
// child's state after its next pick anew during its wave max, off the pick's dependency chain.
// The parent's sqrt for ranks r0..r0+63 is computed once per 64 steps (lane l holds rank
// r0+l); the 64 picks of a block are kept one per lane, and their ranks are counted after the
// block.
//
// Rows of more than 64 children run most steps on a window of at most 64 contenders, one per
// lane: the children with the largest ap at the window's first step.  A non-contender keeps its
// state during the window and its ap only grows with s, so fma(s_end, a, qa) at the last rank
// of the block bounds it for the whole window; a step whose threshold T exceeds that bound has
// the same candidates (and maximum) over the contenders as over the whole row, so the window
// takes the step.  The first step where T does not exceed the bound ends the window before it
// is taken.  Contenders keep their index order in the lanes, so lowest-lane ties remain
// lowest-index ties.
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
// index first.  Lane l, slot j holds the child of order j*64 + l.
template <int R>
__device__ inline int exact_pick(const float* den, const float* wv, const float* cp,
                                 uint32_t bits, bool all, int k, float s, float vlf) {
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

// exact_pick for one child per lane, lanes in index order (a row of at most 64 children, or a
// contender window), among the candidate lanes cm: their exact keys (an unvisited child's by its
// lane, which orders as its index does), the largest key's lowest lane being the pick; -1 when
// no candidate scores above -1e9.  The keys are formed in every lane (a select, not a branch);
// two candidates, the common case, are compared in scalar registers, more by one wave max.
__device__ inline int exact_pick_lane(float den, float wv, float cp, uint64_t cm, float s,
                                      float vlf) {
  const int lane = lane_id();
  const float qe = wv / ((den - 1.0f) + vlf);
  float sc = qe + (cp * s) / den;
  sc = sc + 0.0f;  // -0 -> +0, so that equal scores compare equal
  uint32_t kx = (sc > -1e9f) ? fkey(sc) : 0u;
  kx = den == 1.0f ? 0xFFFF0000u | (uint32_t)(0xFFFF - lane) : kx;
  kx = __builtin_amdgcn_inverse_ballot_w64(cm) ? kx : 0u;
  if (__popcll(cm) == 2) {
    const int l1 = lowest_lane(cm);
    const int l2 = lowest_lane(cm & (cm - 1));
    const uint32_t k1 = (uint32_t)readlane_i((int)kx, l1);
    const uint32_t k2 = (uint32_t)readlane_i((int)kx, l2);
    const uint32_t bk = max(k1, k2);
    return bk == 0u ? -1 : (k2 > k1 ? l2 : l1);
  }
  const uint32_t bk = wave_max_u32(kx);
  if (bk == 0u) return -1;
  return lowest_lane(__ballot(kx == bk));
}

// Selection state of the children held by a lane (R slots).
template <int R>
struct Row {
  float q[R], ar[R];    // current approximate state (qa, a)
  float qn[R], arn[R];  // state after the next pick
  float den[R];         // (float)(1 + N) including this chain's picks
  float wv[R], cp[R];   // W and c_puct * P
  int cn[R];            // picks of the child in this chain so far
};

// Wave max of a float as order-preserving keys (made uniform).
__device__ inline float wave_max_key(float x) { return funkey(wave_max_u32(fkey(x))); }

// Key of the raised value hi = ap + (2|ap| + |qa| + QW) * M of a lane in the steps over one lane
// per child, M = 2^-20.5 rounded up.  QW bounds |qa| of every visited lane that can hold the
// step's maximum (the chain's QB, or the window's contenders' bound).
//
// Why the exact argmax w is a candidate (hi_w >= A, A = max ap, held by lane m): each lane's
// |ap - sc| <= e = 8.1u (|ap| + |Q|) (1 + 2^-20), u = 2^-24 (the argument above run_chain's
// helpers, written per child).  A lane's reciprocals r (of d) and r' are Newton-refined
// (|r d - 1| <= u (1 + 2^-20)) or, in the state after a pick that a step forms, the hardware
// reciprocal alone: |r d - 1| <= 2^-23.38 = 1.54u, the largest error of v_rcp_f32 over every
// float in [1, 2^24], which holds every denominator here (tests/test_gpu_rcp_bound.py).  So
// |qa - Q| <= (1.54u + 2u) |Q| (the reciprocal, qa's product, Q's quotient) and the U's differ
// by (1.54u + u + 2u) U (the reciprocal, a's product, the exact U's product and quotient);
// with u |ap| + u |sc| from the last roundings and U <= |ap| + |Q|, e <= 8.1u (|ap| + |Q|).
// Then sc_w >= sc_m >= A - e_m and ap_w >= A - e_m - e_w; with |A| <= |ap_w| + e_m + e_w and
// |Q_m| <= QW, e_m + e_w <= 8.1u X (1 + 9u) for X = 2|ap_w| + |qa_w| + QW.  hi_w is the rounded
// ap_w + fl(fl(2|ap_w| + |qa_w|) + QW) M >= ap_w + X (1 - 2u) M, and M = 11.3u > 8.1u
// (1 + 9u) / (1 - 2u) covers it; rounding to nearest keeps a real value >= A (a float) >= A.
// The lane holding A has hi >= ap = A.
constexpr float kMarg = 0x1.6a09e8p-21f;
__device__ inline uint32_t raised_key(float ap, float qa, float qw) {
  const float x = (2.0f * __builtin_fabsf(ap) + __builtin_fabsf(qa)) + qw;
  return fkey(__builtin_fmaf(x, kMarg, ap));
}

// qa of a padding lane in the one-lane steps: its ap stays here and its raised value stays
// finite, far below any maximum above -1e9
constexpr float kPadQ = -1e30f;

// Smallest key at which lane_steps takes a step: that of -1e9 (below it no child can be picked
// without the exact comparison).
constexpr uint32_t kKeyFloor = 0x319194D7u;  // fkey(-1e9f)
constexpr uint32_t kKeyInf = 0xFF800000u;    // fkey(+inf)
static_assert(kKeyFloor == ~__builtin_bit_cast(uint32_t, -1e9f), "fkey of a negative float");
static_assert(kKeyInf == (__builtin_bit_cast(uint32_t, __builtin_inff()) ^ 0x80000000u),
              "fkey of a positive float");

// Steps of a chain whose children are held one per lane (rows of at most 64 children, or a
// contender window), from rank rr up to rank rend.
//
// A step ranks the lanes by ap = fma(s, a, qa) and takes the wave max A (as the key Ak).  The
// candidates are the lanes whose raised key (raised_key: hi = ap + (2|ap| + |qa| + QW) * 2^-20.5)
// is at least Ak; the exact argmax is among them (the argument at raised_key), and the lane
// holding A is one, so a step has at least one.  A single candidate is the pick.  A step is
// taken here only when A lies strictly between klo and khi (keys): klo is at least the key of
// -1e9, and khi at most that of +inf (0 in exact-only mode, which takes no step here).  A NaN
// ap can only add candidates (a NaN hi), which sends the step to the exact comparison.
// Padding lanes hold qa = kPadQ, a = 0: their hi stays finite and below any A above -1e9.
//
// A pick advances the picked lane to its next state (a register select); every lane's state
// after its next pick is formed anew during each step's wave max.  The steps with a
// single candidate run in a loop of their own; any other step leaves that loop for the exact
// comparison among its candidates (all children when A is out of range) and comes back.
// Keeping the rare step out of the loop body leaves the common step without the register
// copies that joining the two paths inside it costs.  Lane r of rec / rnk receives the pick at
// rank r (the lane, or -1 for none) and the chain's picks of that child up to and including it
// (its rank among them plus one).
//   WINDOW: contender window; klo is also at least the largest raised key of the
//           non-contenders at the block's last rank, which bounds their raised keys over the
//           whole window (ap and hi only grow with s).  With A above it, no non-contender is a
//           candidate and A is the maximum over the whole row.  The steps end before the first
//           rank whose A is not in range; that rank is returned.  Every step of a window picks.
//   else:   every step up to rend is taken; a rank without a child records -1, and the first
//           such rank goes to first_end (when it is still negative).
// Returns the first rank not taken.
template <bool WINDOW>
__device__ inline int lane_steps(Row<1>& y, float svec, int rr, int rend, float fvl, float vlf,
                                 float qw, uint32_t klo, uint32_t khi, int k, int r0,
                                 int* first_end, uint32_t* rec, uint32_t* rnk) {
  const int lane = lane_id();
  // A in range: (Ak - kbase) < kspan as unsigned
  const uint32_t kbase = klo + 1u;
  const uint32_t kspan = khi > kbase ? khi - kbase : 0u;
  // the ranks are uniform; said explicitly, so that the step loop's counter and exit stay in
  // scalar registers whatever the caller's rr was derived from
  rr = __builtin_amdgcn_readfirstlane(rr);
  // (the row's W and c*P in registers before the loop, so that no wait for their loads is left
  // inside it)
  OMQ_PIN(y.wv[0]);
  OMQ_PIN(y.cp[0]);
  while (rr < rend) {
    // ---- steps with a single candidate: two exits, at the bottom.  The candidates of a step
    // take their next state at once (the single candidate when the step is taken), so that
    // the next step's scores wait only for the compare with the wave max, not for the scalar
    // test of the step; a step that is not taken puts their state back after the loop.  Apart
    // from that, it changes nothing but the states after the next pick (formed anew every
    // step), and nothing of it is kept past the loop.
    rr = __builtin_amdgcn_readfirstlane(rr);
    int pc = 1, pen = 0;
    uint32_t Akl = 0u;
    uint64_t cm = 0;
    float qs = 0.0f;
    // one step; true when it was taken and the next rank is in the block.  Four steps per
    // loop turn: the loop's taken branch back is paid once per four steps (C3 select 197.6 ->
    // 192.5 us, C4 413.5 -> 407.7 us; two per turn: 196.4 and 411.0 us; eight do not build,
    // the inline asm's scalar operands then getting vector registers)
    auto one_step = [&]() -> bool {
      const float s = readlane_f(svec, rr);
      const float ap = __builtin_fmaf(s, y.ar[0], y.q[0]);
      // The wave max of the keys is interleaved with the raised key and with every lane's
      // state after its next pick (both independent of it).  That state follows from the
      // lane's current count, so it is formed anew each step: only the previous step's pick
      // changes it.  It takes the hardware reciprocals as they are (the argument at
      // raised_key covers them).
      // Two independent instructions sit between consecutive DPP steps (a DPP source needs
      // two wait states after its write), so the wave max runs without hazard nops.  Each group
      // pins its inputs first, which keeps its instructions after the previous DPP step.  The
      // raised key is raised_key's expression, split across the groups.
      int v = (int)fkey(ap);
      float d2 = y.den[0] + fvl;
      float e1 = d2 - 1.0f;
      OMQ_SCHED_FENCE();
      OMQ_DPP_MAX(v, 0x111, 0xF);  // row_shr:1
      OMQ_PIN(d2);
      OMQ_PIN(e1);
      float e2 = e1 + vlf;
      float r2 = __builtin_amdgcn_rcpf(d2);
      OMQ_SCHED_FENCE();
      OMQ_DPP_MAX(v, 0x112, 0xF);  // row_shr:2
      OMQ_PIN(e2);
      float apc = ap;
      OMQ_PIN(apc);
      float r1 = __builtin_amdgcn_rcpf(e2);
      float x1 = 2.0f * __builtin_fabsf(apc);
      OMQ_SCHED_FENCE();
      OMQ_DPP_MAX(v, 0x114, 0xF);  // row_shr:4
      OMQ_PIN(x1);
      float qc = y.q[0];
      OMQ_PIN(qc);
      float x2 = x1 + __builtin_fabsf(qc);
      qs = qc;
      OMQ_SCHED_FENCE();
      OMQ_DPP_MAX(v, 0x118, 0xF);  // row_shr:8
      OMQ_PIN(x2);
      OMQ_PIN(r2);
      float x3 = x2 + qw;
      // a picked child is visited afterwards (virtual loss >= 1 here)
      y.arn[0] = y.cp[0] * r2;
      OMQ_SCHED_FENCE();
      OMQ_DPP_MAX(v, 0x142, 0xA);  // row_bcast:15
      OMQ_PIN(x3);
      OMQ_PIN(r1);
      const float hi = __builtin_fmaf(x3, kMarg, apc);
      y.qn[0] = y.wv[0] * r1;
      OMQ_SCHED_FENCE();
      OMQ_DPP_MAX(v, 0x143, 0xC);  // row_bcast:31
      float hic = hi;
      OMQ_PIN(hic);
      const uint32_t hk = fkey(hic);
      const uint32_t Ak = (uint32_t)__builtin_amdgcn_readlane(v, 63);
      const bool cand = hk >= Ak;
      // the candidates take their next state now (d2 is the denominator after a pick)
      y.q[0] = cand ? y.qn[0] : y.q[0];
      y.ar[0] = cand ? y.arn[0] : y.ar[0];
      y.den[0] = cand ? d2 : y.den[0];
      y.cn[0] = cand ? y.cn[0] + 1 : y.cn[0];
      OMQ_PIN(y.q[0]);
      OMQ_PIN(y.ar[0]);
      OMQ_PIN(y.den[0]);
      OMQ_PIN(y.cn[0]);
      OMQ_SCHED_FENCE();
      // The step is taken when A is in range and it has a single candidate l; the loop goes
      // on while the next rank is in the block too.  Both conditions besides the candidate
      // count are folded into pen (bit 1: A out of range, bit 2: the block's last rank), formed
      // in scalar registers while the compare runs (as plain C the compiler routes them
      // through vector registers), so that the branch waits only for pc + pen == 1.
      {
        int tmp;
        asm("s_sub_u32 %0, %2, %3\n\t"
            "s_cmp_lt_u32 %0, %4\n\t"
            "s_cselect_b32 %0, 0, 2\n\t"
            "s_cmp_lt_i32 %5, %6\n\t"
            "s_cselect_b32 %1, 0, 4\n\t"
            "s_or_b32 %0, %0, %1"
            : "=&s"(pen), "=&s"(tmp)
            : "s"(Ak), "s"(kbase), "s"(kspan), "s"(__builtin_amdgcn_readfirstlane(rr + 1)),
              "s"(rend)
            : "scc");
      }
      cm = __ballot(cand);
      pc = __popcll(cm);
      Akl = Ak;
      // (s_ff1 of an empty mask gives -1: then any lane will do for the writes below, which
      // the step that takes rank rr later repeats.)
      int l;
      asm("s_ff1_i32_b64 %0, %1" : "=s"(l) : "s"(cm));
      // lane rr := pick / its rank.  The lane select goes through m0, which the "{m0}"
      // operand hands to the compiler (v_writelane may read only one SGPR besides m0).
      const int rk = readlane_i(y.cn[0], l);
      asm volatile("v_writelane_b32 %0, %1, m0" : "+v"(*rec) : "s"(l), "{m0}"(rr));
      asm volatile("v_writelane_b32 %0, %1, m0" : "+v"(*rnk) : "s"(rk), "{m0}"(rr));
      // (the next rank does not wait for the test either; an untaken step's rank is given
      // back below)
      rr += 1;
      return pc + pen == 1;
    };
    for (;;) {
      if (!one_step()) break;
      if (!one_step()) break;
      if (!one_step()) break;
      if (!one_step()) break;
    }
    if (pc == 1 && (pen & 2) == 0) return rr;  // the last step was taken: the block's end
    // not taken: the candidates' state as it was.  qa comes back from its copy; the count, the
    // denominator (integral and below 2^24, so the subtraction is exact) and a follow from it
    // (a = 0 for an unvisited child; c*P = 0 on a padding lane)
    {
      rr -= 1;
      const bool cand = __builtin_amdgcn_inverse_ballot_w64(cm);
      y.q[0] = qs;
      if (cand) {
        const float d = y.den[0] - fvl;
        y.den[0] = d;
        y.cn[0] -= 1;
        y.ar[0] = d == 1.0f ? 0.0f : y.cp[0] * refined_rcp(d);
      }
    }

    // ---- the step at rr was not taken above (its state is as it was): the
    // window's end, or the exact comparison among its candidates (every child when A is out of
    // range), whose wave max and candidates the loop's last step left in Akl and cm ----
    const float s = readlane_f(svec, rr);
    const bool in_range = Akl - kbase < kspan;
    if (WINDOW && !in_range) return rr;
    uint64_t cset = in_range ? cm : __ballot(lane < k);
    if (in_range && __popcll(cm) >= 2) {
      // The candidates again, against the margin of the lane m that holds A: QW only stands
      // for |Q_m| in the argument at raised_key, so |qa_m| (1 + 2^-20) >= |Q_m| does too, and
      // is usually far below the chain's bound.  The exact argmax is in both sets, so in their
      // intersection; when that is one lane, it is the pick.
      const float ap = __builtin_fmaf(s, y.ar[0], y.q[0]);
      const int m = lowest_lane(__ballot(fkey(ap) == Akl));
      const float qam = __builtin_fabsf(readlane_f(y.q[0], m));
      const float qwm = __builtin_fmaf(qam, 0x1p-20f, qam);
      cset &= __ballot(raised_key(ap, y.q[0], qwm) >= Akl);
    }
    const int win = __builtin_amdgcn_readfirstlane(
        __popcll(cset) == 1 ? lowest_lane(cset)
                            : exact_pick_lane(y.den[0], y.wv[0], y.cp[0], cset, s, vlf));
    if (WINDOW && win < 0) return rr;  // (no child scores above -1e9: not a window step)
    // (first_end is uniform: said so, so that the ranks stay uniform after this branch)
    if (!WINDOW && win < 0 && __builtin_amdgcn_readfirstlane(*first_end) < 0)
      *first_end = r0 + rr;
    const bool hit = win >= 0 && lane == win;
    y.q[0] = hit ? y.qn[0] : y.q[0];
    y.ar[0] = hit ? y.arn[0] : y.ar[0];
    y.den[0] = hit ? y.den[0] + fvl : y.den[0];
    y.cn[0] = hit ? y.cn[0] + 1 : y.cn[0];
    const int rk = readlane_i(y.cn[0], win & (kWave - 1));
    asm volatile("v_writelane_b32 %0, %1, m0" : "+v"(*rec) : "s"(win), "{m0}"(rr));
    asm volatile("v_writelane_b32 %0, %1, m0" : "+v"(*rnk) : "s"(rk), "{m0}"(rr));
    ++rr;
  }
  return rr;
}

// State of a row of more than 64 children held R slots per lane, for steps over the whole row
// (the steps between contender windows): no next states are kept, a pick recomputes the
// picked child's state.
template <int R>
struct WideRow {
  float q[R], ar[R], den[R], wv[R], cp[R];
};

// One step over the whole row (as in lane_steps); returns j*64 + lane of the pick or -1.
template <int R>
__device__ inline int wide_step(WideRow<R>& x, float s, float fvl, float vlf, float qbt_eff,
                                bool exact_only, int k) {
  const int lane = lane_id();
  float ap[R];
#pragma unroll
  for (int j = 0; j < R; ++j) ap[j] = __builtin_fmaf(s, x.ar[j], x.q[j]);
  float t[R];
#pragma unroll
  for (int j = 0; j < R; ++j) t[j] = ap[j];
#pragma unroll
  for (int w = 1; w < R; w <<= 1)
#pragma unroll
    for (int j = 0; j + w < R; j += 2 * w) t[j] = fmaxf(t[j], t[j + w]);
  const float A = funkey(wave_max_u32(fkey(t[0])));
  const float T = __builtin_fmaf(__builtin_fabsf(A), -1.0f / 524288.0f, A) + qbt_eff;
  uint32_t bits = 0;
  uint64_t cm = 0;
  int tot = 0;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const bool bj = ap[j] >= T;
    const uint64_t mj = __ballot(bj);
    bits |= bj ? (1u << j) : 0u;
    cm |= mj;
    tot += __popcll(mj);
  }
  int win;
  if (tot == 1) {
    const int l = lowest_lane(cm);
    win = (__ffs((unsigned)readlane_i((int)bits, l)) - 1) * kWave + l;
  } else {
    win = exact_pick<R>(x.den, x.wv, x.cp, bits, exact_only || tot == 0, k, s, vlf);
    win = __builtin_amdgcn_readfirstlane(win);
  }
  if (win >= 0) {
    const bool mine = lane == (win & (kWave - 1));
    const int jj = win >> 6;
#pragma unroll
    for (int j = 0; j < R; ++j) {
      if (j == jj) {
        const float d = mine ? x.den[j] + fvl : x.den[j];
        float qv, av;
        child_state(d, x.wv[j], x.cp[j], j * kWave + lane, vlf, &qv, &av);
        x.den[j] = d;
        x.q[j] = mine ? qv : x.q[j];
        x.ar[j] = mine ? av : x.ar[j];
      }
    }
  }
  return win;
}


// A key threshold t with at most 64 of the row's k keys >= t, and at least kTopMin of them
// where the search meets such a t: bisection on the keys between the row's smallest and
// largest key, stopped at the first threshold whose count lies in [kTopMin, 64].  Any
// threshold with at most 64 keys above it makes a valid contender set; the early stop only
// trades a few contenders for fewer bisection steps.  Needs k > 64.
constexpr int kTopMin = 56;

template <int R>
struct RowKeys {
  uint32_t v[R];
};

// number of the row's keys >= t (uniform)
template <int R>
__device__ inline int keys_at_least(const uint32_t* key, int k, uint32_t t) {
  const int lane = lane_id();
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < R; ++j) cnt += __popcll(__ballot(j * kWave + lane < k && key[j] >= t));
  return cnt;
}

// the bisection of [lo, hi), where count(>= lo) > 64 >= count(>= hi)
template <int R>
__device__ inline uint32_t top64_bisect(const uint32_t* key, int k, uint64_t lo, uint64_t hi) {
  while (hi - lo > 1) {
    const uint64_t mid = (lo + hi) >> 1;
    const int cnt = keys_at_least<R>(key, k, (uint32_t)mid);
    if (cnt <= kWave) {
      hi = mid;
      if (cnt >= kTopMin) break;
    } else {
      lo = mid;
    }
  }
  return (uint32_t)hi;
}

// [smallest, largest + 1) of the row's keys: count(>= lo) = k > 64 >= count(>= hi) = 0
template <int R>
__device__ inline void key_range(const uint32_t* key, int k, uint64_t* lo, uint64_t* hi) {
  const int lane = lane_id();
  uint32_t kmax = 0u, kmin = 0xFFFFFFFFu;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    if (j * kWave + lane < k) {
      kmax = max(kmax, key[j]);
      kmin = min(kmin, key[j]);
    }
  }
  *lo = ~wave_max_u32(~kmin);
  *hi = (uint64_t)wave_max_u32(kmax) + 1;
}

template <int R>
__device__ inline uint32_t top64_threshold(const uint32_t* key, int k) {
  uint64_t lo, hi;
  key_range<R>(key, k, &lo, &hi);
  return top64_bisect<R>(key, k, lo, hi);
}

// The same search warm-started from hint, the previous window's threshold in the same chain
// (for the kernels that form a window in every block of ranks).  Consecutive windows have
// nearby thresholds, so the answer is first bracketed around the hint, with steps that double
// from 2^16 keys; the bisection then runs in that bracket.  (Not inlined: its working registers
// are not held across the chain; it runs once per window.)
template <int R>
__device__ __noinline__ uint32_t top64_threshold_near(RowKeys<R> keys, int k, uint32_t hint) {
  const uint32_t* key = keys.v;
  uint64_t lo, hi;
  key_range<R>(key, k, &lo, &hi);
  if (hint > lo && hint < hi) {
    const int ch = keys_at_least<R>(key, k, hint);
    if (ch <= kWave && ch >= kTopMin) return hint;
    uint64_t d = 1u << 16;
    if (ch > kWave) {
      lo = hint;  // upwards: hint + d, + 2d, ... until the count is at most 64
      while (lo + d < hi) {
        const int c2 = keys_at_least<R>(key, k, (uint32_t)(lo + d));
        if (c2 <= kWave) {
          if (c2 >= kTopMin) return (uint32_t)(lo + d);
          hi = lo + d;
          break;
        }
        lo += d;
        d <<= 1;
      }
    } else {
      hi = hint;  // downwards: hint - d, - 2d, ... until the count exceeds 64
      while (hi > lo + d) {
        const int c2 = keys_at_least<R>(key, k, (uint32_t)(hi - d));
        if (c2 > kWave) {
          lo = hi - d;
          break;
        }
        hi -= d;
        if (c2 >= kTopMin) return (uint32_t)hi;
        d <<= 1;
      }
    }
  }
  return top64_bisect<R>(key, k, lo, hi);
}

// With `progress` set, the chain publishes its progress after every block of 64 ranks: the
// block's picks are in ch first (workgroup-scope release), then *progress = ranks done.  With
// `stop` set, the chain ends after the first block that finds *stop non-zero (its picks up to
// the last published rank are in ch; its counts in cnt_s are then not kept).
// PARTIAL: ranks [0, npre) were taken before the chain (by the first-unvisited prefix,
// unvisited_prefix, or by a chain run ahead), with their picks in ch and their counts per
// child in cnt_s; the chain starts at rank npre.  Else npre is 0 and cnt_s is cleared here.
// What a chain reads of the forest and the configuration, passed by value: a chain the
// compiler keeps out of line then takes them in registers (a reference to the kernel's SelArgs
// would make every lane store a copy of the whole argument block in its private memory).
struct ChainRows {
  const int32_t* N;
  const float* W;
  const float* P;
};
struct ChainCfg {
  float c_puct;
  float vlf;
  int vli;
};

template <int R, bool PERSIST, bool PARTIAL>
__device__ int run_chain(ChainRows f, int64_t tb, int first, int k, int Np0, int m, int npre,
                         ChainCfg c, uint32_t* ch, uint16_t* cnt_s, float4* cscr,
                         int* progress, const int* stop) {
  const int lane = lane_id();
  const float vlf = c.vlf;
  const float fvl = (float)c.vli;
  // R == 1 keeps next states (Row<1>); wider rows keep the wide state between windows
  Row<1> y;
  WideRow<R> x;
  float qbl = 0.0f;
  bool negcp = false;
  int pre0 = 0;  // (R == 1) the lane's child was taken by the prefix
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int i = j * kWave + lane;
    if (!PARTIAL && i < k) cnt_s[i] = 0;
    float d = 2.0f, w = 0.0f, cpv = 0.0f, qv = -__builtin_inff(), av = 0.0f;
    if (i < k) {
      const int64_t node = tb + first + 1 + i;  // child of edge first+i is node first+i+1
      const int n = f.N[node];
      w = f.W[node];
      cpv = c.c_puct * f.P[node];
      d = (float)(1 + n);
      if (PARTIAL) {
        const int pre = cnt_s[i];  // picks before the chain: a virtual loss each
        d = d + fvl * (float)pre;  // (exact: integers below 2^24)
        if (j == 0) pre0 = pre;
      }
      negcp = negcp || !(cpv >= 0.0f);
      if (child_state(d, w, cpv, i, vlf, &qv, &av)) qbl = fmaxf(qbl, __builtin_fabsf(qv));
    }
    x.den[j] = d;
    x.wv[j] = w;
    x.cp[j] = cpv;
    x.q[j] = qv;
    x.ar[j] = av;
  }
  const uint32_t QBb = wave_max_rows(__float_as_uint(qbl));  // bits of QB (non-negative)
  const float qbt = __uint_as_float(QBb) * (-1.0f / 524288.0f);
  const float qb = __uint_as_float(QBb);  // QB
  const bool exact_only = __ballot(negcp) != 0 || !(__uint_as_float(QBb) < 1e8f);
  if (c.vli == 0) {
    // Without an integer virtual loss a pick changes no visit count: every rank sees the same
    // row and the same parent count, so every rank takes the first rank's choice.
    int win = -1;
    if (Np0 != 0) {  // Np = 0: sqrt(0) exploration, the reference returns no child
      win = exact_pick<R>(x.den, x.wv, x.cp, 0u, true, k, sqrtf((float)Np0), vlf);
      win = __builtin_amdgcn_readfirstlane(win);
    }
    for (int r = lane; r < m; r += kWave)
      ch[r] = win >= 0 ? (((uint32_t)win << 16) | (uint32_t)r) : kNoChild;
    if (lane == 0 && win >= 0) cnt_s[win] = (uint16_t)m;
    wave_sync();
    return (win < 0 && m > 0) ? 0 : -1;
  }
  if (R == 1) {
    y.den[0] = x.den[0];
    y.wv[0] = x.wv[0];
    y.cp[0] = x.cp[0];
    y.q[0] = lane < k ? x.q[0] : kPadQ;  // (padding lanes: see lane_steps)
    y.ar[0] = x.ar[0];
    y.cn[0] = pre0;
    if (lane < k) {
      child_state(y.den[0] + fvl, y.wv[0], y.cp[0], lane, vlf, &y.qn[0], &y.arn[0]);
    } else {
      y.qn[0] = kPadQ;
      y.arn[0] = 0.0f;
    }
  }
  int first_end = -1;
  // a NaN threshold sends every step to the exact comparison
  const float qbt_eff = exact_only ? __builtin_nanf("") : qbt;
  // A contender window stays open across blocks of ranks while its bound holds: its contenders
  // in y (row index cidx, ncon of them) and, per lane, the slots of x that are contenders (bit
  // j: slot j).  The contenders' slots of x are stale while it is open.
  bool wopen = false;
  int ncon = 0, cidx = 0;
  uint32_t tau_hint = 0u;  // the last window's contender threshold (0: none yet)
  uint32_t conbits = 0u;
  // Bound of the non-contenders' raised keys at rank s_end (a NaN ap is never a pick, and not
  // a candidate of the window's steps).  QB bounds |qa| of every visited child, the window's
  // contenders (the lanes that can hold a window step's maximum) among them.
  auto noncon_bound = [&](float s_end) {
    uint32_t ubk = kKeyFloor;
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int i = j * kWave + lane;
      const bool con = ((conbits >> j) & 1u) != 0;
      const float a = __builtin_fmaf(s_end, x.ar[j], x.q[j]);
      const uint32_t ha = raised_key(a, x.q[j], qb);
      ubk = (i < k && !con && a == a) ? max(ubk, ha) : ubk;
    }
    return wave_max_u32(ubk);
  };
  // Closes the window: the contenders' counts go back to cnt_s and their states to x (every
  // state follows from its count).
  auto close_window = [&]() {
    wave_sync();
    if (lane < ncon) {
      cscr[lane].x = y.den[0];
      cnt_s[cidx] = (uint16_t)y.cn[0];
    }
    wave_sync();
    int base = 0;
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int i = j * kWave + lane;
      const bool con = ((conbits >> j) & 1u) != 0;
      const uint64_t cm = __ballot(con);
      const int dest = base + (int)__builtin_amdgcn_mbcnt_hi(
                                  (uint32_t)(cm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)cm, 0u));
      if (con) x.den[j] = cscr[dest].x;
      if (i < k) child_state(x.den[j], x.wv[j], x.cp[j], i, vlf, &x.q[j], &x.ar[j]);
      base += __popcll(cm);
    }
    wave_sync();
    conbits = 0u;
    wopen = false;
  };
  for (int r0 = PARTIAL ? (npre / kWave) * kWave : 0; r0 < m; r0 += kWave) {
    const int Npl = Np0 + c.vli * (r0 + lane + 1);
    const float svec = sqrtf((float)Npl);
    const int rend = __builtin_amdgcn_readfirstlane(min(kWave, m - r0));
    // the block's ranks taken by the prefix (npre is uniform: a call's result is not known
    // to be, so it is made so here)
    const int rs = PARTIAL ? __builtin_amdgcn_readfirstlane(max(0, npre - r0)) : 0;
    // lane rr of rec / rnk: the child picked at rank r0+rr and the chain's picks of that child
    // up to and including it (the picked lane's count after the pick: its rank plus one)
    uint32_t rec = kNoChild;
    uint32_t rnk = 0;
    // Window steps from rank rr of the block on.  A step is the window's while its maximum
    // key exceeds every non-contender's raised key at that step; those keys only grow with s,
    // so a bound taken at a later rank holds for every rank before it.  The bound is taken
    // at the end of a segment of ranks and renewed for the next segment while the window
    // holds.  Where the block raises the parent count by 1/16 or more (s grows 3 % or more
    // over it), a bound at the block's end ends windows early, so the segments are 32 ranks
    // there; elsewhere one bound per block costs less (C2 select 68.0 -> 62.4 us, C3
    // 232.5 -> 225.3 us, against 64-rank segments everywhere; 16- and 8-rank segments
    // measured slower).
    const int npb = Np0 + c.vli * r0;  // the parent count at the block's first rank
    const int seg = npb >= 16 * kWave * c.vli ? kWave : kWave / 2;
    auto window_steps = [&](int rr) {
      while (rr < rend) {
        const int se = __builtin_amdgcn_readfirstlane(min(rend, rr + seg));
        const uint32_t ubk = noncon_bound(readlane_f(svec, se - 1));
        rr = lane_steps<true>(y, svec, rr, se, fvl, vlf, qb, ubk, kKeyInf, ncon, r0,
                              &first_end, &rec, &rnk);
        if (rr < se) break;
      }
      return rr;
    };
    if (R == 1) {
      lane_steps<false>(y, svec, rs, rend, fvl, vlf, qb, kKeyFloor, exact_only ? 0u : kKeyInf,
                        k, r0, &first_end, &rec, &rnk);
    } else {
      int rr = rs;
      bool try_window = !exact_only;
      if (PERSIST && wopen) {
        // ---- the open window continues ----
        rr = window_steps(0);
        const int ci = __shfl(cidx, (int)(rec & 63u), 64);
        if (lane < rr) rec = (uint32_t)ci;
        if (rr < rend) close_window();  // (a fresh window may follow in this block)
      }
      while (rr < rend) {
        if (try_window && rend - rr >= 8) {
          // ---- contender window: the top 64 children by ap 128 ranks past its first rank ----
          // (any 64 children make a valid window: the bound decides each step.  Ranking them at
          // a larger parent count keeps the children whose exploration term grows fastest, which
          // keeps windows open longer: C3 select 201 -> 198 us, C2 61.4 -> 60.2 us; ranked at
          // 32, 64, 256 and 512 ranks ahead: 198.3, 198.0, 200-202 and 202 us)
          const float s0 = sqrtf((float)(Np0 + c.vli * (r0 + rr + 1 + 2 * kWave)));
          RowKeys<R> keys;
          uint32_t* key = keys.v;
#pragma unroll
          for (int j = 0; j < R; ++j) key[j] = fkey(__builtin_fmaf(s0, x.ar[j], x.q[j]));
          // (windows that stay open over rows of at most 4 slots: the plain search; over wider
          // rows the warm start pays: C3 select 245.7 -> 242.8 us, C2 67.9 -> 69.9 us with it)
          const uint32_t tau = (PERSIST && R <= 4)
                                   ? top64_threshold<R>(key, k)
                                   : top64_threshold_near<R>(keys, k, tau_hint);
          tau_hint = tau;
          int base = 0;
#pragma unroll
          for (int j = 0; j < R; ++j) {
            const int i = j * kWave + lane;
            const bool con = i < k && key[j] >= tau;
            const uint64_t cm = __ballot(con);
            const int dest = base + (int)__builtin_amdgcn_mbcnt_hi(
                                        (uint32_t)(cm >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)cm, 0u));
            if (con) cscr[dest] = make_float4(x.den[j], x.wv[j], x.cp[j], __int_as_float(i));
            conbits |= con ? (1u << j) : 0u;
            base += __popcll(cm);
          }
          ncon = base;
          wave_sync();
          const float4 e = lane < ncon ? cscr[lane] : make_float4(2.0f, 0.0f, 0.0f, 0.0f);
          cidx = __float_as_int(e.w);
          y.den[0] = e.x;
          y.wv[0] = e.y;
          y.cp[0] = e.z;
          y.cn[0] = lane < ncon ? (int)cnt_s[cidx] : 0;
          if (lane < ncon) {
            child_state(y.den[0], y.wv[0], y.cp[0], cidx, vlf, &y.q[0], &y.ar[0]);
            child_state(y.den[0] + fvl, y.wv[0], y.cp[0], cidx, vlf, &y.qn[0], &y.arn[0]);
          } else {
            y.q[0] = y.qn[0] = kPadQ;
            y.ar[0] = y.arn[0] = 0.0f;
          }
          wopen = true;
          const int rr0 = rr;
          // window steps record the picked lane; the lanes become child indices below.  A
          // window step always picks (no candidate or an unsafe threshold aborts it first).
          rr = window_steps(rr);
          {
            const int ci = __shfl(cidx, (int)(rec & 63u), 64);
            if (lane >= rr0 && lane < rr) rec = (uint32_t)ci;
          }
          if (rr < rend || !PERSIST) {  // (else the window stays open into the next block)
            close_window();
            if (rr - rr0 < 8) try_window = false;  // no more windows in this block
          }
          continue;
        }
        // ---- one step over the whole row ----
        const float s = readlane_f(svec, rr);
        const int win = wide_step<R>(x, s, fvl, vlf, qbt_eff, exact_only, k);
        if (win < 0 && __builtin_amdgcn_readfirstlane(first_end) < 0) first_end = r0 + rr;
        int rk = 0;
        if (win >= 0) {
          rk = cnt_s[win];
          wave_sync();
          if (lane == 0) cnt_s[win] = (uint16_t)(rk + 1);
          wave_sync();
        }
        rec = (lane == rr) ? (uint32_t)win : rec;
        rnk = (lane == rr) ? (uint32_t)(rk + 1) : rnk;
        ++rr;
      }
    }
    if (lane >= rs && lane < rend)
      ch[r0 + lane] = rec != kNoChild ? ((rec << 16) | (rnk - 1u)) : kNoChild;
    if (progress != nullptr) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      if (lane == 0)
        __hip_atomic_store(progress, r0 + rend, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (stop != nullptr &&
        __builtin_amdgcn_readfirstlane(
            __hip_atomic_load(stop, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) != 0)
      break;
  }
  if (R > 1 && PERSIST && wopen) close_window();
  // the chain's pick counts per child (R == 1 keeps them in the lanes until here)
  if (R == 1 && lane < k) cnt_s[lane] = (uint16_t)y.cn[0];
  wave_sync();
  return first_end;
}

// First-unvisited prefix of a chain.  The reference takes the first unvisited child of a row
// whenever one is left (CythonLockFreeTree.select_best_child_nogil returns at the first child
// with no visits, cython_tree_optimized.pyx:451-452), and a pick makes its child visited (an
// integer virtual loss >= 1).  So while unvisited children remain, rank r of the chain takes
// the r-th of them in index order: the first npre = min(m, unvisited children) ranks are
// decided from the children's visit counts alone.  Writes their picks to ch[0, npre) (each
// child once: rank 0 among its picks) and every child's prefix count (0 or 1) to cnt_s[0, k),
// which the chain starts from; returns npre.  (off: no virtual loss; nothing is taken.)
template <int RMAX>
__device__ __noinline__ int unvisited_prefix(const int32_t* N, int64_t tb, int first, int k, int m,
                                             bool on, uint32_t* ch, uint16_t* cnt_s) {
  const int lane = lane_id();
  int n[RMAX];
#pragma unroll
  for (int j = 0; j < RMAX; ++j) {
    const int i = j * kWave + lane;
    n[j] = 1;
    if (on && i < k) n[j] = N[tb + first + 1 + i];
  }
  int npre = 0;
#pragma unroll
  for (int j = 0; j < RMAX; ++j) {
    const int i = j * kWave + lane;
    const bool u = i < k && n[j] == 0;
    const uint64_t um = __ballot(u);
    const int pos = npre + (int)__builtin_amdgcn_mbcnt_hi(
                               (uint32_t)(um >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)um, 0u));
    const bool pick = u && pos < m;
    if (pick) ch[pos] = (uint32_t)i << 16;
    if (i < k) cnt_s[i] = pick ? 1 : 0;
    npre += __popcll(um);
  }
  wave_sync();
  return min(npre, m);
}

// Chain of a row of k children, instantiated up to RMAX slots per lane (rows of at most
// 64*RMAX children): a kernel holds only the widths its game model can produce, which keeps
// its register demand within the 128 VGPRs of a 1024-thread workgroup.  WIDE: the kernel's
// chains keep up to 256 registers (workgroups of at most 512 threads, one per CU).
template <int RMAX, bool WIDE>
__device__ inline int dispatch_chain(ChainRows rows, int64_t tb, int first, int k, int Np0,
                                     int m, int npre, ChainCfg cc, uint32_t* ch, uint16_t* cnt_s,
                                     float4* cscr, int* progress, const int* stop = nullptr) {
  const int r = (k + kWave - 1) / kWave;  // 1 <= r <= RMAX (checked by the caller)
  // contender windows kept open across blocks in the kernels of up to 4 slots per lane and in
  // the WIDE ones (the other wider kernels' chains have no registers left for it)
  constexpr bool kPersist = RMAX <= 4 || WIDE;
  if (RMAX <= 1 || r <= 1)
    return run_chain<1, kPersist, WIDE>(rows, tb, first, k, Np0, m, npre, cc, ch, cnt_s, cscr, progress, stop);
  if (RMAX >= 2 && r == 2)
    return run_chain<(RMAX >= 2 ? 2 : 1), kPersist, WIDE>(rows, tb, first, k, Np0, m, npre, cc, ch, cnt_s, cscr, progress, stop);
  if (RMAX >= 3 && r == 3)
    return run_chain<(RMAX >= 3 ? 3 : 1), kPersist, WIDE>(rows, tb, first, k, Np0, m, npre, cc, ch, cnt_s, cscr, progress, stop);
  if (RMAX >= 4 && r == 4)
    return run_chain<(RMAX >= 4 ? 4 : 1), kPersist, WIDE>(rows, tb, first, k, Np0, m, npre, cc, ch, cnt_s, cscr, progress, stop);
  if (RMAX >= 5 && r == 5)
    return run_chain<(RMAX >= 5 ? 5 : 1), kPersist, WIDE>(rows, tb, first, k, Np0, m, npre, cc, ch, cnt_s, cscr, progress, stop);
  if (RMAX >= 6 && r == 6)
    return run_chain<(RMAX >= 6 ? 6 : 1), kPersist, WIDE>(rows, tb, first, k, Np0, m, npre, cc, ch, cnt_s, cscr, progress, stop);
  return run_chain<(RMAX >= 8 ? 8 : 1), kPersist, WIDE>(rows, tb, first, k, Np0, m, npre, cc, ch, cnt_s, cscr, progress, stop);
}

// A group's chain: the first-unvisited prefix, and the chain when the prefix does not take
// every rank.  The WIDE kernels' chains start after the prefix; the others derive its ranks
// again (starting after them cost the 1024-thread chains up to 60 spilled registers).
// *all_prefix: every rank was taken by the prefix (distinct children in index order, each
// picked once).  taken > 0 (WIDE): ranks [0, taken) are already in ch and their counts in
// cnt_s (replayed from a chain run ahead, which went past the prefix); the chain goes on from
// there.
template <int RMAX, bool WIDE>
__device__ inline int group_chain(ChainRows rows, int64_t tb, int first, int k, int Np0, int m,
                                  ChainCfg cc, uint32_t* ch, uint16_t* cnt_s, float4* cscr,
                                  int* progress, bool* all_prefix, int* npre_out = nullptr,
                                  const int* stop = nullptr, int taken = 0) {
  if (WIDE && taken > 0) {
    *all_prefix = false;
    return dispatch_chain<RMAX, WIDE>(rows, tb, first, k, Np0, m, taken, cc, ch, cnt_s, cscr,
                                      progress, stop);
  }
  const int npre = unvisited_prefix<RMAX>(rows.N, tb, first, k, m, cc.vli > 0, ch, cnt_s);
  *all_prefix = npre >= m;
  if (npre_out != nullptr) *npre_out = npre;
  if (npre >= m) {
    if (progress != nullptr) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      if (lane_id() == 0)
        __hip_atomic_store(progress, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    return -1;
  }
  // (the WIDE kernels' chains start after the prefix; the others derive its ranks again)
  if (WIDE && npre > 0 && progress != nullptr) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane_id() == 0)
      __hip_atomic_store(progress, npre, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  return dispatch_chain<RMAX, WIDE>(rows, tb, first, k, Np0, m, WIDE ? npre : 0, cc, ch, cnt_s,
                                    cscr, progress, stop);
}

// Block-wide exclusive scan of a[0..n) in place (n <= 4 * NT); returns the total.  a may be
// LDS or global memory (each thread touches its own chunk only).
template <int NT>
__device__ int block_excl_scan(int32_t* a, int n, int* s_wtot) {
  constexpr int NW = NT / kWave;
  const int tid = threadIdx.x;
  const int per = (n + NT - 1) / NT;
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
  for (int i = 0; i < NW; ++i) {
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

// ---- State of the level loop -----------------------------------------------------------
// Dynamic LDS (sized for W, the simulations of the wave; a group's members occupy a segment
// [seg, seg + m) of [0, W) at every level, so the arrays are indexed by absolute positions):
//   cscr_all [NW * 64] float4   contender window scratch, per wave
//   choice   [W]       uint32   chain output per member position
//   gnode    [2W]      uint32   group node, per level parity
//   gsl      [2W]      uint32   group seg | len << 16, per level parity
//   buf      [2W]      uint16   members by position, per level parity
//   cnt_all  [NW * OMQ_MAX_ROW] uint16   child pick counts of each wave's chain
//   pipe_ch  [NW * 64] uint32   (level overlap) the followers' chain output
//   pick2    [W]       uint16   (level overlap) level-1 picks recorded by the followers
struct LevelLds {
  float4* cscr_all;
  uint32_t* choice;
  uint32_t* gnode;
  uint32_t* gsl;
  uint16_t* buf;
  uint16_t* cnt_all;
  uint32_t* pipe_ch;
  uint16_t* pick2;
  uint32_t* spec;  // [kSpecSlots][W] level-1 chains run ahead by the followers (wide kernels)
};

template <int NT>
__host__ __device__ inline size_t level_base_bytes(int W) {
  // cscr_all, then 24 B per simulation (choice 4, gnode 8, gsl 8, buf 4), then cnt_all
  return (size_t)(NT / kWave) * kWave * 16 + (size_t)W * 24 +
         (size_t)(NT / kWave) * OMQ_MAX_ROW * 2;
}
template <int NT>
__host__ __device__ inline size_t level_pipe_offset(int W) {
  return (level_base_bytes<NT>(W) + 15) & ~(size_t)15;
}
constexpr int kPipeMaxW = 2048;  // waves with LDS for the overlap buffers
// Level-1 chains run ahead during the root chain, one per wave other than the root chain's
// (the wide kernels: 8 waves), for waves of at most kPipeMaxW simulations.
constexpr int kSpecSlots = 7;
template <int NT>
__host__ __device__ inline size_t level_lds_bytes(int W, bool with_pipe) {
  if (W > kPipeMaxW) return level_base_bytes<NT>(W);
  if (!with_pipe) return level_pipe_offset<NT>(W) + (size_t)kSpecSlots * W * 4;
  return level_pipe_offset<NT>(W) + (size_t)(NT / kWave) * kWave * 4 + (size_t)W * 2;
}

template <int NT>
__device__ inline LevelLds carve_level_lds(unsigned char* smem, int W, bool with_pipe) {
  constexpr int NW = NT / kWave;
  LevelLds L;
  L.cscr_all = reinterpret_cast<float4*>(smem);
  L.choice = reinterpret_cast<uint32_t*>(L.cscr_all + NW * kWave);
  L.gnode = L.choice + W;
  L.gsl = L.gnode + 2 * W;
  L.buf = reinterpret_cast<uint16_t*>(L.gsl + 2 * W);
  L.cnt_all = L.buf + 2 * W;
  L.pipe_ch = nullptr;
  L.pick2 = nullptr;
  L.spec = nullptr;
  if (with_pipe && W <= kPipeMaxW) {
    L.pipe_ch = reinterpret_cast<uint32_t*>(smem + level_pipe_offset<NT>(W));
    L.pick2 = reinterpret_cast<uint16_t*>(L.pipe_ch + NW * kWave);
  }
  if (!with_pipe && W <= kPipeMaxW && NW == kSpecSlots + 1)
    L.spec = reinterpret_cast<uint32_t*>(smem + level_pipe_offset<NT>(W));
  return L;
}

// Static LDS of the level loop.
template <int NT>
struct LevelShared {
  int nbig[2];    // groups of a level a wave runs as a chain: [0, nbig)
  int nsmall[2];  // (kernels that keep single-member groups apart) those at [W - nsmall, W)
  int next[2];    // next chain group to take at the level (dynamic deal)
  int snext;      // next chunk of the lane pass's groups
  int kept;       // single-member groups of the leaf pass that become chains
  int progress;   // ranks of the root chain published to the followers
  int gbase;      // the level's first group-log entry (allocated once per level)
  int gnext;      // next group-log entry of the level, from gbase
  int hist[16];
  int wtot[NT / kWave];
  int spec_node[8];  // the root child of each run-ahead chain (-1: none)
  int spec_m[8];     // its ranks done
  int spec_npre[8];  // its first-unvisited prefix
  int root_done;     // the root chain is done (the run-ahead chains end)
  unsigned long long st[OMQ_NSTATS];
};

// Groups of at most SelTraits<RMAX>::kSmall members at level d, one group per lane.  Each
// member in turn takes the reference's best child (first unvisited child, else the strict
// argmax of the exact score) at the parent count N + VL*(rank+1), the children picked by
// earlier members carrying their virtual loss; the lane scans the row in order, exactly as
// CythonLockFreeTree.select_best_child_nogil does.  The members of each picked child are
// placed in the parent's segment, children in order of their first pick, members in rank
// order.
constexpr int kLaneGroup = 2;

// Kernels of at least this many slots per lane run 512-thread workgroups (select_threads).
// (The 3-slot kernel at 1024 threads, with the level-1 followers, spilled 62 registers; at 512
// threads it spills none, and a Go 13 x 13 wave's select went 182 -> 170 us.)
constexpr int kWideRmax = 3;

// Single-member groups are kept apart from the chain groups in the kernels with a lane pass
// (rows of at most 192 children) or a leaf pass (256 and 384); the 8-slot kernel keeps every
// group a chain (the passes' registers would add spills to its chains).
template <int RMAX>
struct SelTraits {
  static constexpr bool kLanePass = RMAX <= 3;
  static constexpr bool kLeafPass = RMAX == 4 || RMAX == 6;
  static constexpr bool kSingles = kLanePass || kLeafPass;
  // single-member groups at internal nodes that the leaf pass keeps go through the lane pass
  // (instead of becoming chains) in the 4-slot kernels; the 6- and 8-slot kernels' chains have
  // no registers left for it.  (Measured: no change on C2, whose such groups are leaves.)
  static constexpr bool kWideLanePass = RMAX == 4;
  // members of the groups that the lane pass takes (one group per lane): up to kLaneGroup in
  // the 1- and 2-slot kernels (C4 select 514 -> 506 us with 2 members, 510 with 4, 565 with 8;
  // the 3-slot kernel spills with them), single members elsewhere (the leaf pass takes single
  // members only)
  static constexpr int kSmall = RMAX <= 2 ? kLaneGroup : 1;
  // children whose loads a lane of the lane pass has in flight at a time: as many as the
  // kernel has registers for without spilling (the 3-slot kernel spills already; the 4-slot
  // kernel's 225-child rows: C5 select 47.4 -> 46.3 us with 16, 47.8 with 32)
  static constexpr int kLaneRound = RMAX <= 2 ? 8 : RMAX == 4 ? 16 : 4;
  // small groups decided by the first-unvisited rule one per thread (prefix_pass) in the
  // kernels of 512 threads, whose chains have registers to spare for it
  static constexpr bool kPrefixPass = RMAX >= kWideRmax;
};


template <int RMAX, int NT>
__device__ inline void small_groups_body(const SelArgs& f, const SelCfg& c, int t, int d, int W,
                                         int64_t tb, int64_t gmax, const LevelLds& L,
                                         LevelShared<NT>& sh, int32_t* lfs, int32_t* lflag,
                                         bool vl_done) {
  constexpr int kSmallGroup = SelTraits<RMAX>::kSmall;
  constexpr int kLaneRound = SelTraits<RMAX>::kLaneRound;
  const SelArgs& w = f;
  const int cur = d & 1, nxt = cur ^ 1;
  const int MW = w.max_wave, MD = w.max_depth_buf;
  int32_t* N = f.N;
  uint32_t* gnode = L.gnode;
  uint32_t* gsl = L.gsl;
  uint16_t* buf = L.buf;
  // the small groups of the level sit at the top of the group arrays: [W - ns, W); chunks of 64
  // are dealt from an LDS counter, so that waves done with their chains take them first.  Every
  // fetch advances the counter, so the loop ends after at most ns/64 + 1 fetches.
  const int lane = lane_id();
  const int ns = sh.nsmall[cur];
  for (int it = 0; it <= ns / kWave; ++it) {
    int g0 = 0;
    if (lane == 0) g0 = atomicAdd(&sh.snext, kWave);
    g0 = readlane_i(g0, 0);
    if (g0 >= ns) break;
    const int gi = W - 1 - (g0 + lane);
    const uint32_t sl = g0 + lane < ns ? gsl[cur * W + gi] : 0u;
    const int m0 = (int)(sl >> 16);
    const bool valid = m0 >= 1 && m0 <= kSmallGroup;
    const int m = valid ? m0 : 0;
    // group-log ids and statistics per wave (one LDS atomic each, not one per lane)
    const uint64_t vm = __ballot(valid);
    if (vm == 0) continue;
    int gbase = 0;
    if (lane == 0) gbase = sh.gbase + atomicAdd(&sh.gnext, __popcll(vm));
    gbase = readlane_i(gbase, 0);
    int p = 0, seg = 0, Np0 = 0, k = 0, first = 0;
    int mem[kSmallGroup];
#pragma unroll
    for (int r = 0; r < kSmallGroup; ++r) mem[r] = 0;
    bool leaf = true;
    if (valid) {
      p = (int)gnode[cur * W + gi];
      seg = (int)(sl & 0xFFFFu);
#pragma unroll
      for (int r = 0; r < kSmallGroup; ++r) mem[r] = r < m ? (int)buf[cur * W + seg + r] : 0;
      const int gid = gbase + (int)__builtin_amdgcn_mbcnt_hi(
                                  (uint32_t)(vm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)vm, 0u));
      *reinterpret_cast<int4*>(w.glog + ((int64_t)t * gmax + gid) * 4) = make_int4(p, d, seg, m);
#pragma unroll
      for (int r = 0; r < kSmallGroup; ++r) {
        if (r < m) {
          w.paths[((int64_t)t * MW + mem[r]) * MD + d] = p;
          w.gmembers[((int64_t)t * MD + d) * MW + seg + r] = (uint16_t)mem[r];
        }
      }
      Np0 = N[tb + p];
      k = f.nchild[tb + p];
      first = f.first[tb + p];
      if (vl_done)
        Np0 -= c.vli * m;  // the members' virtual loss is in N already
      else if (c.vl_atomic)
        atomicAdd(&N[tb + p], c.vli * m);
      else
        N[tb + p] = Np0 + c.vli * m;
      leaf = (k <= 0) || (first < 0) || (d == c.max_depth - 1);
      if (!leaf && k > RMAX * kWave) {
        atomicOr(&w.status[0], OMQ_STATUS_ROWLIMIT);
        leaf = true;
      }
    }
    {
      const bool inner = valid && !leaf;
      const int ninner = __popcll(__ballot(inner));
      const int rows = wave_sum_i(inner ? k : 0);
      const int steps = wave_sum_i(inner ? m : 0);
      if (lane == 0) {
        atomicAdd(&sh.st[OMQ_ST_PATHNODES], (unsigned long long)__popcll(vm));
        if (ninner > 0) {
          atomicAdd(&sh.st[OMQ_ST_INTERNAL], (unsigned long long)ninner);
          atomicAdd(&sh.st[OMQ_ST_ROWSUM], (unsigned long long)rows);
          atomicAdd(&sh.st[OMQ_ST_STEPS], (unsigned long long)steps);
        }
      }
    }
    int pick[kSmallGroup];
#pragma unroll
    for (int r = 0; r < kSmallGroup; ++r) pick[r] = -1;
    if (valid && !leaf) {
#pragma unroll
      for (int r = 0; r < kSmallGroup; ++r) {
        if (r >= m) break;
        const int Np = Np0 + c.vli * (r + 1);
        if (Np == 0) continue;  // the reference returns no child for a parent count of 0
        const float sp = sqrtf((float)Np);
        float best = -1e9f;
        int bi = -1, unv = -1;
        // the row in order, kLaneRound children's loads in flight at a time; the first
        // unvisited child ends the scan (it is the reference's pick)
        const int64_t row = tb + first + 1;
        for (int i0 = 0; i0 < k && unv < 0; i0 += kLaneRound) {
          int n4[kLaneRound];
          float w4[kLaneRound], p4[kLaneRound];
#pragma unroll
          for (int j = 0; j < kLaneRound; ++j) {
            const bool in = i0 + j < k;
            n4[j] = in ? N[row + i0 + j] : 1;
            w4[j] = in ? f.W[row + i0 + j] : 0.0f;
            p4[j] = in ? f.P[row + i0 + j] : 0.0f;
          }
#pragma unroll
          for (int j = 0; j < kLaneRound; ++j) {
            const int i = i0 + j;
            int n = n4[j];
#pragma unroll
            for (int r2 = 0; r2 < kSmallGroup - 1; ++r2)
              if (r2 < r && pick[r2] == i) n += c.vli;
            if (i < k && unv < 0) {
              if (n == 0) {
                unv = i;
              } else {
                const float q = w4[j] / ((float)n + c.vlf);
                const float u = ((c.c_puct * p4[j]) * sp) / (float)(1 + n);
                const float sc = q + u;
                if (sc > best) {
                  best = sc;
                  bi = i;
                }
              }
            }
          }
        }
        pick[r] = unv >= 0 ? unv : bi;
        if (pick[r] < 0) atomicOr(&w.status[0], OMQ_STATUS_NOCHILD);
      }
    }
    // the next level's groups (each distinct child: at most kSmallGroup members, a small
    // group) and the members whose path ends here, counted per wave
    int ndist = 0, nend = 0;
#pragma unroll
    for (int r = 0; r < kSmallGroup; ++r) {
      if (r >= m) break;
      if (pick[r] < 0) {
        ++nend;
        continue;
      }
      bool seen = false;
#pragma unroll
      for (int r2 = 0; r2 < kSmallGroup - 1; ++r2)
        if (r2 < r && pick[r2] == pick[r]) seen = true;
      ndist += seen ? 0 : 1;
    }
    int dtot;
    int sbase = wave_excl_scan(ndist, &dtot);
    const int ends = wave_sum_i(nend);
    {
      int sb = 0;
      if (lane == 0) {
        if (dtot > 0) sb = atomicAdd(&sh.nsmall[nxt], dtot);
        if (ends > 0) atomicAdd(&sh.st[OMQ_ST_PATHENTRIES], (unsigned long long)ends * (d + 1));
      }
      sbase += readlane_i(sb, 0);
    }
    if (!valid) continue;
    // children in order of first pick; members of a child contiguous, in rank order
    int pos = seg;
    int s_end = -1;
#pragma unroll
    for (int r = 0; r < kSmallGroup; ++r) {
      if (r >= m) break;
      if (pick[r] < 0) {
        if (s_end < 0) s_end = mem[r];
        w.path_len[(int64_t)t * MW + mem[r]] = d + 1;
        w.leaves[(int64_t)t * MW + mem[r]] = p;
        lfs[mem[r]] = s_end;
        continue;
      }
      bool seen = false;
#pragma unroll
      for (int r2 = 0; r2 < kSmallGroup - 1; ++r2)
        if (r2 < r && pick[r2] == pick[r]) seen = true;
      if (seen) continue;
      int cntc = 0;
#pragma unroll
      for (int r2 = 0; r2 < kSmallGroup; ++r2) {
        if (r2 < m && pick[r2] == pick[r]) {
          buf[nxt * W + pos + cntc] = (uint16_t)mem[r2];
          ++cntc;
        }
      }
      const int g = W - 1 - sbase++;  // (cntc <= m <= kSmallGroup: a small group)
      gnode[nxt * W + g] = (uint32_t)(first + 1 + pick[r]);
      gsl[nxt * W + g] = (uint32_t)pos | ((uint32_t)cntc << 16);
      pos += cntc;
    }
    if (s_end >= 0) lflag[s_end] = 1;
  }
}

// The lane pass: the narrow kernels take every single-member group through it, the 4-slot
// kernels those the leaf pass finds at internal nodes.
template <int RMAX, int NT>
__device__ inline void small_groups(const SelArgs& f, const SelCfg& c, int t, int d, int W,
                                    int64_t tb, int64_t gmax, const LevelLds& L,
                                    LevelShared<NT>& sh, int32_t* lfs, int32_t* lflag,
                                    bool vl_done) {
  small_groups_body<RMAX, NT>(f, c, t, d, W, tb, gmax, L, sh, lfs, lflag, vl_done);
}
template <int RMAX, int NT>
__device__ inline void small_groups_call(const SelArgs& f, const SelCfg& c, int t, int d,
                                               int W, int64_t tb, int64_t gmax,
                                               const LevelLds& L, LevelShared<NT>& sh,
                                               int32_t* lfs, int32_t* lflag, bool vl_done) {
  small_groups_body<RMAX, NT>(f, c, t, d, W, tb, gmax, L, sh, lfs, lflag, vl_done);
}

// Single-member groups of level d in the kernels without a lane pass.  Such a group's node is
// usually a leaf, which needs only the node's header (visit count, row offset, row length):
// every thread takes one group per chunk of NT, so the header loads of a chunk are in flight
// together, and the leaves are finished here as the chain groups finish theirs.  The groups
// that are not leaves are staged in the next level's group arrays (empty at this point) and,
// once every single-member group has been read, appended to the level's chain groups (which
// may overwrite the single-member entries, all read by then).  Called by every thread of the
// workgroup.
template <int RMAX, int NT>
__device__ inline void leaf_pass(const SelArgs& f, const SelCfg& c, int t, int d, int W,
                                 int64_t tb, int64_t gmax, const LevelLds& L,
                                 LevelShared<NT>& sh, int32_t* lfs, int32_t* lflag, int ns,
                                 bool vl_done) {
  const SelArgs& w = f;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int cur = d & 1, nxt = cur ^ 1;
  const int MW = w.max_wave, MD = w.max_depth_buf;
  int32_t* N = f.N;
  if (tid == 0) sh.kept = 0;
  __syncthreads();
  for (int c0 = 0; c0 < ns; c0 += NT) {
    bool keep = false, leaf = false;
    uint32_t sl = 0;
    int p = 0, seg = 0, s = 0, Np0 = 0;
    if (c0 + tid < ns) {
      const int gi = W - 1 - (c0 + tid);
      sl = L.gsl[cur * W + gi];
      p = (int)L.gnode[cur * W + gi];
      seg = (int)(sl & 0xFFFFu);
      s = L.buf[cur * W + seg];
      Np0 = N[tb + p];
      const int k = f.nchild[tb + p];
      const int first = f.first[tb + p];
      leaf = (k <= 0) || (first < 0) || (d == c.max_depth - 1);
      if (!leaf && k > RMAX * kWave) {
        atomicOr(&w.status[0], OMQ_STATUS_ROWLIMIT);
        leaf = true;
      }
      keep = !leaf;
    }
    // the leaves: group log, path entry, the arrival's virtual loss, end of the path
    const uint64_t lm = __ballot(leaf);
    if (lm != 0) {
      const int nl = __popcll(lm);
      int gbase = 0;
      if (lane == 0) {
        gbase = sh.gbase + atomicAdd(&sh.gnext, nl);
        atomicAdd(&sh.st[OMQ_ST_PATHNODES], (unsigned long long)nl);
        atomicAdd(&sh.st[OMQ_ST_PATHENTRIES], (unsigned long long)nl * (d + 1));
      }
      gbase = readlane_i(gbase, 0);
      if (leaf) {
        const int gid = gbase + (int)__builtin_amdgcn_mbcnt_hi(
                                    (uint32_t)(lm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)lm, 0u));
        *reinterpret_cast<int4*>(w.glog + ((int64_t)t * gmax + gid) * 4) = make_int4(p, d, seg, 1);
        w.paths[((int64_t)t * MW + s) * MD + d] = p;
        w.gmembers[((int64_t)t * MD + d) * MW + seg] = (uint16_t)s;
        if (vl_done) {
          // the arrival's virtual loss is in N already
        } else if (c.vl_atomic) {
          atomicAdd(&N[tb + p], c.vli);
        } else {
          N[tb + p] = Np0 + c.vli;
        }
        w.path_len[(int64_t)t * MW + s] = d + 1;
        w.leaves[(int64_t)t * MW + s] = p;
        lfs[s] = s;
        lflag[s] = 1;
      }
    }
    const uint64_t km = __ballot(keep);
    if (km != 0) {
      int gbase = 0;
      if (lane == 0) gbase = atomicAdd(&sh.kept, __popcll(km));
      gbase = readlane_i(gbase, 0);
      if (keep) {
        const int g = gbase + (int)__builtin_amdgcn_mbcnt_hi(
                                  (uint32_t)(km >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)km, 0u));
        L.gnode[nxt * W + g] = (uint32_t)p;
        L.gsl[nxt * W + g] = sl;
      }
    }
  }
  __syncthreads();
  const int kept = sh.kept;
  const int nb = sh.nbig[cur];
  // (kernels with the wide lane pass: back to the single-member section, for the lane pass)
  const int dst = SelTraits<RMAX>::kWideLanePass ? W - kept : nb;
  for (int i = tid; i < kept; i += NT) {
    L.gnode[cur * W + dst + i] = L.gnode[nxt * W + i];
    L.gsl[cur * W + dst + i] = L.gsl[nxt * W + i];
  }
  __syncthreads();
  if (tid == 0) {
    if (SelTraits<RMAX>::kWideLanePass)
      sh.nsmall[cur] = kept;
    else
      sh.nbig[cur] = nb + kept;
  }
}

// Size class of a chain group of m members: 0 for the largest (m >= 2^15), 15 for m = 1.
// Small groups decided by the first-unvisited rule, one group per thread, before a level's
// chains.  A group of at most kPrefixMembers members whose node's first kPrefixWindow
// children hold at least m unvisited ones takes them in index order (unvisited_prefix gives
// the rule): member r goes to the r-th of them, each child a single-member group of the next
// level at segment position seg + r.  A group at a leaf ends its members' paths there.  Both
// log the group, write the path entries and apply the arrival's virtual loss as the chain loop
// does.  The other groups stay chains, compacted in place to [0, kept) in their order.  Ends
// with a barrier; sets sh.nbig[cur] to the kept count.
constexpr int kPrefixMembers = 4;
constexpr int kPrefixWindow = 8;

template <int RMAX, int NT>
__device__ inline void prefix_pass(const SelArgs& f, const SelCfg& c, int t, int d, int W,
                                   int64_t tb, int64_t gmax, const LevelLds& L,
                                   LevelShared<NT>& sh, int32_t* lfs, int32_t* lflag, int nb,
                                   bool vl_done, bool sg) {
  const SelArgs& w = f;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int cur = d & 1, nxt = cur ^ 1;
  const int MW = w.max_wave, MD = w.max_depth_buf;
  int32_t* N = f.N;
  const bool big1 = !sg || 1 > SelTraits<RMAX>::kSmall;  // where single-member groups go
  int kept_total = 0;
  for (int c0 = 0; c0 < nb; c0 += NT) {
    const int gi = c0 + tid;
    bool keep = false, done = false, leaf = false;
    uint32_t sl = 0, pn = 0;
    int p = 0, seg = 0, m = 0, k = 0, first = 0, Np0 = 0, scan = 0;
    uint32_t upos = 0u;  // bit j: child j of the window is taken
    if (gi < nb) {
      sl = L.gsl[cur * W + gi];
      pn = L.gnode[cur * W + gi];
      p = (int)pn;
      seg = (int)(sl & 0xFFFFu);
      m = (int)(sl >> 16);
      keep = true;
      if (m <= kPrefixMembers) {
        Np0 = N[tb + p];
        k = f.nchild[tb + p];
        first = f.first[tb + p];
        leaf = (k <= 0) || (first < 0) || (d == c.max_depth - 1);
        if (!leaf && k > RMAX * kWave) {
          atomicOr(&w.status[0], OMQ_STATUS_ROWLIMIT);
          leaf = true;
        }
        if (leaf) {
          done = true;
        } else if (c.vli > 0) {
          int nv[kPrefixWindow];
#pragma unroll
          for (int j = 0; j < kPrefixWindow; ++j)
            nv[j] = j < k ? N[tb + first + 1 + j] : 1;
          int got = 0;
#pragma unroll
          for (int j = 0; j < kPrefixWindow; ++j) {
            const bool take = nv[j] == 0 && got < m;
            upos |= take ? (1u << j) : 0u;
            scan = take ? j + 1 : scan;
            got += take ? 1 : 0;
          }
          done = got >= m;
        }
        keep = !done;
      }
    }
    // the groups finished here: group log, path entries, the arrival's virtual loss
    const uint64_t dm = __ballot(done);
    if (dm != 0) {
      // per-wave totals: group-log entries, statistics and the next level's groups (one
      // atomic each)
      const bool inner = done && !leaf;
      int ntot;
      const int mg = wave_excl_scan(inner ? m : 0, &ntot);
      const int nleafm = wave_sum_i(done && leaf ? m : 0);
      const int ninner = __popcll(__ballot(inner));
      const int scans = wave_sum_i(inner ? scan : 0);
      int gbase = 0, gb = 0;
      if (lane == 0) {
        gbase = sh.gbase + atomicAdd(&sh.gnext, __popcll(dm));
        if (ntot > 0) gb = atomicAdd(big1 ? &sh.nbig[nxt] : &sh.nsmall[nxt], ntot);
        atomicAdd(&sh.st[OMQ_ST_PATHNODES], (unsigned long long)__popcll(dm));
        if (nleafm > 0)
          atomicAdd(&sh.st[OMQ_ST_PATHENTRIES], (unsigned long long)nleafm * (d + 1));
        if (ninner > 0) {
          atomicAdd(&sh.st[OMQ_ST_INTERNAL], (unsigned long long)ninner);
          atomicAdd(&sh.st[OMQ_ST_ROWSUM], (unsigned long long)scans);
          atomicAdd(&sh.st[OMQ_ST_STEPS], (unsigned long long)ntot);
        }
      }
      gbase = readlane_i(gbase, 0);
      gb = readlane_i(gb, 0) + mg;
      if (done) {
        const int gid = gbase + (int)__builtin_amdgcn_mbcnt_hi(
                                    (uint32_t)(dm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)dm, 0u));
        *reinterpret_cast<int4*>(w.glog + ((int64_t)t * gmax + gid) * 4) = make_int4(p, d, seg, m);
        if (vl_done) {
          // the members' virtual loss is in N already
        } else if (c.vl_atomic) {
          atomicAdd(&N[tb + p], c.vli * m);
        } else {
          N[tb + p] = Np0 + c.vli * m;
        }
        const uint16_t* mem = L.buf + cur * W + seg;
        const int s0 = mem[0];
        if (leaf) lflag[s0] = 1;
        uint32_t rest = upos;
        for (int r = 0; r < m; ++r) {
          const int s = mem[r];
          w.paths[((int64_t)t * MW + s) * MD + d] = p;
          w.gmembers[((int64_t)t * MD + d) * MW + seg + r] = (uint16_t)s;
          if (leaf) {
            w.path_len[(int64_t)t * MW + s] = d + 1;
            w.leaves[(int64_t)t * MW + s] = p;
            lfs[s] = s0;
          } else {
            const int j = __ffs(rest) - 1;  // the r-th child taken
            rest &= rest - 1u;
            const int g = big1 ? gb + r : W - 1 - (gb + r);
            L.gnode[nxt * W + g] = (uint32_t)(first + 1 + j);
            L.gsl[nxt * W + g] = (uint32_t)(seg + r) | (1u << 16);
            L.buf[nxt * W + seg + r] = (uint16_t)s;
          }
        }
      }
    }
    // the groups kept as chains, compacted in place (this chunk's entries were read above;
    // every write lands below the chunk's end)
    const uint64_t km = __ballot(keep);
    const int wid = tid / kWave;
    if (lane == 0) sh.wtot[wid] = __popcll(km);
    __syncthreads();
    int before = kept_total, total = kept_total;
    for (int q = 0; q < NT / kWave; ++q) {
      const int v = sh.wtot[q];
      before += q < wid ? v : 0;
      total += v;
    }
    if (keep) {
      const int g = before + (int)__builtin_amdgcn_mbcnt_hi(
                                 (uint32_t)(km >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)km, 0u));
      L.gnode[cur * W + g] = pn;
      L.gsl[cur * W + g] = sl;
    }
    kept_total = total;
    __syncthreads();
  }
  if (tid == 0) sh.nbig[cur] = kept_total;
  __syncthreads();
}

__device__ inline int size_class(int m) { return 15 - min(15, 31 - __clz(m)); }

// Chain groups [0, nb) of a level reordered by size class, largest first, so that the dynamic
// deal hands out the longest chains first and a level does not end on a long chain taken late.
// The order within a class is arbitrary (groups of one level are independent).  tn/ts is
// scratch of nb entries (a free range of the next level's group arrays).  Called by
// every thread of the workgroup.  Kept out of line: inlined, it changes the register
// allocation of the 6-slot kernel's chains.
template <int NT>
__device__ __noinline__ void order_groups(uint32_t* gn, uint32_t* gs, uint32_t* tn, uint32_t* ts,
                                          int nb, int* s_hist) {
  const int tid = threadIdx.x;
  if (tid < 16) s_hist[tid] = 0;
  __syncthreads();
  for (int i = tid; i < nb; i += NT) atomicAdd(&s_hist[size_class((int)(gs[i] >> 16))], 1);
  __syncthreads();
  if (tid < kWave) {  // class counts -> class cursors (exclusive scan)
    const int v = tid < 16 ? s_hist[tid] : 0;
    int tot;
    const int ex = wave_excl_scan(v, &tot);
    if (tid < 16) s_hist[tid] = ex;
  }
  __syncthreads();
  for (int i = tid; i < nb; i += NT) {
    const uint32_t sl = gs[i];
    const int pos = atomicAdd(&s_hist[size_class((int)(sl >> 16))], 1);
    tn[pos] = gn[i];
    ts[pos] = sl;
  }
  __syncthreads();
  for (int i = tid; i < nb; i += NT) {
    gn[i] = tn[i];
    gs[i] = ts[i];
  }
  __syncthreads();
}

// ---- Level overlap -------------------------------------------------------------------
// The root chain is one step per simulation, and during it the workgroup's other waves have
// nothing to do in the level-by-level schedule.  With the overlap, wave 0 runs the root chain
// and publishes every block of 64 picks; the other waves (followers) run the level-1 chains of
// each published block: the block's members of a root child c, in simulation order, continue
// c's chain where the previous blocks left it.  That is the same chain: the chain of c reads
// only N of c and of c's children, and the followers keep both current in memory (N[c] grows by
// VL per member of the block, and each picked child by VL per pick), so the block's r-th member
// of c sees N[c] + VL*r with every earlier member's virtual loss already counted.  One follower
// owns c (c mod the number of followers), so c's blocks run in order on one wave, and no two
// waves touch the same node.  A follower waits only for the root chain, which waits for no one.
// After the level, the level-1 groups are formed from the whole root chain as usual; their
// chains are not run again: each member's pick is replayed from the followers' record (pick2),
// and the virtual loss of levels 1 and 2 is not applied again.  pick2 starts as kPickNone for
// every simulation, so a member whose block a follower never ran (its bounded wait ran out,
// OMQ_STATUS_STALL) ends its path at its level-1 node.
constexpr uint16_t kPickNone = 0xFFFFu;

// Waits until the root chain has published `need` ranks (bounded by `limit` polls: false when
// the bound runs out, which the caller reports as OMQ_STATUS_STALL).
__device__ inline bool wait_progress(const int* prog, int need, int limit) {
  for (int it = 0; it < limit; ++it) {
    const int v = __hip_atomic_load(prog, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (readlane_i(v, 0) >= need) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      return true;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  return false;
}

// Level-1 chains of the followers (wave index fw among nfol), block by block as the root chain
// publishes its picks in root_ch.  Records each member's pick in pick2 (child index, or
// kPickNone when its node has no child to give).
template <int RMAX>
__device__ inline void level1_followers(const SelArgs& f, const SelCfg& c, int64_t tb, int W,
                                        int root_first, const uint32_t* root_ch, uint16_t* pick2,
                                        uint32_t* chs, uint16_t* cnt_s, float4* cscr,
                                        const int* progress, int fw, int nfol) {
  const int lane = lane_id();
  int32_t* N = f.N;
  for (int b0 = 0; b0 < W; b0 += kWave) {
    if (!wait_progress(progress, min(W, b0 + kWave), c.spin_limit)) {
      if (lane == 0) atomicOr(&f.status[0], OMQ_STATUS_STALL);
      return;
    }
    const int s = b0 + lane;
    const uint32_t cv = s < W ? root_ch[s] : kNoChild;
    const int key = cv == kNoChild ? -1 : (int)(cv >> 16);
    const bool mine = key >= 0 && key % nfol == fw;
    uint64_t rest = __ballot(mine);
    // one root child per iteration; each takes at least one lane out of rest
    for (int it = 0; it < kWave && rest != 0; ++it) {
      const int ck = readlane_i(key, lowest_lane(rest));
      const uint64_t mm = __ballot(mine && key == ck);
      rest &= ~mm;
      const int m = __popcll(mm);
      const int p = root_first + 1 + ck;
      const int Np0 = N[tb + p];
      const int k = f.nchild[tb + p];
      const int first = f.first[tb + p];
      if (lane == 0) N[tb + p] = Np0 + c.vli * m;
      const bool leaf = (k <= 0) || (first < 0) || (c.max_depth <= 2) || (k > RMAX * kWave);
      if (!leaf) {
        bool allp;
        group_chain<RMAX, false>(ChainRows{f.N, f.W, f.P}, tb, first, k, Np0, m,
                                 ChainCfg{c.c_puct, c.vlf, c.vli}, chs, cnt_s, cscr, nullptr,
                                 &allp);
        if ((mm >> lane) & 1ull) {
          const int r = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mm >> 32),
                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)mm, 0u));
          const uint32_t v = chs[r];
          pick2[s] = v == kNoChild ? kPickNone : (uint16_t)(v >> 16);
        }
        for (int i = lane; i < k; i += kWave) {
          const int cn = cnt_s[i];
          if (cn > 0) N[tb + first + 1 + i] += c.vli * cn;
        }
      }
      // the next chain of this wave reads the counts written here
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
    }
  }
}

// Replays the picks of a level-1 group's members (simulation order) from pick2 into ch, as
// the chain would write them: (child << 16) | rank among the members that picked the same
// child, kNoChild for none.  Leaves the child counts in cnt_s[0..k); returns the first member
// without a child, or -1.
__device__ inline int replay_picks(const uint16_t* mem, int m, int k, const uint16_t* pick2,
                                   uint32_t* ch, uint16_t* cnt_s) {
  const int lane = lane_id();
  for (int i = lane; i < k; i += kWave) cnt_s[i] = 0;
  wave_sync();
  int fe = -1;
  for (int r0 = 0; r0 < m; r0 += kWave) {
    const int r = r0 + lane;
    const bool v = r < m;
    const int key = v ? (int)pick2[mem[r]] : (int)kPickNone;
    const bool has = v && key != (int)kPickNone;
    const uint64_t none = __ballot(v && !has);
    if (fe < 0 && none != 0) fe = r0 + lowest_lane(none);
    const int base = has ? (int)cnt_s[key] : 0;
    int rk = 0;
    uint64_t rest = __ballot(has);
    for (int it = 0; it < kWave && rest != 0; ++it) {
      const int leader = lowest_lane(rest);
      const int kk = readlane_i(key, leader);
      const uint64_t mm = __ballot(has && key == kk);
      rest &= ~mm;
      if (has && key == kk)
        rk = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mm >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mm, 0u));
      if (lane == leader) cnt_s[kk] = (uint16_t)(base + __popcll(mm));
    }
    if (v) ch[r] = has ? (((uint32_t)key << 16) | (uint32_t)rk) : kNoChild;
    wave_sync();
  }
  return fe;
}


// Run-ahead of level-1 chains (the wide kernels).  A group's chain depends on its node's row
// and count and on nothing of its members: rank r's pick follows from ranks [0, r) alone (the
// parent count at rank r is N + VL*(r+1)), and no level before 1 writes the counts of a root
// child or of its children.  So while one wave runs the root chain, follower j runs the chain
// of the (j+1)-th most visited root child for up to M ranks, M an estimate of the picks the
// child gets (3 times its share of the root's visits plus 64, in blocks of 64, at most the
// wave), recording its picks in spec[0, M).  The chain publishes its ranks done in *m_out
// after each block and ends early once the root chain is done (*stop), so that level 1 does
// not wait for it.  At level 1 that child's group replays ranks [0, m) when m <= *m_out, and
// otherwise replays the ranks done and runs its chain on from there.  Nothing of the forest
// is written.  Records the node (-1: none run) and the first-unvisited prefix length in
// *node_out / *npre_out.
template <int RMAX>
__device__ __noinline__ void run_ahead_chain(ChainRows rows, ChainCfg cc, const int32_t* nchild,
                                             const int32_t* firsts, int64_t tb, int W,
                                             int root_first, int root_k, int j, uint32_t* spec,
                                             uint16_t* cnt_s, float4* cscr, const int* stop,
                                             int* node_out, int* m_out, int* npre_out) {
  const int lane = lane_id();
  if (lane == 0) *m_out = 0;
  // keys (visits, clamped to 22 bits, + 1) << 9 | (511 - child): the largest is the most
  // visited child, the lower index first among equals; 0 marks no child
  uint32_t key[RMAX];
#pragma unroll
  for (int q = 0; q < RMAX; ++q) {
    const int i = q * kWave + lane;
    key[q] = 0u;
    if (i < root_k) {
      const int n = rows.N[tb + root_first + 1 + i];
      key[q] = ((uint32_t)min(max(n, 0), (1 << 22) - 2) + 1u) << 9 | (uint32_t)(511 - i);
    }
  }
  uint32_t top = 0u;
  for (int it = 0; it <= j; ++it) {
    uint32_t mx = 0u;
#pragma unroll
    for (int q = 0; q < RMAX; ++q) mx = max(mx, key[q]);
    top = wave_max_u32(mx);
    if (top == 0u) break;
#pragma unroll
    for (int q = 0; q < RMAX; ++q)
      if (key[q] == top) key[q] = 0u;  // (keys are distinct: one lane, one slot)
  }
  int node = -1, npre = 0;
  if (top != 0u) {
    const int ci = 511 - (int)(top & 511u);
    const int p = root_first + 1 + ci;
    const int k = nchild[tb + p];
    const int first = firsts[tb + p];
    const int Np0 = rows.N[tb + p];
    const int Nr = rows.N[tb];
    if (k > 0 && first >= 0 && k <= RMAX * kWave && Nr > 0) {
      const float share = (float)Np0 / (float)Nr;
      const int est = (int)(3.0f * share * (float)W) + 64;
      const int m = min(W, (est + kWave - 1) / kWave * kWave);
      bool allp;
      group_chain<RMAX, true>(rows, tb, first, k, Np0, m, cc, spec, cnt_s, cscr, m_out, &allp,
                              &npre, stop);
      node = p;
    }
  }
  if (lane == 0) {
    *node_out = node;
    *npre_out = npre;
  }
}

// Replays ranks [0, n) of a chain run ahead (spec, as the chain wrote them) into ch, and the
// child counts of those ranks into cnt_s[0, k) (packed two to a 32-bit word: counts stay below
// 2^16).  Returns the first rank without a child, or -1.
__device__ inline int replay_spec(const uint32_t* spec, int n, int k, uint32_t* ch,
                                  uint16_t* cnt_s) {
  const int lane = lane_id();
  for (int i = lane; i < k; i += kWave) cnt_s[i] = 0;
  wave_sync();
  uint32_t* cnt2 = reinterpret_cast<uint32_t*>(cnt_s);
  int fe = -1;
  for (int r0 = 0; r0 < n; r0 += kWave) {
    const int r = r0 + lane;
    const bool v = r < n;
    const uint32_t cv = v ? spec[r] : kNoChild;
    if (v) ch[r] = cv;
    const uint64_t none = __ballot(v && cv == kNoChild);
    if (fe < 0 && none != 0) fe = r0 + lowest_lane(none);
    if (cv != kNoChild) {
      const uint32_t i = cv >> 16;
      atomicAdd(&cnt2[i >> 1], 1u << ((i & 1u) * 16u));
    }
  }
  wave_sync();
  return fe;
}


// The level-by-level selection of a set of groups, from level d0 until no group is left or
// level dend is reached (its groups then stay in L at parity dend & 1, for the caller).  The
// groups of level d0 are in L and sh at parity d0 & 1.  Returns the level at which it stopped.
//   pipe:       the root chain is overlapped with the level-1 chains (root kernel, d0 = 0);
//               level 1 then replays the followers' picks
//   vl_done_to: levels 1..vl_done_to have their virtual loss in N already (the overlap)
//   run_ahead:  (wide kernels, d0 = 0) the followers run level-1 chains ahead during the root
//               chain (run_ahead_chain); level 1 replays them where they cover a group
//   root_first, root_k: the root's row (the overlap and the run-ahead)
//   glog_ctr:   counter of the tree's group-log entries (LDS or global)
//   lfs, lflag: the tree's per-simulation leaf records (global)
template <int RMAX, int NT, bool WIDE>
__device__ int level_loop(const SelArgs& f, const SelCfg& c, int t, int d0, int dend, int W,
                          const LevelLds& L, LevelShared<NT>& sh, int* glog_ctr, int32_t* lfs,
                          int32_t* lflag, bool pipe, int root_first, int vl_done_to,
                          bool run_ahead, int root_k) {
  constexpr int NW = NT / kWave;
  using Tr = SelTraits<RMAX>;
  const SelArgs& w = f;
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = lane_id();
  const int64_t tb = (int64_t)t * f.capacity;
  const int MW = w.max_wave, MD = w.max_depth_buf;
  const int64_t gmax = (int64_t)MW * MD;
  int32_t* N = f.N;
  uint16_t* cnt_s = L.cnt_all + wave * OMQ_MAX_ROW;
  float4* cscr = L.cscr_all + wave * kWave;  // contender window scratch of this wave
  uint32_t* gnode = L.gnode;
  uint32_t* gsl = L.gsl;
  uint16_t* buf = L.buf;
  int d = d0;
  for (; d < c.max_depth && d < dend; ++d) {
    const int cur = d & 1, nxt = cur ^ 1;
    const int ng = sh.nbig[cur] + sh.nsmall[cur];
    if (ng == 0) break;
    // every group of the level logs one entry: the level's entries are taken at once (one
    // atomic on the tree's counter), the groups then number themselves in LDS
    if (tid == 0) {
      sh.gbase = atomicAdd(glog_ctr, ng);
      sh.gnext = 0;
    }
    __syncthreads();
    const bool replay = pipe && d == 1;  // level-1 picks recorded by the followers
    const bool vl_done = d > 0 && d <= vl_done_to;
    const bool sg = Tr::kSingles && !(pipe && d == 0);  // level-1 groups of the overlap stay chains
    if (Tr::kLeafPass) {
      // single-member groups: leaves finished by all threads at once, the rest become chains
      const int ns = sh.nsmall[cur];
      if (ns > 0) {
        leaf_pass<RMAX, NT>(f, c, t, d, W, tb, gmax, L, sh, lfs, lflag, ns,
                            vl_done && d == vl_done_to);
        if (!Tr::kWideLanePass && tid == 0) sh.nsmall[cur] = 0;
        __syncthreads();
      }
    }
    // small groups decided by the first-unvisited rule, one per thread (not where level 1
    // replays the followers' picks; not for a level of at most one chain group per wave,
    // whose chains take their prefixes themselves without the pass's barriers)
    if (Tr::kPrefixPass && !replay && sh.nbig[cur] > NW)
      prefix_pass<RMAX, NT>(f, c, t, d, W, tb, gmax, L, sh, lfs, lflag, sh.nbig[cur], vl_done,
                            sg);
    const int nb = sh.nbig[cur];
    // more chain groups than waves: the longest first.  The scratch is the next level's group
    // arrays past the groups already there: the kernels without the single-member passes
    // keep the prefix pass's groups at the bottom (the others put them at the top).  Those
    // groups hold members of finished groups and the chain groups at least one member each,
    // so the free range [nbig[nxt], W - nsmall[nxt]) has room for nb entries.
    if (nb > NW) {
      const int toff = Tr::kSingles ? 0 : sh.nbig[nxt];
      order_groups<NT>(gnode + cur * W, gsl + cur * W, gnode + nxt * W + toff,
                       gsl + nxt * W + toff, nb, sh.hist);
    }
    // The chain groups are dealt dynamically: each wave takes the next index from an LDS
    // counter, so a wave that finishes a short chain takes the next group at once.  The next
    // index is requested when a group starts, so that the answer is back by its end.  Every
    // fetch advances the counter, so a wave sees an index >= nb after at most nb + 1
    // fetches; the loop bound states this (it never ends the loop early).  No barrier is
    // inside the loop.
    if (pipe && d == 0 && wave != 0) {
      level1_followers<RMAX>(f, c, tb, W, root_first, L.choice, L.pick2,
                             L.pipe_ch + wave * kWave, cnt_s, cscr, &sh.progress, wave - 1,
                             NW - 1);
    }
    // (wide kernels) the followers run level-1 chains ahead while wave 0 runs the root chain
    if constexpr (WIDE) {
      if (d == 0 && run_ahead && wave != 0 && wave <= kSpecSlots) {
        const int j = wave - 1;
        run_ahead_chain<RMAX>(ChainRows{f.N, f.W, f.P}, ChainCfg{c.c_puct, c.vlf, c.vli},
                              f.nchild, f.first, tb, W, root_first, root_k, j, L.spec + j * W,
                              cnt_s, cscr, &sh.root_done, &sh.spec_node[j], &sh.spec_m[j],
                              &sh.spec_npre[j]);
      }
    }
    // (at level 0 of the overlap and of the run-ahead only wave 0 takes the root)
    const bool deal = !((pipe || run_ahead) && d == 0 && wave != 0);
    int gnext = 0;
    if (deal && lane == 0) gnext = atomicAdd(&sh.next[cur], 1);
    for (int it = 0; it <= nb && deal; ++it) {
      const int gi = readlane_i(gnext, 0);
      if (gi >= nb) break;
      if (lane == 0) gnext = atomicAdd(&sh.next[cur], 1);
      const int p = (int)gnode[cur * W + gi];
      const uint32_t sl = gsl[cur * W + gi];
      const int seg = (int)(sl & 0xFFFFu);
      const int m = (int)(sl >> 16);
      const uint16_t* mem = buf + cur * W + seg;
      // the node's count and row are read before the group's stores below: a wait for a load
      // issued after them would wait for the stores as well (one counter, in issue order)
      int Np0 = N[tb + p];
      const int k = f.nchild[tb + p];
      const int first = f.first[tb + p];

      // log the group and record the path entries
      int gid = 0;
      if (lane == 0) gid = sh.gbase + atomicAdd(&sh.gnext, 1);
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

      if (vl_done) {
        Np0 -= c.vli * m;  // the members' virtual loss is in N already
      } else if (c.vl_atomic) {
        for (int r = lane; r < m; r += kWave) atomicAdd(&N[tb + p], c.vli);
      } else if (lane == 0) {
        N[tb + p] = Np0 + c.vli * m;
      }
      if (lane == 0) atomicAdd(&sh.st[OMQ_ST_PATHNODES], 1ull);

      bool leaf = (k <= 0) || (first < 0) || (d == c.max_depth - 1);
      if (!leaf && k > RMAX * kWave) {
        if (lane == 0) atomicOr(&w.status[0], OMQ_STATUS_ROWLIMIT);
        leaf = true;
      }
      if (leaf) {
        const int s0 = mem[0];
        for (int r = lane; r < m; r += kWave) {
          const int s = mem[r];
          w.path_len[(int64_t)t * MW + s] = d + 1;
          w.leaves[(int64_t)t * MW + s] = p;
          lfs[s] = s0;
        }
        if (lane == 0) {
          lflag[s0] = 1;
          atomicAdd(&sh.st[OMQ_ST_PATHENTRIES], (unsigned long long)m * (d + 1));
        }
        continue;
      }

      uint32_t* ch = L.choice + seg;
      bool allp = false;
      // a level-1 group whose chain a follower ran ahead replays its ranks: all of them when
      // the follower reached m ranks; else those done, and its chain goes on from there
      // (when the first-unvisited prefix ended inside them, which makes the prefix length
      // known, and none of them is without a child)
      int fe = -1;
      int taken = 0;
      bool ahead_done = false;
      if constexpr (WIDE) {
        if (d == 1 && run_ahead) {
          int sj = -1;
#pragma unroll
          for (int j = 0; j < kSpecSlots; ++j)
            if (sh.spec_node[j] == p) sj = j;
          sj = __builtin_amdgcn_readfirstlane(sj);
          if (sj >= 0) {
            const int Ms = __builtin_amdgcn_readfirstlane(sh.spec_m[sj]);
            const int sp = __builtin_amdgcn_readfirstlane(sh.spec_npre[sj]);
            const uint32_t* spec = L.spec + sj * W;
            if (Ms >= m) {
              fe = replay_spec(spec, m, k, ch, cnt_s);
              allp = sp >= m;
              ahead_done = true;
            } else if (sp < Ms && replay_spec(spec, Ms, k, ch, cnt_s) < 0) {
              taken = Ms;
            }
          }
        }
      }
      // (the root's chain is timed: the serial part of the selection)
      const uint64_t tc0 = d == 0 ? __builtin_amdgcn_s_memrealtime() : 0ull;
      if (replay)
        fe = replay_picks(mem, m, k, L.pick2, ch, cnt_s);
      else if (!ahead_done)
        fe = group_chain<RMAX, WIDE>(ChainRows{f.N, f.W, f.P}, tb, first, k, Np0, m,
                                     ChainCfg{c.c_puct, c.vlf, c.vli}, ch, cnt_s, cscr,
                                     pipe && d == 0 ? &sh.progress : nullptr, &allp, nullptr,
                                     nullptr, taken);
      if constexpr (WIDE) {
        // the followers' chains end at their next block
        if (d == 0 && run_ahead && lane == 0)
          __hip_atomic_store(&sh.root_done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      if (d == 0 && lane == 0)
        atomicAdd(&sh.st[OMQ_ST_ROOTCHAIN],
                  (unsigned long long)(__builtin_amdgcn_s_memrealtime() - tc0 + (uint64_t)(fe & 0)));
      if (lane == 0) {
        atomicAdd(&sh.st[OMQ_ST_INTERNAL], 1ull);
        // (a row whose picks are all first-unvisited children is scanned up to its last pick)
        atomicAdd(&sh.st[OMQ_ST_ROWSUM], (unsigned long long)(allp ? (ch[m - 1] >> 16) + 1 : k));
        atomicAdd(&sh.st[OMQ_ST_STEPS], (unsigned long long)m);
      }

      if (allp) {
        // every member picked its own child, in index order: member r makes the single-member
        // group of child ch[r] at segment position seg + r, the layout the general scatter
        // below gives such picks
        const bool big1 = !sg || 1 > Tr::kSmall;
        int gb = 0;
        if (lane == 0) gb = atomicAdd(big1 ? &sh.nbig[nxt] : &sh.nsmall[nxt], m);
        gb = readlane_i(gb, 0);
        for (int r = lane; r < m; r += kWave) {
          const int i = (int)(ch[r] >> 16);
          const int g = big1 ? gb + r : W - 1 - (gb + r);
          gnode[nxt * W + g] = (uint32_t)(first + 1 + i);
          gsl[nxt * W + g] = (uint32_t)(seg + r) | (1u << 16);
          buf[nxt * W + seg + r] = mem[r];
        }
        wave_sync();
        continue;
      }

      // exclusive scan of the child counts (blocks of B children per lane) -> offsets, and
      // the groups of the next level
      const int B = (k + kWave - 1) / kWave;
      const int lo = lane * B, hi = min(lo + B, k);
      // (chain groups go to the bottom of the next level's group arrays, single-member groups
      // of the kernels that keep them apart to the top)
      int sum = 0, nbg = 0, nsm = 0;
      for (int i = lo; i < hi; ++i) {
        const int v = cnt_s[i];
        sum += v;
        const bool big = !sg || v > Tr::kSmall;
        nbg += v > 0 && big;
        nsm += v > 0 && !big;
      }
      int tot_sum, tot_bg, tot_sm;
      int run = wave_excl_scan(sum, &tot_sum);
      int pbg = wave_excl_scan(nbg, &tot_bg);
      int psm = wave_excl_scan(nsm, &tot_sm);
      int bbase = 0, sbase = 0;
      if (lane == 0 && tot_bg > 0) bbase = atomicAdd(&sh.nbig[nxt], tot_bg);
      if (lane == 0 && tot_sm > 0) sbase = atomicAdd(&sh.nsmall[nxt], tot_sm);
      bbase = readlane_i(bbase, 0);
      sbase = readlane_i(sbase, 0);
      for (int i = lo; i < hi; ++i) {
        const int v = cnt_s[i];
        if (v > 0) {
          const bool big = !sg || v > Tr::kSmall;
          const int g = big ? bbase + pbg++ : W - 1 - (sbase + psm++);
          gnode[nxt * W + g] = (uint32_t)(first + 1 + i);
          gsl[nxt * W + g] = (uint32_t)(seg + run) | ((uint32_t)v << 16);
        }
        cnt_s[i] = (uint16_t)run;
        run += v;
      }
      wave_sync();

      // scatter the members to their child's segment (rank keeps simulation order), kSU
      // members per lane at a time: their reads are issued together (they come from this
      // level's half of buf and from ch and cnt_s, none of which the writes to the next
      // level's half touch).  Two in the 1024-thread kernels, whose registers are fewer.
      constexpr int kSU = NT <= 512 ? 4 : 2;
      const int s_end = fe >= 0 ? (int)mem[fe] : -1;
      for (int r0 = lane; r0 < m; r0 += kSU * kWave) {
        int sv[kSU];
        uint32_t cvv[kSU];
#pragma unroll
        for (int u = 0; u < kSU; ++u) {
          const int r = r0 + u * kWave;
          sv[u] = r < m ? (int)mem[r] : 0;
          cvv[u] = r < m ? ch[r] : 0u;
        }
        int off[kSU];
#pragma unroll
        for (int u = 0; u < kSU; ++u) {
          const bool to_child = r0 + u * kWave < m && cvv[u] != kNoChild;
          off[u] = to_child ? (int)cnt_s[cvv[u] >> 16] : 0;
        }
#pragma unroll
        for (int u = 0; u < kSU; ++u) {
          if (r0 + u * kWave >= m) break;
          const int s = sv[u];
          const uint32_t cv = cvv[u];
          if (cv == kNoChild) {
            w.path_len[(int64_t)t * MW + s] = d + 1;
            w.leaves[(int64_t)t * MW + s] = p;
            lfs[s] = s_end;
            atomicAdd(&sh.st[OMQ_ST_PATHENTRIES], (unsigned long long)(d + 1));
          } else {
            buf[nxt * W + seg + off[u] + (int)(cv & 0xFFFFu)] = (uint16_t)s;
          }
        }
      }
      if (fe >= 0 && lane == 0) {
        lflag[s_end] = 1;
        atomicOr(&w.status[0], OMQ_STATUS_NOCHILD);
      }
      wave_sync();
    }
    if (Tr::kLanePass)
      small_groups<RMAX, NT>(f, c, t, d, W, tb, gmax, L, sh, lfs, lflag,
                             vl_done && d == vl_done_to);
    if (Tr::kWideLanePass && sh.nsmall[cur] > 0)
      small_groups_call<RMAX, NT>(f, c, t, d, W, tb, gmax, L, sh, lfs, lflag,
                                  vl_done && d == vl_done_to);
    __syncthreads();
    if (tid == 0) {
      sh.nbig[cur] = 0;
      sh.nsmall[cur] = 0;
      sh.next[cur] = 0;
      sh.snext = 0;
    }
    __syncthreads();
  }
  return d;
}

// The level-d0 group set of (node p, segment [seg, seg + m)) put into L / sh (members read
// from mem_src, or 0..m-1 when it is null).  Called by every thread; ends with a barrier.
template <int RMAX, int NT>
__device__ inline void start_group(const LevelLds& L, LevelShared<NT>& sh, int W, int d0, int p,
                                   int seg, int m, const uint16_t* mem_src) {
  const int tid = threadIdx.x;
  const int cur = d0 & 1;
  for (int r = tid; r < m; r += NT)
    L.buf[cur * W + seg + r] = mem_src ? mem_src[r] : (uint16_t)(seg + r);
  if (tid < OMQ_NSTATS) sh.st[tid] = 0;
  if (tid < 8) sh.spec_node[tid] = -1;
  if (tid == 0) {
    // a single member goes to the single-member groups of the kernels that keep them apart
    const bool big = !SelTraits<RMAX>::kSingles || m > SelTraits<RMAX>::kSmall;
    const int g0 = big ? 0 : W - 1;
    L.gnode[cur * W + g0] = (uint32_t)p;
    L.gsl[cur * W + g0] = (uint32_t)seg | ((uint32_t)m << 16);
    sh.nbig[cur] = big ? 1 : 0;
    sh.nsmall[cur] = big ? 0 : 1;
    sh.nbig[cur ^ 1] = 0;
    sh.nsmall[cur ^ 1] = 0;
    sh.next[0] = 0;
    sh.next[1] = 0;
    sh.snext = 0;
    sh.progress = 0;
    sh.root_done = 0;
  }
  __syncthreads();
}

// Unique leaves of tree t in order of first occurrence, from the per-simulation leaf records
// lflag / lfs (global; lflag is scanned in place), and, with kRecords, each unique leaf's key
// and legal count (leaf_key_count, as omq_leaf_info forms them).  Called by every thread of
// the workgroup.
template <int NT, bool kRecords>
__device__ inline void finish_tree(const SelArgs& w, const RecordArgs& ra, int t, int W,
                                   int32_t* lfs, int32_t* lflag, int* s_wtot,
                                   unsigned long long* s_uleafpath) {
  const int tid = threadIdx.x;
  const int MW = w.max_wave;
  const int nu = block_excl_scan<NT>(lflag, W, s_wtot);
  int rc = 0;
  omq_forest fo{};
  omq_wave wo{};
  if constexpr (kRecords) {
    fo.capacity = w.capacity;
    fo.num_actions = ra.num_actions;
    fo.game = ra.game;
    fo.legal_words = ra.legal_words;
    fo.min_legal = ra.min_legal;
    fo.max_legal = ra.max_legal;
    fo.actions = const_cast<int32_t*>(ra.actions);
    fo.root_keys = const_cast<uint64_t*>(ra.root_keys);
    fo.root_legal = const_cast<uint32_t*>(ra.root_legal);
    wo.max_wave = MW;
    wo.max_depth = w.max_depth_buf;
    wo.paths = w.paths;
    wo.path_len = w.path_len;
    rc = fo.game != OMQ_GAME_SPARSE ? root_legal_count(fo, t) : 0;
  }
  int plen_sum = 0;
  for (int s = tid; s < W; s += NT) {
    const int s0 = lfs[s];
    const int uid = lflag[s0];
    w.sim_uid[(int64_t)t * MW + s] = uid;
    if (s0 == s) {
      w.uleaf[(int64_t)t * MW + uid] = w.leaves[(int64_t)t * MW + s];
      w.ufirst[(int64_t)t * MW + uid] = s;
      if constexpr (kRecords) {
        uint64_t key;
        int count;
        plen_sum += leaf_key_count(fo, wo, t, s, rc, &key, &count);
        ra.ukey[(int64_t)t * MW + uid] = key;
        ra.ulegal[(int64_t)t * MW + uid] = count;
      }
    }
  }
  if constexpr (kRecords) {
    const int ws = wave_sum_i(plen_sum);
    if (lane_id() == 0 && ws > 0) atomicAdd(s_uleafpath, (unsigned long long)ws);
  }
  if (tid == 0) {
    w.ucount[t] = nu;
    atomicAdd(reinterpret_cast<unsigned long long*>(&w.stats[(int64_t)t * OMQ_NSTATS +
                                                             OMQ_ST_ULEAVES]),
              (unsigned long long)nu);
    atomicAdd(reinterpret_cast<unsigned long long*>(&w.stats[(int64_t)t * OMQ_NSTATS +
                                                             OMQ_ST_SIMS]),
              (unsigned long long)W);
  }
}

template <int NT>
__device__ inline void flush_stats(const SelArgs& w, int t, LevelShared<NT>& sh) {
  const int tid = threadIdx.x;
  if (tid < OMQ_NSTATS && sh.st[tid] != 0)
    atomicAdd(reinterpret_cast<unsigned long long*>(&w.stats[(int64_t)t * OMQ_NSTATS + tid]),
              sh.st[tid]);
}

// ---- Kernels ---------------------------------------------------------------------------
// The select kernel: one workgroup per tree runs every level of its tree's wave, then the
// unique-leaf pass (with kRecords, the unique leaves' keys and legal counts too).  The kRecords
// kernels are compiled in a code object of their own (tree_select_records.hip): compiled into
// this one, the records' code cost C3's 6-slot kernel 2.3 us per launch though it did not run
// there (behind a run-time test), and as a second instantiation beside it, 2.0 us (the
// out-of-line chain functions the two kernels share were compiled differently).
template <int RMAX, int NT, bool kRecords>
__global__ __launch_bounds__(NT, 1) void select_root_kernel(SelArgs f, SelCfg c,
                                                           RecordArgs ra) {
  // the level overlap in the kernels whose chains keep their registers with a second copy of
  // the chain code (the followers'), with a full workgroup of followers (the 1- and 2-slot
  // kernels: every kernel of more slots runs 512 threads)
  constexpr bool kPipe = RMAX <= 3 && NT == 1024;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ LevelShared<NT> sh;
  __shared__ int s_glog;
  const int W = c.W;
  const LevelLds L = carve_level_lds<NT>(smem, W, kPipe);
  const int t = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t tb = (int64_t)t * f.capacity;
  const int MW = f.max_wave;
  int32_t* lflag = f.lflag + (int64_t)t * MW;
  int32_t* lfs = f.lfs + (int64_t)t * MW;
  // the level overlap needs an internal root, an integer virtual loss and the ordered mode
  const int root_k = f.nchild[tb], root_first = f.first[tb];
  const bool pipe = kPipe && L.pick2 != nullptr && W > kWave && !c.vl_atomic && c.vli > 0 &&
                    c.max_depth >= 2 && root_k > 0 && root_first >= 0 &&
                    root_k <= RMAX * kWave;
  for (int s = tid; s < W; s += NT) {
    lflag[s] = 0;
    if (L.pick2 != nullptr) L.pick2[s] = kPickNone;
  }
  if (tid == 0) {
    s_glog = 0;
    // the chains keep a row's counts as floats (1 + N) advanced by the virtual loss, exact
    // while below 2^24; every node's count is at most its root's
    if ((int64_t)f.N[tb] + 1 + (int64_t)c.vli * W >= (int64_t)(1 << 24))
      atomicOr(&f.status[0], OMQ_STATUS_COUNTLIMIT);
  }
  start_group<RMAX, NT>(L, sh, W, 0, 0, 0, W, nullptr);
  // the run-ahead needs an internal root of a row the kernel takes, an integer virtual loss
  // and levels below 1 (a level-1 group at the last level is a leaf)
  const bool run_ahead = NT <= 512 && L.spec != nullptr && c.vli > 0 && c.max_depth >= 3 &&
                         root_k > 0 && root_first >= 0 && root_k <= RMAX * kWave;
  level_loop<RMAX, NT, NT <= 512>(f, c, t, 0, c.max_depth, W, L, sh, &s_glog, lfs, lflag, pipe,
                                  root_first, pipe ? 2 : -1, run_ahead, root_k);
  __syncthreads();
  finish_tree<NT, kRecords>(f, ra, t, W, lfs, lflag, sh.wtot, &sh.st[OMQ_ST_ULEAFPATH]);
  __syncthreads();
  if (tid == 0) f.gcount[t] = s_glog;
  flush_stats<NT>(f, t, sh);
}

}  // namespace omq

namespace omq {
// Threads of the whole-wave kernel: 512 for the kernels of more than 4 slots per lane, whose
// chains then keep up to 256 registers (at 1024 threads, 128: the 6-slot chains spilled 12-100
// registers, depending on the code around them).  The first-unvisited prefix leaves their
// levels below the root few chains, so 8 waves suffice there.
constexpr int select_threads(int rmax) { return rmax >= kWideRmax ? 512 : 1024; }

// The kRecords select kernel of rmax slots per lane (tree_select_records.hip).
const void* select_records_kernel(int rmax);
}  // namespace omq

#ifdef OMQ_SELECT_RECORDS_TU
// ---- the kRecords kernels (this file compiled again by tree_select_records.hip) ----
namespace omq {
const void* select_records_kernel(int rmax) {
  switch (rmax) {
#define OMQ_PICK(R) \
  case R:           \
    return (const void*)select_root_kernel<R, select_threads(R), true>;
    OMQ_PICK(1)
    OMQ_PICK(2)
    OMQ_PICK(3)
    OMQ_PICK(4)
    OMQ_PICK(5)
    OMQ_PICK(6)
    default:
    OMQ_PICK(8)
#undef OMQ_PICK
  }
}
}  // namespace omq
#else
// ---- host launcher (C++ linkage; the C ABI wrappers live in capi.hip) ----
namespace omq {

namespace {
std::atomic<int> g_spin_limit{OMQ_SPIN_LIMIT_DEFAULT};  // polls of a follower's bounded wait
constexpr int kMaxDevices = 64;
std::atomic<bool> g_attr_set[kMaxDevices][9][2];

struct SelKernel {
  const void* fn;
  int threads;
};

SelKernel pick_kernel(int rmax, bool records) {
  if (records) return SelKernel{select_records_kernel(rmax), select_threads(rmax)};
  switch (rmax) {
#define OMQ_PICK(R) \
  case R:           \
    return SelKernel{(const void*)select_root_kernel<R, select_threads(R), false>, \
                     select_threads(R)};
    OMQ_PICK(1)
    OMQ_PICK(2)
    OMQ_PICK(3)
    OMQ_PICK(4)
    OMQ_PICK(5)
    OMQ_PICK(6)
    default:
    OMQ_PICK(8)
#undef OMQ_PICK
  }
}
}  // namespace

void select_set_options(int spin_limit) {
  g_spin_limit.store(spin_limit, std::memory_order_relaxed);
}

int select_spin_limit() { return g_spin_limit.load(std::memory_order_relaxed); }

hipError_t launch_select(const omq_forest& f, const omq_wave& w, int W, float c_puct,
                         float virtual_loss, int max_depth, int vl_atomic, hipStream_t stream) {
  SelCfg c;
  c.W = W;
  c.c_puct = c_puct;
  c.vlf = virtual_loss;
  c.vli = (int)virtual_loss;
  c.max_depth = max_depth;
  c.vl_atomic = vl_atomic;
  c.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
  // widest row the game model can produce: every legal action (board games) or max_legal
  const int max_row = f.game == OMQ_GAME_SPARSE ? f.max_legal : f.num_actions;
  int rmax = (max_row + kWave - 1) / kWave;
  if (rmax < 1) rmax = 1;
  if (rmax > 6) rmax = 8;
  // the unique leaves' records in select for the waves of at most OMQ_SELECT_RECORDS_MAX_WAVE
  const bool records = W <= OMQ_SELECT_RECORDS_MAX_WAVE;
  const SelKernel k = pick_kernel(rmax, records);
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const bool cache = dev >= 0 && dev < kMaxDevices;
  // the LDS limit is raised once per device and kernel (the attribute is idempotent, so two
  // threads racing here both set it)
  if (!cache || !g_attr_set[dev][rmax][records].load(std::memory_order_acquire)) {
    const size_t lds_max =
        k.threads == 1024
            ? std::max(level_lds_bytes<1024>(OMQ_MAX_WAVE, true), level_lds_bytes<1024>(kPipeMaxW, true))
            : std::max(level_lds_bytes<512>(OMQ_MAX_WAVE, false), level_lds_bytes<512>(kPipeMaxW, false));
    e = hipFuncSetAttribute(k.fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_max);
    if (e != hipSuccess) return e;
    if (cache) g_attr_set[dev][rmax][records].store(true, std::memory_order_release);
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
  a.num_trees = f.num_trees;
  const int64_t TM = (int64_t)f.num_trees * w.max_wave;
  a.lflag = w.sel_scratch;
  a.lfs = w.sel_scratch + TM;
  RecordArgs ra;
  ra.actions = f.actions;
  ra.root_keys = f.root_keys;
  ra.root_legal = f.root_legal;
  ra.ukey = w.ukey;
  ra.ulegal = w.ulegal;
  ra.game = f.game;
  ra.num_actions = f.num_actions;
  ra.legal_words = f.legal_words;
  ra.min_legal = f.min_legal;
  ra.max_legal = f.max_legal;
  void* args[] = {&a, &c, &ra};
  const size_t lds = k.threads == 1024 ? level_lds_bytes<1024>(W, true)
                                       : level_lds_bytes<512>(W, false);
  e = hipLaunchKernel(k.fn, dim3(f.num_trees), dim3(k.threads), args, lds, stream);
  if (e != hipSuccess) return e;
  return hipGetLastError();
}

}  // namespace omq
#endif  // OMQ_SELECT_RECORDS_TU
