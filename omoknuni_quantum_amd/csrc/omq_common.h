// Device-side helpers shared by the tree-operation kernels (gfx950, wave64).
//
// Arithmetic rules: every floating-point expression here is evaluated in IEEE binary32 with
// round-to-nearest-even, no contraction into FMA (-ffp-contract=off), correctly rounded
// division and square root (-fhip-fp32-correctly-rounded-divide-sqrt).  Under those rules the
// expressions give the same bits on any IEEE machine, which is what makes the selection
// decisions and the synthetic workload reproducible on the host.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "omq_tree_ops.h"

namespace omq {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------------------
// Hashing: SplitMix64 finaliser (Steele, Lea, Flood, "Fast splittable pseudorandom number
// generators", OOPSLA 2014; constants of Vigna's splitmix64.c).
// ---------------------------------------------------------------------------------------
constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;
constexpr uint64_t kSaltValue = 0xD1B54A32D192ED03ull;
constexpr uint64_t kSaltLogit = 0xC2B2AE3D27D4EB4Full;
constexpr uint64_t kSaltCount = 0x165667B19E3779F9ull;
constexpr uint64_t kSaltFloyd = 0xFF51AFD7ED558CCDull;

__host__ __device__ inline uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + kGolden;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// key of the child reached from a node with key `k` by action `a`
__host__ __device__ inline uint64_t child_key(uint64_t k, int a) {
  return splitmix64(k ^ ((uint64_t)(a + 1) * kGolden));
}

// leaf value in [-1, 1): v = 2u - 1, u = 24-bit hash fraction (exact in binary32)
__device__ inline float key_value(uint64_t k) {
  uint32_t u24 = (uint32_t)(splitmix64(k ^ kSaltValue) >> 40);
  float u = (float)u24 * (1.0f / 16777216.0f);
  return 2.0f * u - 1.0f;
}

// Approximately standard-normal draw for (key, action): Irwin-Hall sum of twelve discrete
// uniforms (u16 + 1/2)/65536 minus 6.  Mean 0, variance 1 - 2^-32.  Computed in integers and
// converted exactly: z = (S + 6 - 393216) / 65536 with |S + 6 - 393216| < 2^19.
__device__ inline float key_normal(uint64_t k, int a) {
  uint64_t h0 = splitmix64(k ^ ((uint64_t)(a + 1) * kSaltLogit));
  uint64_t h1 = splitmix64(h0);
  uint64_t h2 = splitmix64(h1);
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += (int32_t)((h0 >> (16 * i)) & 0xFFFF);
    s += (int32_t)((h1 >> (16 * i)) & 0xFFFF);
    s += (int32_t)((h2 >> (16 * i)) & 0xFFFF);
  }
  return (float)(s + 6 - 393216) * (1.0f / 65536.0f);
}

// e^x from basic operations: Cody-Waite reduction x = k ln2 + r (ln2 split into a 15-bit
// head and a tail, so k*head is exact for |k| < 2^9), degree-6 Taylor polynomial of e^r in
// Horner form, scaling by 2^k.  Results below e^-87 are returned as 0 (no subnormals).
__device__ inline float exp_cw(float x) {
  if (!(x > -87.0f)) return 0.0f;
  if (x > 88.0f) x = 88.0f;
  const float k = __builtin_rintf(x * 1.44269502f);
  const float r = (x - k * 0.693145751953125f) - k * 1.42860677e-06f;
  float p = 1.0f / 720.0f;
  p = p * r + 1.0f / 120.0f;
  p = p * r + 1.0f / 24.0f;
  p = p * r + 1.0f / 6.0f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  return __builtin_ldexpf(p, (int)k);
}

// ---------------------------------------------------------------------------------------
// Wave64 helpers
// ---------------------------------------------------------------------------------------
__device__ inline int lane_id() { return __lane_id(); }

__device__ inline void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// index of the lowest set bit of a non-zero mask
__device__ inline int lowest_lane(uint64_t m) { return __ffsll((unsigned long long)m) - 1; }

__device__ inline float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ inline int readlane_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }

// Max over the 64 lanes (any value, no NaN), broadcast to every lane.  Max is exact and
// order-free, so the DPP reduction tree below (row shifts, then row broadcasts into lane 63)
// gives the same result as any other order.
__device__ inline float wave_max_f32(float x) {
  const int ninf = (int)0xFF800000u;
  int xi = __float_as_int(x);
  int y;
  y = __builtin_amdgcn_update_dpp(ninf, xi, 0x111, 0xF, 0xF, false);  // row_shr:1
  x = fmaxf(x, __int_as_float(y)); xi = __float_as_int(x);
  y = __builtin_amdgcn_update_dpp(ninf, xi, 0x112, 0xF, 0xF, false);  // row_shr:2
  x = fmaxf(x, __int_as_float(y)); xi = __float_as_int(x);
  y = __builtin_amdgcn_update_dpp(ninf, xi, 0x114, 0xF, 0xF, false);  // row_shr:4
  x = fmaxf(x, __int_as_float(y)); xi = __float_as_int(x);
  y = __builtin_amdgcn_update_dpp(ninf, xi, 0x118, 0xF, 0xF, false);  // row_shr:8
  x = fmaxf(x, __int_as_float(y)); xi = __float_as_int(x);
  y = __builtin_amdgcn_update_dpp(ninf, xi, 0x142, 0xA, 0xF, false);  // row_bcast:15
  x = fmaxf(x, __int_as_float(y)); xi = __float_as_int(x);
  y = __builtin_amdgcn_update_dpp(ninf, xi, 0x143, 0xC, 0xF, false);  // row_bcast:31
  x = fmaxf(x, __int_as_float(y)); xi = __float_as_int(x);
  return __int_as_float(__builtin_amdgcn_readlane(xi, 63));
}

// Order-preserving map of binary32 onto uint32 (a < b  <=>  fkey(a) < fkey(b) for non-NaN
// values; NaNs map above +inf), and its inverse.
__device__ inline uint32_t fkey(float x) {
  const uint32_t b = __float_as_uint(x);
  return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}
__device__ inline float funkey(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

// Max over the 64 lanes of a uint32, broadcast to every lane.  DPP row shifts 1,2,4,8 and
// row broadcasts 15,31 accumulate into lane 63; a lane whose DPP source is outside its row,
// or whose row is masked off, reads its own value (max-neutral).
__device__ inline uint32_t wave_max_u32(uint32_t x) {
  // the DPP source of an invalid or masked lane reads 0, the identity of the max, so each
  // step is one fused v_max_u32_dpp
  int v = (int)x;
  v = (int)max((uint32_t)v, (uint32_t)__builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true));
  v = (int)max((uint32_t)v, (uint32_t)__builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true));
  v = (int)max((uint32_t)v, (uint32_t)__builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true));
  v = (int)max((uint32_t)v, (uint32_t)__builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true));
  v = (int)max((uint32_t)v, (uint32_t)__builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, true));
  v = (int)max((uint32_t)v, (uint32_t)__builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, true));
  return (uint32_t)__builtin_amdgcn_readlane(v, 63);
}

// Canonical wave sum: lane l has already accumulated, in ascending element order starting
// from +0, the elements whose index is congruent to l mod 64; the 64 partial sums are then
// combined by the xor butterfly with distances 32,16,8,4,2,1.  Every lane ends with the same
// value.  (The host restatement of this order must match it exactly.)
// Workgroups are dispatched to the chip's XCDs round-robin in linear order (workgroup i to XCD
// i mod kXcds, as its (i / kXcds)-th).  xcd_block gives each XCD one contiguous run of the
// grid's blocks instead: block i takes logical block start(i mod kXcds) + i / kXcds, where XCD x
// owns blocks [start(x), start(x) + q + (x < r)) of nblk = 8q + r.  A bijection on the grid;
// (bx, by) become the logical block's coordinates.
constexpr int kXcds = 8;
__device__ inline void xcd_block(int* bx, int* by) {
  const int X = (int)gridDim.x;
  const int nblk = X * (int)gridDim.y;
  const int lin = (int)blockIdx.y * X + (int)blockIdx.x;
  const int q = nblk / kXcds, r = nblk % kXcds;
  const int x = lin % kXcds;
  const int logical = x * q + min(x, r) + lin / kXcds;
  *bx = logical % X;
  *by = logical / X;
}

__device__ inline float wave_sum_canonical(float partial) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) partial = partial + __shfl_xor(partial, off, 64);
  return partial;
}
__device__ inline double wave_sum_canonical_d(double partial) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) partial = partial + __shfl_xor(partial, off, 64);
  return partial;
}

__device__ inline int wave_sum_i(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// exclusive prefix sum over lanes (lane 0 gets 0); total returned through *total
__device__ inline int wave_excl_scan(int v, int* total) {
  const int lane = lane_id();
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  *total = __shfl(x, 63, 64);
  return x - v;
}

// ---------------------------------------------------------------------------------------
// Game models: legal actions of a leaf
// ---------------------------------------------------------------------------------------

// number of legal actions of a SPARSE-model node with key k
__device__ inline int sparse_legal_count(const omq_forest& f, uint64_t k) {
  const uint32_t span = (uint32_t)(f.max_legal - f.min_legal + 1);
  return f.min_legal + (int)((uint32_t)(splitmix64(k ^ kSaltCount) >> 33) % span);
}

// Sorted legal list of a SPARSE-model node: Floyd's sampling of n distinct values of
// [0, A) (Bentley & Floyd, "A sample of brilliance", CACM 30(9), 1987), then sorted by rank.
// Requires n <= 64.  `list` is wave-private LDS of at least n entries; `bm` is wave-private LDS
// of f.legal_words words (a scratch bitmap of [0, A), used when it covers A).  Returns n.
__device__ inline int sparse_legal_list(const omq_forest& f, uint64_t k, int* list,
                                        uint32_t* bm) {
  const int lane = lane_id();
  const int A = f.num_actions;
  const int n = sparse_legal_count(f, k);
  // lane i draws step i's value r_i in [0, j_i], j_i = A - n + i (the draws are independent)
  const int jl = A - n + lane;
  int r = -1;
  if (lane < n)
    r = (int)((uint32_t)(splitmix64(k ^ ((uint64_t)(jl + 1) * kSaltFloyd)) >> 32) %
              (uint32_t)(jl + 1));
  // With no two equal draws, every step adds its own draw; otherwise the steps are replayed
  // in order, a draw already taken being replaced by j_i.  The test for equal draws also ranks
  // the draws, which is the rank sort of the sampled values when they are distinct.
  bool dup = false;
  int rank = 0;
  const int nw = (A + 31) >> 5;
  if (f.legal_words >= nw && nw <= 3 * kWave) {
    // the draws as bits of an LDS bitmap: an OR that finds its bit set has an equal draw
    for (int i = lane; i < nw; i += kWave) bm[i] = 0u;
    wave_sync();
    uint32_t old = 0u;
    if (lane < n) old = atomicOr(&bm[r >> 5], 1u << (r & 31));
    dup = lane < n && ((old >> (r & 31)) & 1u);
    wave_sync();
    // a value's rank is the number of bits below it: lane l holds words 3l .. 3l+2, whose
    // popcounts are scanned over the lanes; a value in word v takes the scan at lane v / 3, the
    // counts of that lane's words before v, and the bits below it in word v
    auto rank_of = [&](int x) -> int {
      const uint32_t x0 = 3 * lane < nw ? bm[3 * lane] : 0u;
      const uint32_t x1 = 3 * lane + 1 < nw ? bm[3 * lane + 1] : 0u;
      const uint32_t x2 = 3 * lane + 2 < nw ? bm[3 * lane + 2] : 0u;
      const int c0 = __popc(x0), c1 = __popc(x1);
      int tot;
      const int e = wave_excl_scan(c0 + c1 + __popc(x2), &tot);
      const int v = lane < n ? (x >> 5) : 0;
      const int src = v / 3, sub = v - 3 * src;
      const int pe = __shfl(e, src, kWave), p0 = __shfl(c0, src, kWave),
                p1 = __shfl(c1, src, kWave);
      const uint32_t xv = bm[v];
      return pe + (sub >= 1 ? p0 : 0) + (sub == 2 ? p1 : 0) +
             __popc(xv & ((1u << (x & 31)) - 1u));
    };
    const uint64_t fl0 = __ballot(dup);
    if (fl0 != 0) {
      // Floyd's steps without replaying them: step i takes j_i instead of its draw when the
      // draw is already in the set, that is when an earlier lane drew the same value (D), or
      // when the draw is j_k of an earlier step k that took j_k.  The second rule links a step
      // to one earlier step, so the rounds below settle it (at most n of them).
      bool D = false;
      uint64_t fl = fl0;
      for (int it = 0; it < kWave && fl != 0; ++it) {
        const int v = readlane_i(r, lowest_lane(fl));
        const uint64_t eq = __ballot(lane < n && r == v);
        D = D || (lane < n && r == v && lane > lowest_lane(eq));
        fl &= ~eq;
      }
      const int kk = r - (A - n);
      const bool link = lane < n && kk >= 0 && kk < lane;
      bool col = D;
      for (int it = 0; it < n; ++it) {
        const int ck = __shfl((int)col, link ? kk : lane, kWave);
        const bool nc = D || (link && ck != 0);
        const bool changed = __ballot(nc != col) != 0;
        col = nc;
        if (!changed) break;
      }
      if (col) r = A - n + lane;
      // the sampled values are distinct now: their bitmap ranks them
      wave_sync();
      for (int i = lane; i < nw; i += kWave) bm[i] = 0u;
      wave_sync();
      if (lane < n) atomicOr(&bm[r >> 5], 1u << (r & 31));
      wave_sync();
      dup = false;
    }
    rank = rank_of(r);
  } else {
    for (int i = 0; i < n; ++i) {
      const int v = readlane_i(r, i);
      dup = dup || (lane > i && v == r);
      rank += (lane < n && v < r) ? 1 : 0;
    }
  }
  int mine = r;  // lane i holds the i-th sampled value
  if (__ballot(dup && lane < n) != 0) {
    mine = -1;
    for (int i = 0; i < n; ++i) {
      const int ri = readlane_i(r, i);
      const bool hit = __ballot(lane < i && mine == ri) != 0;
      if (lane == i) mine = hit ? A - n + i : ri;
    }
    // rank sort of the replayed values (distinct)
    rank = 0;
    for (int i = 0; i < n; ++i) {
      const int v = readlane_i(mine, i);
      rank += (lane < n && v < mine) ? 1 : 0;
    }
  }
  if (lane < n) list[rank] = mine;
  wave_sync();
  return n;
}

// Leaf record of a unique leaf whose first simulation is s0: the key (the root key folded with
// the actions of the path's nodes, depths 1..L-1) and the legal count (board games: the root's
// count, root_count, less the path's moves, a pass excepted: every legal list excludes the
// moves on its path, so they are distinct and legal at the root; sparse model: from the key).
// One thread per leaf; returns the path length L.
__device__ inline int leaf_key_count(const omq_forest& f, const omq_wave& w, int t, int s0,
                                     int root_count, uint64_t* key_out, int* count_out) {
  const int64_t wb = (int64_t)t * w.max_wave;
  const int64_t tb = (int64_t)t * f.capacity;
  const int L = w.path_len[wb + s0];
  const int32_t* path = w.paths + (wb + s0) * w.max_depth;
  const bool board = f.game != OMQ_GAME_SPARSE;
  const int pass = f.game == OMQ_GAME_GO ? f.num_actions - 1 : -1;
  const uint32_t* root = f.root_legal + (int64_t)t * f.legal_words;
  uint64_t key = f.root_keys[t];
  int taken = 0;
  // eight depths at a time: their path entries, then their actions, in flight together
  constexpr int kB = 8;
  for (int d0 = 1; d0 < L; d0 += kB) {
    int pv[kB], av[kB];
#pragma unroll
    for (int j = 0; j < kB; ++j) pv[j] = d0 + j < L ? path[d0 + j] : 0;
#pragma unroll
    for (int j = 0; j < kB; ++j) av[j] = d0 + j < L ? f.actions[tb + pv[j]] : 0;
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      if (d0 + j >= L) break;
      const int a = av[j];
      key = child_key(key, a);
      if (board && a != pass && a >= 0 && a < f.num_actions) taken += (root[a >> 5] >> (a & 31)) & 1u;
    }
  }
  *key_out = key;
  *count_out = board ? root_count - taken : sparse_legal_count(f, key);
  return L;
}

// The root's legal count of tree t (board games).
__device__ inline int root_legal_count(const omq_forest& f, int t) {
  const uint32_t* root = f.root_legal + (int64_t)t * f.legal_words;
  int c = 0;
  for (int i = 0; i < f.legal_words; ++i) c += __popc(root[i]);
  return c;
}

// Load the actions on the path of simulation s (depths 1..L-1) into lanes: lane j holds
// the action at depth j+1 (and depth j+65 in *a_hi).  Returns L.
__device__ inline int load_path_actions(const omq_forest& f, const omq_wave& w, int t, int s,
                                        int* a_lo, int* a_hi) {
  const int lane = lane_id();
  const int64_t tb = (int64_t)t * f.capacity;
  const int L = w.path_len[(int64_t)t * w.max_wave + s];
  const int32_t* path = w.paths + ((int64_t)t * w.max_wave + s) * w.max_depth;
  int lo = -1, hi = -1;
  if (lane + 1 < L) lo = f.actions[tb + path[lane + 1]];
  if (lane + 65 < L) hi = f.actions[tb + path[lane + 65]];
  *a_lo = lo;
  *a_hi = hi;
  return L;
}

// Board legal mask of a leaf into wave-private LDS words: root mask minus path cells.
// For OMQ_GAME_GO the pass action (A-1) is never cleared.
__device__ inline void board_legal_mask(const omq_forest& f, int t, int L, int a_lo, int a_hi,
                                        uint32_t* mask) {
  const int lane = lane_id();
  const int nw = f.legal_words;
  const uint32_t* root = f.root_legal + (int64_t)t * nw;
  for (int i = lane; i < nw; i += kWave) mask[i] = root[i];
  wave_sync();
  const int pass = (f.game == OMQ_GAME_GO) ? f.num_actions - 1 : -1;
  if (lane + 1 < L && a_lo >= 0 && a_lo != pass)
    atomicAnd(&mask[a_lo >> 5], ~(1u << (a_lo & 31)));
  if (lane + 65 < L && a_hi >= 0 && a_hi != pass)
    atomicAnd(&mask[a_hi >> 5], ~(1u << (a_hi & 31)));
  wave_sync();
}

// Legal mask of unique leaf u of tree t from the wave's umask (the rule kernel's) into
// wave-private LDS words.
__device__ inline void leaf_umask(const omq_forest& f, const omq_wave& w, int t, int u,
                                  uint32_t* mask) {
  const uint32_t* src = w.umask + ((int64_t)t * w.max_wave + u) * f.legal_words;
  for (int i = lane_id(); i < f.legal_words; i += kWave) mask[i] = src[i];
  wave_sync();
}

// Sorted legal list from a board mask (ascending actions).  Returns the count.
__device__ inline int board_legal_list(const omq_forest& f, const uint32_t* mask, int* list) {
  const int lane = lane_id();
  const int A = f.num_actions;
  int base = 0;
  for (int c = 0; c < A; c += kWave) {
    const int a = c + lane;
    const bool legal = a < A && ((mask[a >> 5] >> (a & 31)) & 1u);
    const uint64_t b = __ballot(legal);
    if (legal) {
      const int pos = base + __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32),
                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0));
      list[pos] = a;
    }
    base += __popcll(b);
  }
  wave_sync();
  return base;
}

// Legal list of unique leaf u of tree t (sorted ascending) into wave-private LDS.
// `mask` must hold legal_words words (board games), `list` the maximum legal count.
__device__ inline int leaf_legal_list(const omq_forest& f, const omq_wave& w, int t, int u,
                                      uint32_t* mask, int* list) {
  if (f.game == OMQ_GAME_SPARSE) {
    return sparse_legal_list(f, w.ukey[(int64_t)t * w.max_wave + u], list, mask);
  }
  if (w.umask != nullptr) {
    leaf_umask(f, w, t, u, mask);
    return board_legal_list(f, mask, list);
  }
  const int s0 = w.ufirst[(int64_t)t * w.max_wave + u];
  int a_lo, a_hi;
  const int L = load_path_actions(f, w, t, s0, &a_lo, &a_hi);
  board_legal_mask(f, t, L, a_lo, a_hi, mask);
  return board_legal_list(f, mask, list);
}

}  // namespace omq
