// Gomoku positions of the unique leaves of a wave: terminal check and feature planes (gfx950).
//
// The reference decides after every move whether a child state is terminal.
// CPUGameStates.apply_actions (python/mcts/cpu/cpu_game_states.py:352-412) calls
// FastTerminalChecker._check_gomoku_terminal_cpu with last_move=None, which is a full-board
// scan (python/mcts/utils/fast_terminal_check.py:132-232):
//   - cells are visited in row-major order; at an occupied cell, the directions horizontal,
//     vertical, down-right and down-left are tried in that order;
//   - a direction counts when there is room for five cells (col <= bs-5 / row <= bs-5 / both /
//     row <= bs-5 and col >= 4) and all five belong to the cell's player;
//   - the first cell with a counting direction names the winner;
//   - with use_renju, a five of player 1 that continues on either side (an overline) does not
//     count, and it ends the scan of that cell: the reference's `continue` skips the
//     remaining directions of the cell;
//   - a full board without a five is a draw.
// The driver does not expand a terminal leaf (python/mcts/cpu/optimized_wave_search.py:374-376),
// but it still backs up the evaluator's value for it.
//
// Here a leaf's position is never stored.  It is rebuilt in LDS from the root board and the
// moves on the leaf's path: one wavefront per unique leaf, colours alternating from the
// root's player to move.  The leaf is then scanned cell-parallel: lane l takes cells
// l, l+64, ..., and a wave min over the winning cells reproduces the row-major first.  A
// terminal leaf gets ulegal = 0, which keeps omq_expand from expanding it.
#include "omq_common.h"

namespace omq {

// Rebuilds the position of unique leaf u of tree t into the wave's LDS board b: the root board
// with the path's moves played in alternating colours from the root's player to move.  Returns
// the path length L (the leaf has L-1 moves on it).  *rp_out receives the root's player to
// move: root_player[t], or 1 when the root board holds an even number of stones, else 2
// (python/mcts/core/mcts.py:1503-1508); *stones_out the root board's stone count.
__device__ inline int rebuild_leaf_board(const omq_forest& f, const omq_wave& w,
                                         const int8_t* root_boards, const int32_t* root_player,
                                         int t, int u, int cells, int8_t* b, int* rp_out,
                                         int* stones_out) {
  const int lane = lane_id();
  const int8_t* rb = root_boards + (int64_t)t * cells;
  int stones = 0;
  for (int i = lane; i < cells; i += kWave) {
    const int8_t v = rb[i];
    b[i] = v;
    stones += v != 0;
  }
  stones = wave_sum_i(stones);
  const int s0 = w.ufirst[(int64_t)t * w.max_wave + u];
  int a_lo, a_hi;
  const int L = load_path_actions(f, w, t, s0, &a_lo, &a_hi);
  const int rp = root_player != nullptr ? root_player[t] : ((stones & 1) == 0 ? 1 : 2);
  wave_sync();
  // move j (0-based, depth j+1) is played by rp when j is even; lane l holds moves l and l+64
  const int8_t mine = (int8_t)((lane & 1) == 0 ? rp : 3 - rp);
  if (lane + 1 < L && a_lo >= 0 && a_lo < cells) b[a_lo] = mine;
  if (lane + 65 < L && a_hi >= 0 && a_hi < cells) b[a_hi] = mine;
  wave_sync();
  *rp_out = rp;
  *stones_out = stones;
  return L;
}

__global__ void gomoku_terminal_kernel(omq_forest f, omq_wave w, const int8_t* root_boards,
                                       const int32_t* root_player, int rule, int bs,
                                       int32_t* uterm) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int cells = bs * bs;
  const int stride = (cells + 15) & ~15;
  const int t = blockIdx.y;
  const int wave = threadIdx.x / kWave;
  const int u = blockIdx.x * (blockDim.x / kWave) + wave;
  const int lane = lane_id();
  const int64_t wb = (int64_t)t * w.max_wave;
  if (u >= w.ucount[t]) return;
  int8_t* b = reinterpret_cast<int8_t*>(smem + (size_t)wave * stride);
  int rp, stones;
  const int L = rebuild_leaf_board(f, w, root_boards, root_player, t, u, cells, b, &rp, &stones);
  if (L <= 1) {  // the root position itself is not checked (the reference never flags it)
    if (uterm != nullptr && lane == 0) uterm[wb + u] = OMQ_TERM_NONE;
    return;
  }

  constexpr int dr[4] = {0, 1, 1, 1};
  constexpr int dc[4] = {1, 0, 1, -1};
  int win = 0x7FFFFFFF;
  int empty = 0;
  for (int cell = lane; cell < cells; cell += kWave) {
    const int p = b[cell];
    if (p == 0) {
      ++empty;
      continue;
    }
    const int r = cell / bs, c = cell - (cell / bs) * bs;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int re = r + 4 * dr[d], ce = c + 4 * dc[d];
      if (re >= bs || ce < 0 || ce >= bs) continue;  // no room for five in this direction
      bool five = true;
#pragma unroll
      for (int k = 1; k < 5; ++k) five = five && b[(r + k * dr[d]) * bs + c + k * dc[d]] == p;
      if (!five) continue;
      if (rule == OMQ_RULE_RENJU && p == 1) {
        const int rn = r + 5 * dr[d], cn = c + 5 * dc[d];
        const int rq = r - dr[d], cq = c - dc[d];
        const bool after = rn < bs && cn >= 0 && cn < bs && b[rn * bs + cn] == p;
        const bool before = rq >= 0 && cq >= 0 && cq < bs && b[rq * bs + cq] == p;
        if (after || before) break;  // overline: the reference skips the rest of this cell
      }
      win = min(win, cell);
      break;
    }
  }
  win = (int)~wave_max_u32(~(uint32_t)win);  // wave min
  empty = wave_sum_i(empty);
  int code = OMQ_TERM_NONE;
  if (win != 0x7FFFFFFF) code = b[win];
  else if (empty == 0) code = OMQ_TERM_DRAW;
  if (lane == 0) {
    if (code != OMQ_TERM_NONE) w.ulegal[wb + u] = 0;
    if (uterm != nullptr) uterm[wb + u] = code;
  }
}

// Go rules of unique leaf u of tree t (one wavefront per leaf): the leaf's position is rebuilt
// as for Gomoku (a pass, action cells, places no stone), then lane l takes the points l, l+64,
// ... of the board.  A point is legal when it is empty, is not the root's ko point (OMQ_GO_KO:
// the reference's clones inherit a state's ko point, so it holds at every depth), and, with
// OMQ_GO_SUICIDE, has an empty orthogonal neighbour; the pass is always legal.  The 64 points of each chunk become two mask words by one ballot.  Trailing passes are
// counted from the path's end (the root's own when every path move is a pass).
__global__ void go_rules_kernel(omq_forest f, omq_wave w, const int8_t* root_boards,
                                const int32_t* root_player, const int32_t* root_passes,
                                const int32_t* root_ko, int flags, int bs, int32_t* uterm) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int cells = bs * bs;
  const int stride = (cells + 15) & ~15;
  const int t = blockIdx.y;
  const int wave = threadIdx.x / kWave;
  const int u = blockIdx.x * (blockDim.x / kWave) + wave;
  const int lane = lane_id();
  const int64_t wb = (int64_t)t * w.max_wave;
  if (u >= w.ucount[t]) return;
  int8_t* b = reinterpret_cast<int8_t*>(smem + (size_t)wave * stride);
  int rp, stones;
  const int L = rebuild_leaf_board(f, w, root_boards, root_player, t, u, cells, b, &rp, &stones);
  // trailing passes of the path (moves 0..L-2; lane j holds move j, lane j holds move j+64 in
  // the high word)
  const int s0 = w.ufirst[wb + u];
  int a_lo, a_hi;
  load_path_actions(f, w, t, s0, &a_lo, &a_hi);
  int trail = 0;
  for (int j = L - 2; j >= 0; --j) {
    const int a = j < kWave ? readlane_i(a_lo, j) : readlane_i(a_hi, j - kWave);
    if (a != cells) break;
    ++trail;
  }
  if (trail == L - 1 && root_passes != nullptr) trail += root_passes[t];
  const int ko = ((flags & OMQ_GO_KO) && root_ko != nullptr) ? root_ko[t] : -1;
  const bool suicide = (flags & OMQ_GO_SUICIDE) != 0;
  uint32_t* mask = w.umask + (wb + u) * (int64_t)f.legal_words;
  int legal = 0, empty = 0;
  // points 0..cells-1, then the pass (action cells, always legal)
  for (int c0 = 0; c0 <= cells; c0 += kWave) {
    const int c = c0 + lane;
    bool ok = c == cells;
    if (c < cells && b[c] == 0) {
      ++empty;
      ok = c != ko;
      if (ok && suicide) {
        const int r = c / bs, col = c - r * bs;
        const bool lib = (r > 0 && b[c - bs] == 0) || (r + 1 < bs && b[c + bs] == 0) ||
                         (col > 0 && b[c - 1] == 0) || (col + 1 < bs && b[c + 1] == 0);
        ok = lib;
      }
    }
    const uint64_t m = __ballot(ok);
    legal += ok ? 1 : 0;
    // words c0/32 and c0/32 + 1 (legal_words = ceil((cells + 1) / 32) covers the pass)
    if (lane == 0) mask[c0 >> 5] = (uint32_t)m;
    if (lane == 1 && (c0 >> 5) + 1 < f.legal_words) mask[(c0 >> 5) + 1] = (uint32_t)(m >> 32);
  }
  legal = wave_sum_i(legal);
  empty = wave_sum_i(empty);
  if (lane == 0) {
    const bool term = L > 1 && (trail >= 2 || empty == 0);
    w.ulegal[wb + u] = term ? 0 : legal;
    if (uterm != nullptr) uterm[wb + u] = term ? OMQ_TERM_END : OMQ_TERM_NONE;
  }
}

hipError_t launch_go_rules(const omq_forest& f, const omq_wave& w, const int8_t* boards,
                           const int32_t* root_player, const int32_t* root_passes,
                           const int32_t* root_ko, int flags, int bs, int32_t* uterm,
                           hipStream_t st) {
  constexpr int wpb = 4;
  const size_t lds = (size_t)(((bs * bs) + 15) & ~15) * wpb;
  dim3 grid((w.max_wave + wpb - 1) / wpb, f.num_trees);
  hipLaunchKernelGGL(go_rules_kernel, grid, dim3(wpb * kWave), lds, st, f, w, boards,
                     root_player, root_passes, root_ko, flags, bs, uterm);
  return hipGetLastError();
}

hipError_t launch_gomoku_terminal(const omq_forest& f, const omq_wave& w, const int8_t* boards,
                                  const int32_t* root_player, int rule, int bs, int32_t* uterm,
                                  hipStream_t st) {
  constexpr int wpb = 4;
  const size_t lds = (size_t)(((bs * bs) + 15) & ~15) * wpb;
  dim3 grid((w.max_wave + wpb - 1) / wpb, f.num_trees);
  hipLaunchKernelGGL(gomoku_terminal_kernel, grid, dim3(wpb * kWave), lds, st, f, w, boards,
                     root_player, rule, bs, uterm);
  return hipGetLastError();
}

// Feature planes of every wave slot (one 256-thread workgroup per slot u of tree t).  Slot
// u < ucount[t] holds the position of unique leaf u; the other slots are written with zeros.
// Planes follow CPUGameStates.get_nn_features, representation 'basic'
// (python/mcts/cpu/cpu_game_states.py:430-494), with the leaf's player to move and move count
// as CPUGameStates.apply_actions (cpu_game_states.py:352-412) leaves them after the path:
//   0 stones of the player to move, 1 stones of the opponent, 2-15 zero (history, unused by
//   the reference), 16 ones when player 1 is to move, 17 move count / 100 (the reference's
//   int16 count divided in double, stored as float), 18 ones (only with 19 planes).
// Wave 0 rebuilds the leaf's board in LDS; then the whole workgroup writes the slot's planes,
// one contiguous block of PLANES*cells values, element i by thread i mod 256, two values per
// store where the block has an even length.
constexpr int kFeatThreads = 256;

template <typename OutT>
struct PlaneStore;
template <>
struct PlaneStore<float> {
  using Pair = float2;
  __device__ static float one(float v) { return v; }
  __device__ static float2 two(float a, float b) { return make_float2(a, b); }
};
template <>
struct PlaneStore<uint16_t> {  // bfloat16, rounded to nearest even
  using Pair = uint32_t;
  __device__ static uint16_t one(float v) {
    const uint32_t x = __float_as_uint(v);
    return (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
  }
  __device__ static uint32_t two(float a, float b) {
    return (uint32_t)one(a) | ((uint32_t)one(b) << 16);
  }
};

template <typename OutT, int PLANES, bool NHWC>
__global__ __launch_bounds__(kFeatThreads) void leaf_features_kernel(
    omq_forest f, omq_wave w, const int8_t* root_boards, const int32_t* root_player,
    const int32_t* root_moves, int bs, OutT* out) {
  using S = PlaneStore<OutT>;
  using Pair = typename S::Pair;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float s_val[4];  // player to move is 1, move count / 100, player to move
  const int cells = bs * bs;
  const int t = blockIdx.y;
  const int u = blockIdx.x;
  const int tid = threadIdx.x;
  const int per = PLANES * cells;
  OutT* o = out + ((int64_t)t * w.max_wave + u) * per;
  const bool pairs = (per & 1) == 0;  // then every slot starts on a pair boundary
  if (u >= w.ucount[t]) {
    if (pairs) {
      Pair* o2 = reinterpret_cast<Pair*>(o);
      for (int i = tid; i < per / 2; i += kFeatThreads) o2[i] = S::two(0.0f, 0.0f);
    } else {
      for (int i = tid; i < per; i += kFeatThreads) o[i] = S::one(0.0f);
    }
    return;
  }
  int8_t* b = reinterpret_cast<int8_t*>(smem);
  if (tid < kWave) {
    int rp, stones;
    const int L = rebuild_leaf_board(f, w, root_boards, root_player, t, u, cells, b, &rp,
                                     &stones);
    if (tid == 0) {
      const int moves = L - 1;
      const int tm = (moves & 1) == 0 ? rp : 3 - rp;  // player to move at the leaf
      const int mc = (root_moves != nullptr ? root_moves[t] : stones) + moves;
      s_val[0] = tm == 1 ? 1.0f : 0.0f;
      s_val[1] = (float)((double)mc / 100.0);
      s_val[2] = (float)tm;
    }
  }
  __syncthreads();
  const float colour = s_val[0], mcv = s_val[1];
  const int tm = (int)s_val[2];
  auto value = [&](int i) -> float {
    int c, cell;
    if (NHWC) {
      cell = i / PLANES;
      c = i - cell * PLANES;
    } else {
      c = i / cells;
      cell = i - c * cells;
    }
    if (c == 0) return b[cell] == tm ? 1.0f : 0.0f;
    if (c == 1) return b[cell] == 3 - tm ? 1.0f : 0.0f;
    if (c == 16) return colour;
    if (c == 17) return mcv;
    if (c == 18) return 1.0f;
    return 0.0f;
  };
  if (pairs) {
    Pair* o2 = reinterpret_cast<Pair*>(o);
    for (int i = tid; i < per / 2; i += kFeatThreads) o2[i] = S::two(value(2 * i), value(2 * i + 1));
  } else {
    for (int i = tid; i < per; i += kFeatThreads) o[i] = S::one(value(i));
  }
}

template <typename OutT>
hipError_t launch_leaf_features_t(const omq_forest& f, const omq_wave& w, const int8_t* boards,
                                  const int32_t* root_player, const int32_t* root_moves, int bs,
                                  int planes, bool nhwc, OutT* out, hipStream_t st) {
  const size_t lds = (size_t)(((bs * bs) + 15) & ~15);
  dim3 grid(w.max_wave, f.num_trees);
#define OMQ_FEAT_LAUNCH(P, NH)                                                                  \
  hipLaunchKernelGGL((leaf_features_kernel<OutT, P, NH>), grid, dim3(kFeatThreads), lds, st, f, \
                     w, boards, root_player, root_moves, bs, out)
  if (planes == 18) {
    if (nhwc) OMQ_FEAT_LAUNCH(18, true);
    else OMQ_FEAT_LAUNCH(18, false);
  } else {
    if (nhwc) OMQ_FEAT_LAUNCH(19, true);
    else OMQ_FEAT_LAUNCH(19, false);
  }
#undef OMQ_FEAT_LAUNCH
  return hipGetLastError();
}

hipError_t launch_leaf_features(const omq_forest& f, const omq_wave& w, const int8_t* boards,
                                const int32_t* root_player, const int32_t* root_moves, int bs,
                                int planes, int dtype, int nhwc, void* out, hipStream_t st) {
  if (dtype == OMQ_DTYPE_BF16)
    return launch_leaf_features_t(f, w, boards, root_player, root_moves, bs, planes, nhwc != 0,
                                  static_cast<uint16_t*>(out), st);
  return launch_leaf_features_t(f, w, boards, root_player, root_moves, bs, planes, nhwc != 0,
                                static_cast<float*>(out), st);
}

}  // namespace omq
