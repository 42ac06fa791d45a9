/*
 * tree_oracle.c -- CPU oracle of the wave-MCTS tree operations.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP library is compared
 * against; it is loaded by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
 * leg, and by nothing in the product path.
 *
 * It restates, sequentially and in plain C, the CPU tree path of the reference
 * (cosmosapjw-quantum/omoknuni_quantum):
 *   - tree state and init ........ python/mcts/cpu/cython_tree_optimized.pyx:36-103
 *   - select_path (VL on arrival)  cython_tree_optimized.pyx:177-202
 *   - best child (UCB) ........... cython_tree_optimized.pyx:421-464
 *   - expand_node ................ cython_tree_optimized.pyx:232-277
 *   - backup with VL revert ...... cython_tree_optimized.pyx:204-230 (VL part) with the driver's
 *                                  leaf-positive sign, optimized_wave_search.py:457-483
 *   - expansion policy ........... optimized_wave_search.py:367-438
 *   - search / waves ............. python/mcts/core/mcts.py:923-1063, root expansion 1659-1691
 * with the canonical choices documented at each function (orders that the reference leaves
 * to numpy are fixed here).  Compile with -ffp-contract=off and without -ffast-math: every
 * float expression is evaluated in IEEE binary32 in source order.
 *
 * The synthetic workload (node keys, legal sets, evaluator) is restated here from its
 * specification, independently of the device code.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_GAME_BOARD 0
#define ORC_GAME_GO 1
#define ORC_GAME_SPARSE 2
#define ORC_EXPAND_FULL 0
#define ORC_EXPAND_REFERENCE_PW 1
#define ORC_SIGN_LEAF_POSITIVE 0
#define ORC_SIGN_ROOT_POSITIVE 1
#define ORC_RULE_FREESTYLE 0
#define ORC_RULE_RENJU 1
#define ORC_TERM_NONE 0
#define ORC_TERM_DRAW 3
#define ORC_TERM_END 4
#define ORC_GO_KO 1
#define ORC_GO_SUICIDE 2

typedef struct orc_forest {
  /* shape */
  int T, cap, A, game, legal_words, min_legal, max_legal;
  int max_wave, max_depth;
  /* parameters */
  float c_puct, vl;
  int expand_policy, sign_mode;
  float logit_scale;
  double eps;
  /* tree arrays [T*cap] */
  int32_t *N;
  float *W, *P;
  int32_t *parent, *first, *nchild, *action;
  uint8_t *expanded;
  int32_t *children, *child_actions; /* edges [T*cap] */
  int32_t *num_nodes, *num_edges;    /* [T] */
  uint64_t *root_keys;               /* [T] */
  uint32_t *root_legal;              /* [T*legal_words] */
  double *root_noise;                /* [T*A] or NULL */
  /* last-wave trace [T*max_wave(*max_depth)] */
  int32_t *paths, *path_len, *leaves, *sim_uid, *uleaf, *ufirst, *ucount;
  uint64_t *ukey;
  int32_t *ulegal, *uexpanded;
  float *policy, *values; /* [T*max_wave*A] (legal slots written), [T*max_wave] */
  int32_t *seen;          /* [T*cap] unique-leaf index of a node during a wave, else -1 */
  /* Gomoku rules (terminal leaves are not expanded); off unless orc_set_gomoku_rules */
  int rules_on, rule;
  int8_t *root_boards;    /* [T*A] 0 empty, 1/2 stones */
  int32_t *root_player;   /* [T] player of the first path move */
  int32_t *uterm;         /* [T*max_wave] ORC_TERM_* of each unique leaf */
  /* Go rules (legal moves from the leaf position, terminal leaves); off unless
     orc_set_go_rules */
  int go_on, go_flags;
  int8_t *go_boards;                      /* [T*(A-1)] root positions */
  int32_t *go_player, *go_passes, *go_ko; /* [T]: player of the first path move, the root's
                                             trailing passes, the root's ko point (-1: none) */
} orc_forest;

/* ---- synthetic workload (same specification as the device code) ---------------------- */
static const uint64_t GOLDEN = 0x9E3779B97F4A7C15ull;
static const uint64_t SALT_VALUE = 0xD1B54A32D192ED03ull;
static const uint64_t SALT_LOGIT = 0xC2B2AE3D27D4EB4Full;
static const uint64_t SALT_COUNT = 0x165667B19E3779F9ull;
static const uint64_t SALT_FLOYD = 0xFF51AFD7ED558CCDull;

uint64_t orc_splitmix64(uint64_t x) {
  uint64_t z = x + GOLDEN;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t orc_child_key(uint64_t k, int a) { return orc_splitmix64(k ^ ((uint64_t)(a + 1) * GOLDEN)); }

float orc_key_value(uint64_t k) {
  uint32_t u24 = (uint32_t)(orc_splitmix64(k ^ SALT_VALUE) >> 40);
  float u = (float)u24 * (1.0f / 16777216.0f);
  return 2.0f * u - 1.0f;
}

/* Irwin-Hall(12) with 16-bit uniforms: z = (sum + 6 - 12*32768) / 65536 */
float orc_key_normal(uint64_t k, int a) {
  uint64_t h[3];
  h[0] = orc_splitmix64(k ^ ((uint64_t)(a + 1) * SALT_LOGIT));
  h[1] = orc_splitmix64(h[0]);
  h[2] = orc_splitmix64(h[1]);
  int32_t s = 0;
  for (int j = 0; j < 3; ++j)
    for (int i = 0; i < 4; ++i) s += (int32_t)((h[j] >> (16 * i)) & 0xFFFF);
  return (float)(s + 6 - 393216) * (1.0f / 65536.0f);
}

/* e^x: Cody-Waite reduction by ln2 (15-bit head), degree-6 Taylor polynomial, 2^k scaling */
float orc_exp_cw(float x) {
  if (!(x > -87.0f)) return 0.0f;
  if (x > 88.0f) x = 88.0f;
  const float k = rintf(x * 1.44269502f);
  const float r = (x - k * 0.693145751953125f) - k * 1.42860677e-06f;
  float p = 1.0f / 720.0f;
  p = p * r + 1.0f / 120.0f;
  p = p * r + 1.0f / 24.0f;
  p = p * r + 1.0f / 6.0f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  return ldexpf(p, (int)k);
}

/* canonical 64-lane sum: lane l adds elements l, l+64, ... in order from +0, then the xor
   butterfly with distances 32..1 (element i of x, n elements) */
float orc_sum64(const float *x, int n) {
  float part[64], tmp[64];
  for (int l = 0; l < 64; ++l) part[l] = 0.0f;
  for (int i = 0; i < n; ++i) part[i & 63] = part[i & 63] + x[i];
  for (int off = 32; off >= 1; off >>= 1) {
    for (int l = 0; l < 64; ++l) tmp[l] = part[l] + part[l ^ off];
    memcpy(part, tmp, sizeof part);
  }
  return part[0];
}

double orc_sum64d(const double *x, int n) {
  double part[64], tmp[64];
  for (int l = 0; l < 64; ++l) part[l] = 0.0;
  for (int i = 0; i < n; ++i) part[i & 63] = part[i & 63] + x[i];
  for (int off = 32; off >= 1; off >>= 1) {
    for (int l = 0; l < 64; ++l) tmp[l] = part[l] + part[l ^ off];
    memcpy(part, tmp, sizeof part);
  }
  return part[0];
}

static int sparse_count(const orc_forest *f, uint64_t k) {
  uint32_t span = (uint32_t)(f->max_legal - f->min_legal + 1);
  return f->min_legal + (int)((uint32_t)(orc_splitmix64(k ^ SALT_COUNT) >> 33) % span);
}

/* Floyd's sampling of n distinct actions of [0,A), sorted ascending */
static int sparse_list(const orc_forest *f, uint64_t k, int *list) {
  const int A = f->A;
  const int n = sparse_count(f, k);
  int S[64];
  for (int i = 0; i < n; ++i) {
    const int j = A - n + i;
    const uint32_t r = (uint32_t)(orc_splitmix64(k ^ ((uint64_t)(j + 1) * SALT_FLOYD)) >> 32) %
                       (uint32_t)(j + 1);
    int hit = 0;
    for (int q = 0; q < i; ++q)
      if (S[q] == (int)r) hit = 1;
    S[i] = hit ? j : (int)r;
  }
  /* insertion sort */
  for (int i = 1; i < n; ++i) {
    int v = S[i], q = i - 1;
    while (q >= 0 && S[q] > v) {
      S[q + 1] = S[q];
      --q;
    }
    S[q + 1] = v;
  }
  memcpy(list, S, sizeof(int) * (size_t)n);
  return n;
}

/* legal list of a node given its path actions (depth 1..L-1) and key */
static int go_legal_list(const orc_forest *f, int t, const int *acts, int np, int *list);

static int legal_list(const orc_forest *f, int t, const int *pacts, int npacts, uint64_t key,
                      int *list) {
  if (f->game == ORC_GAME_SPARSE) return sparse_list(f, key, list);
  if (f->go_on) return go_legal_list(f, t, pacts, npacts, list);
  const int A = f->A;
  const int pass = f->game == ORC_GAME_GO ? A - 1 : -1;
  const uint32_t *root = f->root_legal + (size_t)t * f->legal_words;
  int n = 0;
  for (int a = 0; a < A; ++a) {
    if (!((root[a >> 5] >> (a & 31)) & 1u)) continue;
    int on_path = 0;
    if (a != pass)
      for (int q = 0; q < npacts; ++q)
        if (pacts[q] == a) on_path = 1;
    if (!on_path) list[n++] = a;
  }
  return n;
}

/* ---- forest ----------------------------------------------------------------------------- */
orc_forest *orc_create(int T, int cap, int A, int game, int min_legal, int max_legal,
                       int max_wave, int max_depth) {
  orc_forest *f = (orc_forest *)calloc(1, sizeof(orc_forest));
  if (!f) return NULL;
  f->T = T;
  f->cap = cap;
  f->A = A;
  f->game = game;
  f->legal_words = (A + 31) / 32;
  f->min_legal = min_legal;
  f->max_legal = max_legal;
  f->max_wave = max_wave;
  f->max_depth = max_depth;
  f->c_puct = 1.414f;
  f->vl = 3.0f;
  f->logit_scale = 1.0f;
  size_t nc = (size_t)T * cap, nw = (size_t)T * max_wave;
  f->N = (int32_t *)calloc(nc, 4);
  f->W = (float *)calloc(nc, 4);
  f->P = (float *)calloc(nc, 4);
  f->parent = (int32_t *)calloc(nc, 4);
  f->first = (int32_t *)calloc(nc, 4);
  f->nchild = (int32_t *)calloc(nc, 4);
  f->action = (int32_t *)calloc(nc, 4);
  f->expanded = (uint8_t *)calloc(nc, 1);
  f->children = (int32_t *)calloc(nc, 4);
  f->child_actions = (int32_t *)calloc(nc, 4);
  f->num_nodes = (int32_t *)calloc((size_t)T, 4);
  f->num_edges = (int32_t *)calloc((size_t)T, 4);
  f->root_keys = (uint64_t *)calloc((size_t)T, 8);
  f->root_legal = (uint32_t *)calloc((size_t)T * f->legal_words, 4);
  f->paths = (int32_t *)calloc(nw * max_depth, 4);
  f->path_len = (int32_t *)calloc(nw, 4);
  f->leaves = (int32_t *)calloc(nw, 4);
  f->sim_uid = (int32_t *)calloc(nw, 4);
  f->uleaf = (int32_t *)calloc(nw, 4);
  f->ufirst = (int32_t *)calloc(nw, 4);
  f->ucount = (int32_t *)calloc((size_t)T, 4);
  f->ukey = (uint64_t *)calloc(nw, 8);
  f->ulegal = (int32_t *)calloc(nw, 4);
  f->uexpanded = (int32_t *)calloc(nw, 4);
  f->policy = (float *)calloc(nw * (size_t)A, 4);
  f->values = (float *)calloc(nw, 4);
  f->uterm = (int32_t *)calloc(nw, 4);
  f->seen = (int32_t *)malloc(nc * 4);
  if (f->seen) memset(f->seen, 0xFF, nc * 4);
  if (!f->seen || !f->N || !f->W || !f->P || !f->parent || !f->first || !f->nchild || !f->action ||
      !f->expanded || !f->children || !f->child_actions || !f->paths || !f->policy ||
      !f->uterm) {
    return NULL;
  }
  return f;
}

void orc_destroy(orc_forest *f) {
  if (!f) return;
  void *ptrs[] = {f->N, f->W, f->P, f->parent, f->first, f->nchild, f->action, f->expanded,
                  f->children, f->child_actions, f->num_nodes, f->num_edges, f->root_keys,
                  f->root_legal, f->paths, f->path_len, f->leaves, f->sim_uid, f->uleaf,
                  f->ufirst, f->ucount, f->ukey, f->ulegal, f->uexpanded, f->policy, f->values,
                  f->root_noise, f->seen, f->uterm, f->root_boards, f->root_player,
                  f->go_boards, f->go_player, f->go_passes, f->go_ko};
  for (size_t i = 0; i < sizeof ptrs / sizeof ptrs[0]; ++i) free(ptrs[i]);
  free(f);
}

void orc_set_params(orc_forest *f, float c_puct, float vl, int expand_policy, int sign_mode,
                    float logit_scale, double eps) {
  f->c_puct = c_puct;
  f->vl = vl;
  f->expand_policy = expand_policy;
  f->sign_mode = sign_mode;
  f->logit_scale = logit_scale;
  f->eps = eps;
}

void orc_set_roots(orc_forest *f, const uint64_t *keys, const uint32_t *legal,
                   const double *noise) {
  memcpy(f->root_keys, keys, sizeof(uint64_t) * (size_t)f->T);
  if (legal) memcpy(f->root_legal, legal, sizeof(uint32_t) * (size_t)f->T * f->legal_words);
  free(f->root_noise);
  f->root_noise = NULL;
  if (noise) {
    f->root_noise = (double *)malloc(sizeof(double) * (size_t)f->T * f->A);
    memcpy(f->root_noise, noise, sizeof(double) * (size_t)f->T * f->A);
  }
}

/* Gomoku rules for the leaves of later waves: boards [T*A] (0 empty, 1/2 stones) are the root
   positions; root_player[T] is the player of the first path move, or NULL for 1 when the root
   board holds an even number of stones, else 2 (mcts.py:1506).  enable=0 switches them off. */
void orc_set_gomoku_rules(orc_forest *f, int enable, int rule, const int8_t *boards,
                          const int32_t *root_player) {
  free(f->root_boards);
  free(f->root_player);
  f->root_boards = NULL;
  f->root_player = NULL;
  f->rules_on = 0;
  if (!enable) return;
  f->rule = rule;
  f->root_boards = (int8_t *)malloc((size_t)f->T * f->A);
  f->root_player = (int32_t *)malloc(sizeof(int32_t) * (size_t)f->T);
  memcpy(f->root_boards, boards, (size_t)f->T * f->A);
  for (int t = 0; t < f->T; ++t) {
    if (root_player) {
      f->root_player[t] = root_player[t];
    } else {
      int stones = 0;
      for (int a = 0; a < f->A; ++a) stones += boards[(size_t)t * f->A + a] != 0;
      f->root_player[t] = stones % 2 == 0 ? 1 : 2;
    }
  }
  f->rules_on = 1;
}

/* Go rules for every wave's leaves: boards [T*(A-1)] (0 empty, 1/2 stones) are the root
   positions, root_player[T] the player of the first path move (NULL: 1 for an even stone
   count, else 2), root_passes[T] the root's trailing passes (NULL: 0), root_ko[T] the root's
   ko point or -1 (NULL: none).  flags: ORC_GO_KO, ORC_GO_SUICIDE.  enable=0 switches them
   off.  The rules are stated at go_legal_list and go_terminal below. */
void orc_set_go_rules(orc_forest *f, int enable, int flags, const int8_t *boards,
                      const int32_t *root_player, const int32_t *root_passes,
                      const int32_t *root_ko) {
  free(f->go_boards);
  free(f->go_player);
  free(f->go_passes);
  free(f->go_ko);
  f->go_boards = NULL;
  f->go_player = f->go_passes = f->go_ko = NULL;
  f->go_on = 0;
  if (!enable) return;
  const int cells = f->A - 1;
  f->go_flags = flags;
  f->go_boards = (int8_t *)malloc((size_t)f->T * cells);
  memcpy(f->go_boards, boards, (size_t)f->T * cells);
  f->go_player = (int32_t *)malloc(sizeof(int32_t) * (size_t)f->T);
  f->go_passes = (int32_t *)malloc(sizeof(int32_t) * (size_t)f->T);
  f->go_ko = (int32_t *)malloc(sizeof(int32_t) * (size_t)f->T);
  for (int t = 0; t < f->T; ++t) {
    int stones = 0;
    for (int c = 0; c < cells; ++c) stones += boards[(size_t)t * cells + c] != 0;
    f->go_player[t] = root_player ? root_player[t] : (stones % 2 == 0 ? 1 : 2);
    f->go_passes[t] = root_passes ? root_passes[t] : 0;
    f->go_ko[t] = root_ko ? root_ko[t] : -1;
  }
  f->go_on = 1;
}

/* the Go position after the path moves acts[0..np): the root board, move q played by the root's
   player when q is even, else by the other; a pass (action A-1) places no stone and no stone
   is ever captured (GPUGameStates.apply_moves, python/mcts/gpu/gpu_game_states.py:430-441) */
static void go_board(const orc_forest *f, int t, const int *acts, int np, int8_t *board) {
  const int cells = f->A - 1;
  memcpy(board, f->go_boards + (size_t)t * cells, (size_t)cells);
  const int rp = f->go_player[t];
  for (int q = 0; q < np; ++q)
    if (acts[q] >= 0 && acts[q] < cells) board[acts[q]] = (int8_t)(q % 2 == 0 ? rp : 3 - rp);
}

/* legal moves of the position after acts, ascending: every empty point that is not the root's
   ko point (with ORC_GO_KO; get_legal_moves_mask, gpu_game_states.py:373-395, excludes the
   state's ko point, and clone_states, :336-337, hands it on to every descendant unchanged)
   and, with ORC_GO_SUICIDE, has an empty orthogonal neighbour (gpu_get_legal_moves,
   python/mcts/gpu/go_kernels.py:46-110: a 4-neighbour count of empty points > 0); then the
   pass, always legal */
static int go_legal_list(const orc_forest *f, int t, const int *acts, int np, int *list) {
  int8_t board[8192];
  const int cells = f->A - 1;
  int bs = 0;
  while ((bs + 1) * (bs + 1) <= cells) ++bs;
  go_board(f, t, acts, np, board);
  const int ko = (f->go_flags & ORC_GO_KO) ? f->go_ko[t] : -1;
  int n = 0;
  for (int c = 0; c < cells; ++c) {
    if (board[c] != 0 || c == ko) continue;
    if (f->go_flags & ORC_GO_SUICIDE) {
      const int r = c / bs, k = c % bs;
      const int up = r > 0 && board[c - bs] == 0;
      const int down = r < bs - 1 && board[c + bs] == 0;
      const int left = k > 0 && board[c - 1] == 0;
      const int right = k < bs - 1 && board[c + 1] == 0;
      if (!(up || down || left || right)) continue;
    }
    list[n++] = c;
  }
  list[n++] = cells;
  return n;
}

/* gpu_check_terminal_states (go_kernels.py:17-44): two consecutive passes (the trailing passes
   of the path, plus the root's own when every path move is a pass) or no empty point.  The
   root itself (np = 0) is never terminal. */
static int go_terminal(const orc_forest *f, int t, const int *acts, int np) {
  if (np < 1) return ORC_TERM_NONE;
  const int cells = f->A - 1;
  int trail = 0;
  while (trail < np && acts[np - 1 - trail] == cells) ++trail;
  if (trail == np) trail += f->go_passes[t];
  int8_t board[8192];
  go_board(f, t, acts, np, board);
  int empty = 0;
  for (int c = 0; c < cells; ++c) empty += board[c] == 0;
  return (trail >= 2 || empty == 0) ? ORC_TERM_END : ORC_TERM_NONE;
}

/* the Go rules of one position, for the known-answer tests: legal list and terminal code */
int orc_go_leaf_rules(const orc_forest *f, int t, const int *acts, int np, int *list,
                      int *term) {
  if (!f->go_on) return -1;
  *term = go_terminal(f, t, acts, np);
  return go_legal_list(f, t, acts, np, list);
}

/* FastTerminalChecker._check_gomoku_terminal_cpu without last_move
   (python/mcts/utils/fast_terminal_check.py:132-232), literally: for each occupied cell in
   row-major order, the horizontal, vertical, '\' and '/' windows of five starting there are
   tried in turn; a renju overline of player 1 skips the rest of the cell (the reference's
   `continue` of its column loop); the first full window returns its player.  A full board
   without a five is a draw.  Returns the player (1, 2), ORC_TERM_DRAW or ORC_TERM_NONE. */
int orc_gomoku_terminal(const int8_t *board, int bs, int rule) {
  const int renju = rule == ORC_RULE_RENJU;
#define CELL(r, c) board[(r) * bs + (c)]
  for (int row = 0; row < bs; ++row) {
    for (int col = 0; col < bs; ++col) {
      const int player = CELL(row, col);
      if (player == 0) continue;
      int skip = 0;
      /* horizontal */
      if (col <= bs - 5) {
        int all = 1;
        for (int i = 0; i < 5; ++i) all &= CELL(row, col + i) == player;
        if (all) {
          if (renju && player == 1) {
            if (col + 5 < bs && CELL(row, col + 5) == player) skip = 1;
            else if (col > 0 && CELL(row, col - 1) == player) skip = 1;
          }
          if (skip) continue;
          return player;
        }
      }
      /* vertical */
      if (row <= bs - 5) {
        int all = 1;
        for (int i = 0; i < 5; ++i) all &= CELL(row + i, col) == player;
        if (all) {
          if (renju && player == 1) {
            if (row + 5 < bs && CELL(row + 5, col) == player) skip = 1;
            else if (row > 0 && CELL(row - 1, col) == player) skip = 1;
          }
          if (skip) continue;
          return player;
        }
      }
      /* diagonal down-right */
      if (row <= bs - 5 && col <= bs - 5) {
        int all = 1;
        for (int i = 0; i < 5; ++i) all &= CELL(row + i, col + i) == player;
        if (all) {
          if (renju && player == 1) {
            if (row + 5 < bs && col + 5 < bs && CELL(row + 5, col + 5) == player) skip = 1;
            else if (row > 0 && col > 0 && CELL(row - 1, col - 1) == player) skip = 1;
          }
          if (skip) continue;
          return player;
        }
      }
      /* diagonal down-left */
      if (row <= bs - 5 && col >= 4) {
        int all = 1;
        for (int i = 0; i < 5; ++i) all &= CELL(row + i, col - i) == player;
        if (all) {
          if (renju && player == 1) {
            if (row + 5 < bs && col - 5 >= 0 && CELL(row + 5, col - 5) == player) skip = 1;
            else if (row > 0 && col < bs - 1 && CELL(row - 1, col + 1) == player) skip = 1;
          }
          if (skip) continue;
          return player;
        }
      }
    }
  }
  for (int i = 0; i < bs * bs; ++i)
    if (board[i] == 0) return ORC_TERM_NONE;
  return ORC_TERM_DRAW;
#undef CELL
}

/* terminal code of a leaf reached by the path moves acts[0..np) (np >= 1) */
static int leaf_terminal(const orc_forest *f, int t, const int *acts, int np) {
  int8_t board[8192];
  const int A = f->A;
  int bs = 0;
  while ((bs + 1) * (bs + 1) <= A) ++bs;
  memcpy(board, f->root_boards + (size_t)t * A, (size_t)A);
  const int rp = f->root_player[t];
  for (int q = 0; q < np; ++q)
    if (acts[q] >= 0 && acts[q] < A) board[acts[q]] = (int8_t)(q % 2 == 0 ? rp : 3 - rp);
  return orc_gomoku_terminal(board, bs, f->rule);
}

/* ---- per-move root operations ------------------------------------------------------------
   Restated from their specification: the visit-count policy (mcts.py:1069-1137), move
   selection with a temperature (mcts.py:1167-1203, np.random.choice semantics) and root
   Dirichlet noise, with the draws taken from a SplitMix64 stream keyed by (seed, counter, tree,
   item).  Gamma variates by Marsaglia and Tsang (ACM TOMS 26(3), 2000; shape < 1 boosted by
   U^(1/alpha)), normal variates by Marsaglia's polar method, log and exp by textbook methods
   (Cody-Waite reduction + Taylor polynomial; exponent split + atanh series), all in IEEE double
   with +, -, *, /, sqrt and floor only. */
static double orc_pow2i(int k) {
  const uint64_t b = (uint64_t)(k + 1023) << 52;
  double d;
  memcpy(&d, &b, 8);
  return d;
}

double orc_exp_d(double x) {
  static const double ln2_hi = 0x1.62e42feep-1, ln2_lo = 0x1.a39ef35793c76p-33;
  if (x < -745.0) return 0.0;
  if (x > 709.0) return INFINITY;
  const double kf = floor(x * (1.0 / 0.6931471805599453) + 0.5);
  const int k = (int)kf;
  const double r = (x - kf * ln2_hi) - kf * ln2_lo;
  /* e^r = sum r^n / n!, n = 0..13, by Horner from the top */
  static const double fact[14] = {1.0, 1.0, 2.0, 6.0, 24.0, 120.0, 720.0, 5040.0, 40320.0,
                                  362880.0, 3628800.0, 39916800.0, 479001600.0, 6227020800.0};
  double p = 1.0 / fact[13];
  for (int n = 12; n >= 0; --n) p = p * r + 1.0 / fact[n];
  if (k < -1021) return (p * orc_pow2i(k + 1000)) * orc_pow2i(-1000);
  return p * orc_pow2i(k);
}

double orc_log_d(double x) {
  static const double ln2_hi = 0x1.62e42feep-1, ln2_lo = 0x1.a39ef35793c76p-33;
  uint64_t b;
  memcpy(&b, &x, 8);
  int e = 0;
  if ((b >> 52) == 0) {
    x = x * 0x1p54;
    memcpy(&b, &x, 8);
    e = -54;
  }
  e += (int)((b >> 52) & 0x7FF) - 1023;
  const uint64_t mb = (b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull;
  double m;
  memcpy(&m, &mb, 8);
  if (m > 0x1.6a09e667f3bcdp+0) {
    m = m * 0.5;
    e += 1;
  }
  const double s = (m - 1.0) / (m + 1.0);
  const double z = s * s;
  /* atanh series: log m = 2 s (1 + z/3 + z^2/5 + ... + z^11/23) */
  double p = 1.0 / 23.0;
  for (int n = 21; n >= 1; n -= 2) p = p * z + 1.0 / (double)n;
  const double ed = (double)e;
  return (ed * ln2_lo + 2.0 * s * p) + ed * ln2_hi;
}

typedef struct {
  uint64_t base, j;
} orc_stream;

static orc_stream orc_make_stream(uint64_t seed, uint64_t counter, int t, int item) {
  orc_stream s;
  const uint64_t tag = ((uint64_t)(uint32_t)t << 32) | (uint32_t)item;
  s.base = orc_splitmix64(orc_splitmix64(orc_splitmix64(seed) ^ counter) ^ tag);
  s.j = 0;
  return s;
}

static double orc_uniform_open(orc_stream *s) {
  const uint64_t b = orc_splitmix64(s->base + s->j * GOLDEN);
  s->j += 1;
  return ((double)(b >> 11) + 0.5) * 0x1p-53;
}

static double orc_normal_polar(orc_stream *s) {
  for (;;) {
    const double u = 2.0 * orc_uniform_open(s) - 1.0;
    const double v = 2.0 * orc_uniform_open(s) - 1.0;
    const double q = u * u + v * v;
    if (q > 0.0 && q < 1.0) return u * sqrt(-2.0 * orc_log_d(q) / q);
  }
}

static double orc_gamma_s(double alpha, orc_stream *s) {
  const int boost = alpha < 1.0;
  const double a = boost ? alpha + 1.0 : alpha;
  const double d = a - 1.0 / 3.0;
  const double c = 1.0 / sqrt(9.0 * d);
  double x, v;
  for (;;) {
    do {
      x = orc_normal_polar(s);
      v = 1.0 + c * x;
    } while (v <= 0.0);
    v = v * v * v;
    const double u = orc_uniform_open(s);
    const double x2 = x * x;
    if (u < 1.0 - 0.0331 * (x2 * x2)) break;
    if (orc_log_d(u) < 0.5 * x2 + d * (1.0 - v + orc_log_d(v))) break;
  }
  double g = d * v;
  if (boost) g = g * orc_exp_d(orc_log_d(orc_uniform_open(s)) / alpha);
  return g;
}

double orc_gamma(double alpha, uint64_t seed, uint64_t counter, int t, int item) {
  orc_stream s = orc_make_stream(seed, counter, t, item);
  return orc_gamma_s(alpha, &s);
}

/* Dirichlet(alpha) over the L legal root actions of tree t into row[0..A) (zeros past L) */
void orc_root_dirichlet(const orc_forest *f, int t, double alpha, uint64_t seed,
                        uint64_t counter, double *row) {
  int L = 0;
  if (f->game == ORC_GAME_SPARSE) {
    L = sparse_count(f, f->root_keys[t]);
  } else {
    for (int w = 0; w < f->legal_words; ++w)
      L += __builtin_popcount(f->root_legal[(size_t)t * f->legal_words + w]);
  }
  for (int i = 0; i < f->A; ++i) row[i] = 0.0;
  for (int i = 0; i < L; ++i) row[i] = orc_gamma(alpha, seed, counter, t, i);
  const double S = orc_sum64d(row, L);
  for (int i = 0; i < L; ++i) row[i] = S > 0.0 ? row[i] / S : 1.0 / (double)L;
}

/* select_action on one policy row: first maximum at temperature 0; otherwise the normalised
   cumulative sums of p^(1/T) / sum against u in [0, 1) (first entry above u) */
int orc_sample_action(const double *p, int A, double temperature, uint64_t seed,
                      uint64_t counter, int t) {
  if (temperature == 0.0) {
    int best = 0;
    for (int a = 1; a < A; ++a)
      if (p[a] > p[best]) best = a;
    return best;
  }
  const double inv_t = 1.0 / temperature;
  const int unit = temperature == 1.0;
  double *w = (double *)malloc(sizeof(double) * (size_t)A);
  double S = 0.0;
  for (int a = 0; a < A; ++a) {
    w[a] = p[a] > 0.0 ? (unit ? p[a] : orc_exp_d(orc_log_d(p[a]) * inv_t)) : 0.0;
    S = S + w[a];
  }
  double last = 0.0;
  for (int a = 0; a < A; ++a) last = last + w[a] / S;
  const orc_stream st = orc_make_stream(seed, counter, t, -1);
  const double u = (double)(orc_splitmix64(st.base) >> 11) * 0x1p-53;
  double c = 0.0;
  int pick = A - 1;
  for (int a = 0; a < A; ++a) {
    c = c + w[a] / S;
    if (c / last > u) {
      pick = a;
      break;
    }
  }
  free(w);
  return pick;
}

/* CSRTree.shift_root (python/mcts/gpu/csr_tree.py:1020-1229) on tree t: breadth-first queue
   from node r over the children in row order, visited-marked; new index = queue position;
   N, W, P, expanded flag and action copied, parents remapped (root: -1, action -1); the edge
   arrays rebuilt node by node in the new order.  Returns the number of kept nodes (the tree
   is unchanged and 0 is returned when r is 0 or out of range). */
int orc_shift_root(orc_forest *f, int t, int r) {
  const size_t b = (size_t)t * f->cap;
  const int n_old = f->num_nodes[t];
  if (r <= 0 || r >= n_old) return 0;
  int32_t *queue = (int32_t *)malloc(sizeof(int32_t) * (size_t)n_old);
  int32_t *new_of = (int32_t *)malloc(sizeof(int32_t) * (size_t)n_old);
  if (!queue || !new_of) {
    free(queue);
    free(new_of);
    return 0;
  }
  for (int i = 0; i < n_old; ++i) new_of[i] = -1;
  int kept = 0, rd = 0;
  queue[kept] = r;
  new_of[r] = kept++;
  while (rd < kept) {
    const int cur = queue[rd++];
    if (f->first[b + cur] < 0) continue;
    for (int j = 0; j < f->nchild[b + cur]; ++j) {
      const int c = f->children[b + f->first[b + cur] + j];
      if (new_of[c] < 0) {
        new_of[c] = kept;
        queue[kept++] = c;
      }
    }
  }
  /* copies of the kept nodes in the new order, and their children's new ids row by row,
     all read before the tree is overwritten */
  int32_t *N = (int32_t *)malloc(4 * (size_t)kept), *par = (int32_t *)malloc(4 * (size_t)kept);
  int32_t *act = (int32_t *)malloc(4 * (size_t)kept), *kids = (int32_t *)malloc(4 * (size_t)kept);
  int32_t *kid_new = (int32_t *)malloc(4 * (size_t)kept);
  float *W = (float *)malloc(4 * (size_t)kept), *P = (float *)malloc(4 * (size_t)kept);
  uint8_t *ex = (uint8_t *)malloc((size_t)kept);
  int nk = 0;
  for (int i = 0; i < kept; ++i) {
    const int o = queue[i];
    N[i] = f->N[b + o];
    W[i] = f->W[b + o];
    P[i] = f->P[b + o];
    ex[i] = f->expanded[b + o];
    act[i] = f->action[b + o];
    par[i] = f->parent[b + o] >= 0 ? new_of[f->parent[b + o]] : -1;
    kids[i] = 0;
    if (f->first[b + o] < 0) continue;
    for (int j = 0; j < f->nchild[b + o]; ++j) {
      const int c = new_of[f->children[b + f->first[b + o] + j]];
      if (c >= 0 && nk < kept) { /* a child reached earlier from another row is not kept twice */
        kid_new[nk++] = c;
        kids[i] += 1;
      }
    }
  }
  par[0] = -1;
  act[0] = -1;
  int e = 0;
  for (int i = 0; i < kept; ++i) {
    f->N[b + i] = N[i];
    f->W[b + i] = W[i];
    f->P[b + i] = P[i];
    f->parent[b + i] = par[i];
    f->action[b + i] = act[i];
    f->expanded[b + i] = ex[i];
    f->first[b + i] = kids[i] > 0 ? e : -1;
    f->nchild[b + i] = kids[i];
    for (int j = 0; j < kids[i]; ++j, ++e) {
      f->children[b + e] = kid_new[e];
      f->child_actions[b + e] = act[kid_new[e]];
    }
  }
  /* the reference resets the tree before writing the kept nodes back: clear the rest */
  for (int i = kept; i < n_old; ++i) {
    f->N[b + i] = 0;
    f->W[b + i] = 0.0f;
    f->P[b + i] = 0.0f;
    f->parent[b + i] = -1;
    f->first[b + i] = -1;
    f->nchild[b + i] = 0;
    f->action[b + i] = 0;
    f->expanded[b + i] = 0;
  }
  f->num_nodes[t] = kept;
  f->num_edges[t] = e;
  free(N);
  free(par);
  free(act);
  free(kids);
  free(kid_new);
  free(W);
  free(P);
  free(ex);
  free(queue);
  free(new_of);
  return kept;
}

/* CythonLockFreeTree.__cinit__ / reset: one node, N[0]=1, P[0]=1 (pyx:92-100, 537-558) */
void orc_reset_tree(orc_forest *f, int t) {
  size_t b = (size_t)t * f->cap;
  for (int i = 0; i < f->cap; ++i) {
    f->N[b + i] = 0;
    f->W[b + i] = 0.0f;
    f->P[b + i] = 0.0f;
    f->parent[b + i] = -1;
    f->first[b + i] = -1;
    f->nchild[b + i] = 0;
    f->action[b + i] = 0;
    f->expanded[b + i] = 0;
  }
  f->action[b] = -1;
  f->num_nodes[t] = 1;
  f->num_edges[t] = 0;
  f->N[b] = 1;
  f->P[b] = 1.0f;
}

/* ---- tree operations ------------------------------------------------------------------- */

/* select_best_child_nogil (pyx:421-464), literally: first child with N==0 wins, else the
   strict-'>' argmax of q + exploration starting from -1e9 */
int orc_best_child(const orc_forest *f, int t, int node) {
  const size_t b = (size_t)t * f->cap;
  if (node < 0 || node >= f->num_nodes[t]) return -1;
  const int first_child = f->first[b + node];
  const int n_children = f->nchild[b + node];
  if (n_children == 0 || first_child < 0) return -1;
  const int parent_visits = f->N[b + node];
  if (parent_visits == 0) return -1;
  const float sqrt_parent = (float)sqrt((double)(float)parent_visits);
  int best_child = -1;
  float best_ucb = -1e9f;
  for (int i = 0; i < n_children; ++i) {
    if (first_child + i >= f->cap) break;
    const int child_idx = f->children[b + first_child + i];
    if (child_idx < 0 || child_idx >= f->num_nodes[t]) continue;
    const int child_visits = f->N[b + child_idx];
    if (child_visits == 0) return child_idx;
    const float q_value = f->W[b + child_idx] / (child_visits + f->vl);
    const float exploration = f->c_puct * f->P[b + child_idx] * sqrt_parent / (1 + child_visits);
    const float ucb = q_value + exploration;
    if (ucb > best_ucb) {
      best_ucb = ucb;
      best_child = child_idx;
    }
  }
  return best_child;
}

/* select_path (pyx:177-202) for simulation s of the current wave.  Canonical depth limit:
   a node reached at depth max_depth-1 ends the path (the reference's loop exit returns a
   node outside the path there). */
static void select_path(orc_forest *f, int t, int s, int max_depth) {
  const size_t b = (size_t)t * f->cap;
  const int vli = (int)f->vl;
  int32_t *path = f->paths + ((size_t)t * f->max_wave + s) * f->max_depth;
  int cur = 0, depth = 0;
  for (;;) {
    path[depth] = cur;
    f->N[b + cur] += vli;
    if (!f->expanded[b + cur] || f->nchild[b + cur] == 0 || depth == max_depth - 1) break;
    const int c = orc_best_child(f, t, cur);
    if (c < 0) break;
    cur = c;
    ++depth;
  }
  f->path_len[(size_t)t * f->max_wave + s] = depth + 1;
  f->leaves[(size_t)t * f->max_wave + s] = cur;
}

static int path_actions(const orc_forest *f, int t, int s, int *acts) {
  const size_t b = (size_t)t * f->cap;
  const int32_t *path = f->paths + ((size_t)t * f->max_wave + s) * f->max_depth;
  const int L = f->path_len[(size_t)t * f->max_wave + s];
  for (int d = 1; d < L; ++d) acts[d - 1] = f->action[b + path[d]];
  return L - 1;
}

/* unique leaves in first-occurrence order, keys and legal counts */
static void leaves_info(orc_forest *f, int t, int W) {
  const size_t wb = (size_t)t * f->max_wave;
  const size_t b = (size_t)t * f->cap;
  int nu = 0;
  int acts[256], list[8192];
  for (int s = 0; s < W; ++s) {
    const int leaf = f->leaves[wb + s];
    int u = f->seen[b + leaf];
    if (u < 0) {
      u = nu++;
      f->seen[b + leaf] = u;
      f->uleaf[wb + u] = leaf;
      f->ufirst[wb + u] = s;
    }
    f->sim_uid[wb + s] = u;
  }
  for (int u = 0; u < nu; ++u) f->seen[b + f->uleaf[wb + u]] = -1;
  f->ucount[t] = nu;
  for (int u = 0; u < nu; ++u) {
    const int s0 = f->ufirst[wb + u];
    const int np = path_actions(f, t, s0, acts);
    uint64_t k = f->root_keys[t];
    for (int q = 0; q < np; ++q) k = orc_child_key(k, acts[q]);
    f->ukey[wb + u] = k;
    f->ulegal[wb + u] = legal_list(f, t, acts, np, k, list);
    f->uterm[wb + u] = ORC_TERM_NONE;
    if (f->rules_on && np >= 1) {  /* the root itself is never flagged */
      f->uterm[wb + u] = leaf_terminal(f, t, acts, np);
      if (f->uterm[wb + u] != ORC_TERM_NONE) f->ulegal[wb + u] = 0;
    }
    if (f->go_on) {
      f->uterm[wb + u] = go_terminal(f, t, acts, np);
      if (f->uterm[wb + u] != ORC_TERM_NONE) f->ulegal[wb + u] = 0;
    }
  }
}

/* synthetic evaluator: softmax of scale*z over the legal actions; v = 2u-1 */
static void synth_eval(orc_forest *f, int t) {
  const size_t wb = (size_t)t * f->max_wave;
  int acts[256], list[8192];
  float e[8192];
  for (int u = 0; u < f->ucount[t]; ++u) {
    const int s0 = f->ufirst[wb + u];
    const int np = path_actions(f, t, s0, acts);
    const uint64_t k = f->ukey[wb + u];
    const int n = legal_list(f, t, acts, np, k, list);
    float *row = f->policy + (wb + u) * (size_t)f->A; /* only the legal slots are written */
    float mx = -INFINITY;
    for (int i = 0; i < n; ++i) {
      const float z = f->logit_scale * orc_key_normal(k, list[i]);
      if (z > mx) mx = z;
    }
    for (int i = 0; i < n; ++i) e[i] = orc_exp_cw(f->logit_scale * orc_key_normal(k, list[i]) - mx);
    const float S = orc_sum64(e, n);
    for (int i = 0; i < n; ++i) row[list[i]] = e[i] / S;
    f->values[wb + u] = orc_key_value(k);
  }
}

static int pw_root_mc(int L, int N0) {
  int m1 = (int)(10.0 * sqrt((double)N0)) + 1;
  if (L < m1) m1 = L;
  int mc = m1 < 15 ? m1 : 15;
  return mc > 5 ? mc : 5;
}

/* expansion of the wave's unique leaves in first-occurrence order
   (optimized_wave_search.py:367-438 + expand_node pyx:232-277) */
static void expand_leaves(orc_forest *f, int t, int W) {
  const size_t b = (size_t)t * f->cap;
  const size_t wb = (size_t)t * f->max_wave;
  const int vli = (int)f->vl;
  int acts[256], list[8192];
  float pf[8192];
  double pd[8192];
  int chosen[8192];
  for (int u = 0; u < f->ucount[t]; ++u) {
    const int leaf = f->uleaf[wb + u];
    f->uexpanded[wb + u] = 0;
    if (f->expanded[b + leaf]) continue;
    if (f->uterm[wb + u] != ORC_TERM_NONE) continue; /* terminal: not expanded (:374-376) */
    const int s0 = f->ufirst[wb + u];
    const int np = path_actions(f, t, s0, acts);
    const int n = legal_list(f, t, acts, np, f->ukey[wb + u], list);
    if (n == 0) continue;
    const float *row = f->policy + (wb + u) * (size_t)f->A;
    /* legal_priors = policy[legal] / sum */
    for (int i = 0; i < n; ++i) pf[i] = row[list[i]];
    const float S = orc_sum64(pf, n);
    for (int i = 0; i < n; ++i) pf[i] = pf[i] / S;
    /* Dirichlet at the root: float32 (1-eps)*p promoted to double, + eps*noise */
    const int noisy = leaf == 0 && f->root_noise != NULL && f->eps > 0.0;
    const float w32 = (float)(1.0 - f->eps);
    for (int i = 0; i < n; ++i)
      pd[i] = noisy ? (double)(w32 * pf[i]) + f->eps * f->root_noise[(size_t)t * f->A + i]
                    : (double)pf[i];
    /* chosen list (ascending actions) */
    int nch = n;
    for (int i = 0; i < n; ++i) chosen[i] = i;
    int k = n;
    if (f->expand_policy == ORC_EXPAND_REFERENCE_PW) {
      const int sel = leaf == 0 ? pw_root_mc(n, f->N[b] - vli * W) : 3;
      if (n > sel) {
        /* top-sel by (prior desc, action asc), kept in ascending order */
        static __thread int taken[8192];
        for (int i = 0; i < n; ++i) taken[i] = 0;
        for (int it = 0; it < sel; ++it) {
          int bi = -1;
          for (int i = 0; i < n; ++i)
            if (!taken[i] && (bi < 0 || pd[i] > pd[bi])) bi = i;
          taken[bi] = 1;
        }
        nch = 0;
        for (int i = 0; i < n; ++i)
          if (taken[i]) chosen[nch++] = i;
        if (noisy) {
          double v[64];
          for (int j = 0; j < nch; ++j) v[j] = pd[chosen[j]];
          const double Sd = orc_sum64d(v, nch);
          for (int j = 0; j < nch; ++j) pd[chosen[j]] = pd[chosen[j]] / Sd;
        } else {
          float v[64];
          for (int j = 0; j < nch; ++j) v[j] = (float)pd[chosen[j]];
          const float Sf = orc_sum64(v, nch);
          for (int j = 0; j < nch; ++j) pd[chosen[j]] = (double)((float)pd[chosen[j]] / Sf);
        }
      }
      k = leaf == 0 ? (nch < 8 ? nch : 8) : nch;
    }
    if (k > 512) continue; /* row limit of the device library (refused there as well) */
    /* expand_node: contiguous nodes and edges, refuse when full */
    if (f->num_edges[t] + k > f->cap) continue;
    if (f->num_nodes[t] + k > f->cap) continue;
    const int first_edge = f->num_edges[t];
    f->num_edges[t] += k;
    const int first_child = f->num_nodes[t];
    f->num_nodes[t] += k;
    f->first[b + leaf] = first_edge;
    f->nchild[b + leaf] = k;
    f->expanded[b + leaf] = 1;
    for (int j = 0; j < k; ++j) {
      const int c = first_child + j;
      f->parent[b + c] = leaf;
      f->P[b + c] = (float)pd[chosen[j]];
      f->action[b + c] = list[chosen[j]];
      f->N[b + c] = 0;
      f->W[b + c] = 0.0f;
      f->first[b + c] = -1;
      f->nchild[b + c] = 0;
      f->expanded[b + c] = 0;
      f->children[b + first_edge + j] = c;
      f->child_actions[b + first_edge + j] = list[chosen[j]];
    }
    f->uexpanded[wb + u] = k;
  }
}

/* backup of every simulation in order: N = N - VL + 1, W += sign * v along the path */
static void backup(orc_forest *f, int t, int W) {
  const size_t b = (size_t)t * f->cap;
  const size_t wb = (size_t)t * f->max_wave;
  const int vli = (int)f->vl;
  for (int s = 0; s < W; ++s) {
    const float v = f->values[wb + f->sim_uid[wb + s]];
    const int L = f->path_len[wb + s];
    const int32_t *path = f->paths + (wb + s) * (size_t)f->max_depth;
    for (int d = 0; d < L; ++d) {
      const int x = path[d];
      const int e = f->sign_mode == ORC_SIGN_LEAF_POSITIVE ? (L - 1 - d) : d;
      f->N[b + x] = f->N[b + x] - vli + 1;
      f->W[b + x] += (e & 1) ? -v : v;
    }
  }
}

/* ---- waves and searches ---------------------------------------------------------------- */

/* phase-wise wave API (tests compare after each phase) */
void orc_wave_select(orc_forest *f, int t, int W, int max_depth) {
  for (int s = 0; s < W; ++s) select_path(f, t, s, max_depth);
  leaves_info(f, t, W);
}
void orc_wave_evaluate(orc_forest *f, int t) { synth_eval(f, t); }
void orc_wave_expand(orc_forest *f, int t, int W) { expand_leaves(f, t, W); }
void orc_wave_backup(orc_forest *f, int t, int W) { backup(f, t, W); }

/* one wave of tree t; replay_policy/values (rows of the unique leaves) replace the synthetic
   evaluator when given */
void orc_wave(orc_forest *f, int t, int W, int max_depth, const float *replay_policy,
              const float *replay_values) {
  orc_wave_select(f, t, W, max_depth);
  const size_t wb = (size_t)t * f->max_wave;
  if (replay_policy) {
    const int nu = f->ucount[t];
    memcpy(f->policy + wb * (size_t)f->A, replay_policy, sizeof(float) * (size_t)nu * f->A);
    memcpy(f->values + wb, replay_values, sizeof(float) * (size_t)nu);
  } else {
    synth_eval(f, t);
  }
  expand_leaves(f, t, W);
  backup(f, t, W);
}

/* MCTS.search for tree t with the synthetic evaluator: reset, root expansion (a one-simulation
   wave: path [0]), then waves of min(max_wave, n - done) simulations */
void orc_search_tree(orc_forest *f, int t, int num_sims, int wave, int max_depth) {
  orc_reset_tree(f, t);
  orc_wave(f, t, 1, max_depth, NULL, NULL);
  int done = 0;
  while (done < num_sims) {
    int w = num_sims - done;
    if (w > wave) w = wave;
    orc_wave(f, t, w, max_depth, NULL, NULL);
    done += w;
  }
}

typedef struct {
  orc_forest *f;
  int t0, t1, num_sims, wave, max_depth;
} orc_job;

static void *orc_worker(void *arg) {
  orc_job *j = (orc_job *)arg;
  for (int t = j->t0; t < j->t1; ++t) orc_search_tree(j->f, t, j->num_sims, j->wave, j->max_depth);
  return NULL;
}

/* all trees, distributed over nthreads threads (trees are independent) */
int orc_search(orc_forest *f, int num_sims, int wave, int max_depth, int nthreads) {
  if (nthreads <= 1) {
    for (int t = 0; t < f->T; ++t) orc_search_tree(f, t, num_sims, wave, max_depth);
    return 0;
  }
  if (nthreads > f->T) nthreads = f->T;
  pthread_t th[256];
  orc_job jobs[256];
  if (nthreads > 256) nthreads = 256;
  for (int i = 0; i < nthreads; ++i) {
    jobs[i].f = f;
    jobs[i].t0 = (int)((long)f->T * i / nthreads);
    jobs[i].t1 = (int)((long)f->T * (i + 1) / nthreads);
    jobs[i].num_sims = num_sims;
    jobs[i].wave = wave;
    jobs[i].max_depth = max_depth;
    if (pthread_create(&th[i], NULL, orc_worker, &jobs[i]) != 0) return -1;
  }
  for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
  return 0;
}

/* accessors for ctypes */
#define ORC_GET(name, type) \
  type *orc_##name(orc_forest *f) { return f->name; }
ORC_GET(N, int32_t)
ORC_GET(W, float)
ORC_GET(P, float)
ORC_GET(parent, int32_t)
ORC_GET(first, int32_t)
ORC_GET(nchild, int32_t)
ORC_GET(action, int32_t)
ORC_GET(expanded, uint8_t)
ORC_GET(children, int32_t)
ORC_GET(child_actions, int32_t)
ORC_GET(num_nodes, int32_t)
ORC_GET(num_edges, int32_t)
ORC_GET(paths, int32_t)
ORC_GET(path_len, int32_t)
ORC_GET(leaves, int32_t)
ORC_GET(sim_uid, int32_t)
ORC_GET(uleaf, int32_t)
ORC_GET(ufirst, int32_t)
ORC_GET(ucount, int32_t)
ORC_GET(ukey, uint64_t)
ORC_GET(ulegal, int32_t)
ORC_GET(uexpanded, int32_t)
ORC_GET(uterm, int32_t)
ORC_GET(policy, float)
ORC_GET(values, float)
