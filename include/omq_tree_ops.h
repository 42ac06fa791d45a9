/*
 * omq_tree_ops.h -- C ABI of the MI355X (gfx950) wave-MCTS tree-operation library
 * (libomq_tree_ops.so).
 *
 * The library implements the tree operations of a batched, wave-parallel MCTS over
 * CSR trees: PUCT selection with virtual loss, leaf expansion that appends children
 * to the CSR arrays, and backup along the selected paths.  Every pointer in the
 * structures below is a DEVICE pointer (memory owned by the caller, e.g. torch
 * tensors); every entry point launches work on the HIP stream it is given and
 * returns without synchronising.  Entry points return 0 on success and a negative
 * OMQ_E_* code on a rejected argument or a failed launch; omq_last_error() then
 * holds a message for the calling thread.
 *
 * Tree layout (per tree t, node ids local to the tree, node i of tree t stored at
 * index t*capacity + i in every node array):
 *   visit_counts[i]  int32   N   (includes in-flight virtual loss between select and backup)
 *   value_sums[i]    float   W
 *   priors[i]        float   P
 *   parents[i]       int32   parent node, -1 for the root
 *   first_child[i]   int32   CSR row offset: edge index of the first child, -1 if none
 *   num_children[i]  int32   CSR row length
 *   actions[i]       int32   action that leads from the parent to node i, -1 for the root
 *   num_nodes[t]     int32   allocated nodes (the number of edges is num_nodes-1)
 * Children are allocated by a bump pointer in blocks, and nodes and edges are bumped by
 * the same amount, so edge e always points at node e+1.  The CSR column array is therefore
 * implicit: the children of i are the nodes first_child[i]+1 ... first_child[i]+num_children[i].
 *
 * Reference interface replaced (cosmosapjw-quantum/omoknuni_quantum):
 *   the pybind11 module `mcts_cuda_kernels` (python/mcts/gpu/mcts_kernels.cu:2342-2410)
 *   reached through MCTSGPUAccelerator (python/mcts/gpu/mcts_gpu_accelerator.py:81-207)
 *   and the torch.library ops of python/mcts/gpu/torch_custom_ops.py:26-193, together
 *   with the CPU tree python/mcts/cpu/cython_tree_optimized.pyx that the CPU backend
 *   drives.  Each entry point below names the functions it replaces.
 */
#ifndef OMQ_TREE_OPS_H
#define OMQ_TREE_OPS_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OMQ_ABI_VERSION 4

/* error codes */
#define OMQ_OK 0
#define OMQ_E_ARG (-1)     /* invalid argument (size, mode, null pointer)  */
#define OMQ_E_LAUNCH (-2)  /* HIP launch or runtime error                  */
#define OMQ_E_LIMIT (-3)   /* size beyond a compiled limit (wave, row, depth) */

/* game models (how legal actions of a node are derived) */
#define OMQ_GAME_BOARD 0   /* legal = empty cells of the root board minus the actions on the path */
#define OMQ_GAME_GO 1      /* as BOARD over num_actions-1 cells, plus a pass action (num_actions-1) that is always legal */
#define OMQ_GAME_SPARSE 2  /* legal = hash-keyed sample of min_legal..max_legal distinct actions of [0,num_actions) */

/* expansion policies */
#define OMQ_EXPAND_FULL 0          /* every legal action becomes a child */
#define OMQ_EXPAND_REFERENCE_PW 1  /* progressive widening of the reference CPU driver */

/* backup sign conventions */
#define OMQ_SIGN_LEAF_POSITIVE 0   /* W[x] += v * (-1)^(distance of x from the leaf) */
#define OMQ_SIGN_ROOT_POSITIVE 1   /* W[x] += v * (-1)^(depth of x) */

/* W accumulation */
#define OMQ_WACC_ORDERED 0  /* per node, contributions added in simulation order (deterministic) */
#define OMQ_WACC_ATOMIC 1   /* hardware float atomics per path entry (order not fixed) */

/* Gomoku rules of omq_gomoku_terminal */
#define OMQ_RULE_FREESTYLE 0  /* five or more in a row win */
#define OMQ_RULE_RENJU 1      /* as FREESTYLE, but an overline of player 1 does not win (the
                                 reference's simplified renju: no other forbidden moves) */

/* terminal codes of omq_gomoku_terminal */
#define OMQ_TERM_NONE 0
#define OMQ_TERM_WIN1 1  /* player 1 has five */
#define OMQ_TERM_WIN2 2  /* player 2 has five */
#define OMQ_TERM_DRAW 3  /* full board without five */
#define OMQ_TERM_END 4   /* Go: two consecutive passes, or no empty point (omq_go_rules) */

/* flags of omq_go_rules */
#define OMQ_GO_KO 1       /* the root's ko point (root_ko) is not a legal move in the tree */
#define OMQ_GO_SUICIDE 2  /* a point without an empty orthogonal neighbour is not a legal move */

/* workspace of omq_shift_root: int32 entries per node of capacity, per tree */
#define OMQ_SHIFT_WORKSPACE_PER_NODE 8
/* the library's own workspace of omq_shift_root_noalloc: int32 entries (32 MiB per GPU), so
   num_trees * capacity * OMQ_SHIFT_WORKSPACE_PER_NODE may be at most this */
#define OMQ_NOALLOC_SHIFT_INTS (8 * 1024 * 1024)

/* output of omq_leaf_features */
#define OMQ_DTYPE_F32 0   /* float32 planes */
#define OMQ_DTYPE_BF16 1  /* bfloat16 planes, rounded to nearest even */
#define OMQ_LAYOUT_NCHW 0 /* [slot][plane][cell] */
#define OMQ_LAYOUT_NHWC 1 /* [slot][cell][plane] (channels-last) */

/* limits of this build */
#define OMQ_MAX_WAVE 4096   /* simulations per tree per wave */
#define OMQ_MAX_ROW 512     /* children per node (a selection row is held in registers) */
#define OMQ_MAX_DEPTH 128   /* nodes on a path */
/* omq_select forms the unique leaves' records (ukey, ulegal) for waves of at most this many
 * simulations; after a larger wave the caller runs omq_leaf_info, whose launch over all the
 * wave's leaves, spread over the device, is the faster of the two there (one workgroup per
 * tree forms them inside select) */
#define OMQ_SELECT_RECORDS_MAX_WAVE 512
#define OMQ_MAX_ACTIONS 8192

typedef struct omq_forest {
  int32_t num_trees;        /* T */
  int32_t capacity;         /* node capacity per tree */
  int32_t num_actions;      /* A */
  int32_t game;             /* OMQ_GAME_* */
  int32_t legal_words;      /* 32-bit words of a board legal mask: (num_actions+31)/32 */
  int32_t min_legal;        /* OMQ_GAME_SPARSE: fewest legal actions of a node */
  int32_t max_legal;        /* OMQ_GAME_SPARSE: most legal actions of a node */
  int32_t reserved;
  int32_t* visit_counts;    /* [T*capacity] */
  float* value_sums;        /* [T*capacity] */
  float* priors;            /* [T*capacity] */
  int32_t* parents;         /* [T*capacity] */
  int32_t* first_child;     /* [T*capacity] */
  int32_t* num_children;    /* [T*capacity] */
  int32_t* actions;         /* [T*capacity] */
  int32_t* num_nodes;       /* [T] */
  uint64_t* root_keys;      /* [T] hash key of each root position */
  uint32_t* root_legal;     /* [T*legal_words] legal actions at the root (BOARD, GO) */
} omq_forest;

/* Per-wave scratch and outputs, allocated by the caller for max_wave simulations per tree. */
typedef struct omq_wave {
  int32_t max_wave;         /* capacity of the per-simulation arrays, <= OMQ_MAX_WAVE */
  int32_t max_depth;        /* path capacity, <= OMQ_MAX_DEPTH */
  int32_t* paths;           /* [T*max_wave*max_depth] node ids root..leaf of every simulation */
  int32_t* path_len;        /* [T*max_wave] */
  int32_t* leaves;          /* [T*max_wave] leaf node of every simulation */
  int32_t* sim_uid;         /* [T*max_wave] index of the simulation's leaf among the unique leaves */
  int32_t* uleaf;           /* [T*max_wave] unique leaves, in order of first occurrence */
  int32_t* ufirst;          /* [T*max_wave] first simulation that reached each unique leaf */
  int32_t* ucount;          /* [T] number of unique leaves */
  int32_t* glog;            /* [T*max_wave*max_depth*4] visited-node groups: node, depth, seg, len */
  int32_t* gcount;          /* [T] number of groups */
  uint16_t* gmembers;       /* [T*max_depth*max_wave] simulations of each group, in simulation order */
  uint64_t* ukey;           /* [T*max_wave] hash key of each unique leaf */
  int32_t* ulegal;          /* [T*max_wave] number of legal actions of each unique leaf */
  int32_t* uedge;           /* [T*max_wave] edge offset of the children created, -1 if not expanded */
  int32_t* unew;            /* [T*max_wave] number of children created */
  float* policy;            /* [T*max_wave*num_actions] evaluator policy rows of the unique leaves */
  float* values;            /* [T*max_wave] evaluator values of the unique leaves */
  float* sim_value;         /* [T*max_wave] backup scratch: signed leaf value of every simulation
                               (written in atomic mode and for waves of more than 512) */
  int64_t* stats;           /* [T*OMQ_NSTATS] accumulated operation counters */
  int32_t* status;          /* [4] device-side error flags (bit set, never cleared by the library) */
  int32_t* sel_scratch;     /* [OMQ_SEL_SCRATCH_INTS(T, max_wave)] omq_select's scratch: per-
                               simulation leaf records (no contents to keep between calls) */
  uint32_t* umask;          /* NULL, or [T*max_wave*legal_words]: legal-action masks of the unique
                               leaves, written by omq_go_rules.  When it is not NULL,
                               omq_synthetic_evaluate and omq_expand take a board leaf's legal
                               actions from it (the caller then runs omq_go_rules after
                               the leaf records are formed in every wave) instead of the root
                               mask minus the path's cells. */
} omq_wave;

/* default bound of the polls of a wait inside omq_select (omq_select_options) */
#define OMQ_SPIN_LIMIT_DEFAULT (1 << 22)

/* int32 entries of omq_wave::sel_scratch for T trees of max_wave simulations */
#define OMQ_SEL_SCRATCH_INTS(T, MW) (2 * (int64_t)(T) * (MW))

/* stats counters (per tree, accumulated over waves) */
#define OMQ_ST_INTERNAL 0     /* groups that selected a child (distinct internal nodes per wave) */
#define OMQ_ST_ROWSUM 1       /* sum of row lengths read by those groups (a row whose picks
                                 are all first-unvisited children: up to its last pick) */
#define OMQ_ST_PATHNODES 2    /* distinct path nodes (groups) */
#define OMQ_ST_PATHENTRIES 3  /* sum over simulations of path length */
#define OMQ_ST_ULEAVES 4      /* unique leaves */
#define OMQ_ST_EXPANDED 5     /* leaves expanded */
#define OMQ_ST_NEWCHILD 6     /* children created */
#define OMQ_ST_SIMS 7         /* simulations selected */
#define OMQ_ST_STEPS 8        /* argmax steps (simulation x level decisions) */
#define OMQ_ST_CAPFAIL 9      /* expansions refused for lack of capacity */
#define OMQ_ST_ULEAFPATH 10   /* sum over unique leaves of path length (leaf records) */
#define OMQ_ST_ROOTCHAIN 11   /* omq_select: duration of the root's chain (the serial part of a
                                 wave's selection), in ticks of the device's constant wall clock
                                 (omq_wall_clock_khz) */
#define OMQ_NSTATS 16

/* device status bits */
#define OMQ_STATUS_NOCHILD 1    /* best-child returned -1 at an expanded node */
#define OMQ_STATUS_ROWLIMIT 2   /* a row longer than OMQ_MAX_ROW was met or refused */
#define OMQ_STATUS_STALL 4      /* a bounded wait inside omq_select ran out (internal error: the
                                   wave's selection is incomplete) */
#define OMQ_STATUS_COUNTLIMIT 8 /* omq_select met a root with 1 + N + virtual_loss * wave >= 2^24:
                                   the selection keeps a row's visit counts as floats advanced
                                   by the virtual loss, which are exact only below 2^24 (every
                                   node's count is at most its root's); the wave's picks may
                                   then differ from the reference's */

/* ---- library ---------------------------------------------------------------------- */
int omq_abi_version(void);
const char* omq_last_error(void);

/* Reset every tree to a lone root: N=1, P=1, W=0, no children, num_nodes=1.
 * Replaces CythonLockFreeTree.__cinit__/reset (python/mcts/cpu/cython_tree_optimized.pyx:64-103,537-558)
 * and CSRTree.reset (python/mcts/gpu/csr_tree.py). */
int omq_forest_reset(const omq_forest* f, void* stream);

/* Select one wave of `wave_size` simulations in every tree, with virtual loss.
 * Result equals running CythonLockFreeTree.select_path (cython_tree_optimized.pyx:177-202,
 * best child :421-464) for simulations 0..wave_size-1 one after another: every node on a
 * path receives +(int)virtual_loss visits as the simulation arrives, and later simulations
 * see it.  Writes paths, path_len, leaves, the unique-leaf list and the group log, and, for
 * waves of at most OMQ_SELECT_RECORDS_MAX_WAVE simulations, each unique leaf's key and legal
 * count (ukey, ulegal, as omq_leaf_info forms them; OMQ_ST_ULEAFPATH), and adds the virtual
 * loss to visit_counts.  vl_atomic=1 applies the virtual loss with
 * one atomic per path entry instead of one add per visited node.
 * Replaces fused_select_expand(_optimized) / parallel_select_with_virtual_loss /
 * batch_apply_virtual_loss (python/mcts/gpu/mcts_kernels.cu:451-643,845-860,962-1053). */
int omq_select(const omq_forest* f, const omq_wave* w, int32_t wave_size, float c_puct,
               float virtual_loss, int32_t max_depth, int32_t vl_atomic, void* stream);

/* Process-wide option of omq_select, for tests; no counterpart in the reference.
 * spin_limit bounds the polls of a wait inside omq_select (default OMQ_SPIN_LIMIT_DEFAULT,
 * at least 0).  Running out sets OMQ_STATUS_STALL, and the simulations it held up end their
 * paths early; the trees must then be reset.  The value is read at each omq_select call, so a
 * recorded graph keeps the value of its recording.  Returns OMQ_E_ARG for a negative limit. */
int omq_select_options(int32_t spin_limit);

/* The spin limit omq_select launches with (for callers that record graphs and key them by
 * the launch arguments); no counterpart in the reference. */
int32_t omq_select_spin_limit(void);

/* Frequency (kHz) of the constant wall clock of the current device, the unit of
 * OMQ_ST_ROOTCHAIN; no counterpart in the reference (measurement of selection's serial part). */
int omq_wall_clock_khz(int32_t* khz);

/* Compute the hash key and the number of legal actions of every unique leaf of the wave.
 * (Game-model step between selection and evaluation; no reference counterpart in the
 * kernel module: the reference reads GPUGameStates, python/mcts/gpu/gpu_game_states.py.)
 * Needed after a wave of more than OMQ_SELECT_RECORDS_MAX_WAVE simulations; after a smaller
 * one omq_select has formed them, and this forms them again (adding to OMQ_ST_ULEAFPATH
 * again). */
int omq_leaf_info(const omq_forest* f, const omq_wave* w, void* stream);

/* Synthetic evaluator: for every unique leaf, priors = softmax of seeded approximately
 * normal logits (scale logit_scale) over its legal actions, written into policy rows at
 * the legal action slots only; value = 2u-1 with u a 24-bit hash fraction of the leaf key.
 * Stands in for Evaluator.evaluate_batch (python/mcts/core/evaluator.py:85-104). */
int omq_synthetic_evaluate(const omq_forest* f, const omq_wave* w, float logit_scale,
                           void* stream);

/* Expand the unique leaves of the wave in first-occurrence order: priors = policy at the legal
 * actions renormalised over them; progressive widening (OMQ_EXPAND_REFERENCE_PW) sizes the root
 * row from the root's visit count without the wave's in-flight virtual loss
 * (wave_size*(int)virtual_loss); at the root, optional Dirichlet mixing with the noise
 * vector root_noise[t*num_actions + i] (i = position among the root's legal actions, double);
 * children allocated by bump pointer, skipping a leaf whose children do not fit.
 * Replaces OptimizedCPUWaveSearch._batch_expand_and_backup expansion part
 * (python/mcts/cpu/optimized_wave_search.py:367-438) + CythonLockFreeTree.expand_node
 * (cython_tree_optimized.pyx:232-277) and batched_add_children (mcts_kernels.cu:1122-1189). */
int omq_expand(const omq_forest* f, const omq_wave* w, int32_t wave_size, float virtual_loss,
               int32_t expand_policy, const double* root_noise, double dirichlet_epsilon,
               void* stream);

/* Back up the wave: for every node x on the path of every simulation,
 * N[x] += 1 - (int)virtual_loss (reverting the virtual loss of omq_select) and
 * W[x] += sign * value(leaf).  w_mode OMQ_WACC_ORDERED adds the contributions to each node
 * in simulation order (bit-identical to the sequential reference loop).
 * Replaces CythonLockFreeTree.backup_value (cython_tree_optimized.pyx:204-230),
 * OptimizedCPUWaveSearch._batch_backup_paths (optimized_wave_search.py:457-483),
 * vectorized_backup / batch_remove_virtual_loss (mcts_kernels.cu:121-158,934-953). */
int omq_backup(const omq_forest* f, const omq_wave* w, int32_t wave_size, float virtual_loss,
               int32_t sign_mode, int32_t w_mode, void* stream);

/* omq_expand followed by omq_backup, with the same arguments, and the same results: the two
 * write no common address and neither reads what the other writes, so their kernels run side
 * by side, in two launches instead of four (the expansion plan beside the signed leaf values,
 * then the child records beside the group backup).  Under OMQ_EXPAND_REFERENCE_PW (whose rule
 * reads the root's count, which the backup changes), with OMQ_WACC_ATOMIC, or where the
 * expansion's LDS per leaf exceeds 16 KiB, it runs the two one after the other.
 * Replaces the expansion and the backup of OptimizedCPUWaveSearch._batch_expand_and_backup
 * (python/mcts/cpu/optimized_wave_search.py:367-483), run back to back. */
int omq_expand_backup(const omq_forest* f, const omq_wave* w, int32_t wave_size,
                      float virtual_loss, int32_t expand_policy, const double* root_noise,
                      double dirichlet_epsilon, int32_t sign_mode, int32_t w_mode,
                      void* stream);

/* Gomoku terminal check of every unique leaf of the wave; call it after the leaf records are
 * formed (by omq_select, or by omq_leaf_info after a wave of more than
 * OMQ_SELECT_RECORDS_MAX_WAVE simulations) and before omq_expand.  Needs an OMQ_GAME_BOARD forest with num_actions = bs*bs.
 * - Position.  A leaf's position is the root board root_boards[t*num_actions + cell] (int8:
 *   0 empty, 1 and 2 stones) with the moves of the leaf's path played in alternating colours.
 *   The first move is played by root_player[t]. When root_player is NULL, it is player 1 if the
 *   root board holds an even number of stones, else player 2 (python/mcts/core/mcts.py:1506).
 * - Scan.  The position is scanned as FastTerminalChecker._check_gomoku_terminal_cpu scans it
 *   (python/mcts/utils/fast_terminal_check.py:132-232): cells in row-major order, directions
 *   horizontal, vertical, down-right and down-left. The first cell that starts a five names the
 *   winner. Under OMQ_RULE_RENJU an overline of player 1 does not count, and it ends that
 *   cell's scan as in the reference. A full board without a five is a draw.
 * - Terminal leaves.  A terminal leaf gets ulegal = 0, so omq_expand leaves it unexpanded
 *   (python/mcts/cpu/optimized_wave_search.py:374-376). Its value is still the evaluator's. The
 *   root (a path of length 1) is never terminal.
 * - Output.  uterminal, when not NULL, is [T*max_wave] and receives OMQ_TERM_* per unique leaf.
 * Replaces the terminal detection run by CPUGameStates.apply_actions
 * (python/mcts/cpu/cpu_game_states.py:352-412) and the GPU Gomoku terminal kernels
 * (python/mcts/gpu/gomoku_kernels.py:14-160). */
int omq_gomoku_terminal(const omq_forest* f, const omq_wave* w, const int8_t* root_boards,
                        const int32_t* root_player, int32_t rule, int32_t* uterminal,
                        void* stream);

/* Go rules of every unique leaf of the wave; call it after the leaf records are formed (as for
 * omq_gomoku_terminal) and before the evaluator and omq_expand.  Needs an OMQ_GAME_GO forest with num_actions = bs*bs + 1 (the pass
 * is action bs*bs), w->umask set, and the root positions root_boards [T*bs*bs] (int8: 0 empty,
 * 1 and 2 stones).
 * - Position.  A leaf's position is its root board with the path's moves played in alternating
 *   colours from root_player[t] (NULL: 1 when the root board holds an even number of stones,
 *   else 2); a pass places no stone.  No stone is captured, as in the reference's GPU game
 *   states (GPUGameStates.apply_moves, python/mcts/gpu/gpu_game_states.py:405-460).
 * - Legal moves (umask).  The empty points, except: with OMQ_GO_KO, root_ko[t] (a point, or -1
 *   for none) at every node of the tree (GPUGameStates.get_legal_moves_mask,
 *   gpu_game_states.py:373-395, excludes a state's ko point; clone_states, :336-337, copies it
 *   from parent to child and apply_moves never updates it, so the root's ko point holds in the
 *   whole tree); with OMQ_GO_SUICIDE, the points without an empty orthogonal neighbour (the
 *   simplified suicide rule of gpu_get_legal_moves, python/mcts/gpu/go_kernels.py:46-110).
 *   The pass is always legal.
 * - Terminal (gpu_check_terminal_states, go_kernels.py:17-44).  A leaf whose path ends in two
 *   consecutive passes (the root's own trailing passes root_passes[t] counting when every path
 *   move is a pass; NULL: 0), or whose position has no empty point (that function's legal
 *   moves are the empty points: it passes no player), is terminal: uterminal OMQ_TERM_END and
 *   ulegal 0, so omq_expand leaves it unexpanded.  The root (a path of length 1) is never
 *   terminal.  (The reference's FastTerminalChecker.check_terminal_gpu,
 *   python/mcts/utils/fast_terminal_check.py:87-93, hands that function zero pass counts;
 *   here the passes are counted.)
 * - Otherwise ulegal is the number of legal moves.  uterminal, when not NULL, is [T*max_wave].
 * Replaces the Go legality and terminal checks of the reference's GPU game states
 * (gpu_game_states.py:373-395, go_kernels.py:17-110), which its GPU search runs per leaf. */
int omq_go_rules(const omq_forest* f, const omq_wave* w, const int8_t* root_boards,
                 const int32_t* root_player, const int32_t* root_passes, const int32_t* root_ko,
                 int32_t flags, int32_t* uterminal, void* stream);

/* Neural-network feature planes of every wave slot of a Gomoku forest; call it after the leaf
 * records are formed (as for omq_gomoku_terminal).  Needs an OMQ_GAME_BOARD forest with num_actions = bs*bs.
 * - Slots.  out holds num_trees*max_wave slots of planes*bs*bs values (slot t*max_wave+u).
 *   Slot u < ucount[t] receives the position of unique leaf u; the other slots receive zeros.
 * - Position.  As in omq_gomoku_terminal: the root board with the path's moves in alternating
 *   colours from root_player[t] (NULL: 1 when the root board holds an even number of stones,
 *   else 2). The leaf's move count is root_moves[t] (NULL: the root board's stone count) plus
 *   the moves on the path (python/mcts/core/mcts.py:1503-1508, cpu_game_states.py:352-412).
 * - Planes (planes = 18 or 19).  0 stones of the player to move; 1 the opponent's stones;
 *   2-15 zero; 16 ones when player 1 is to move; 17 move count / 100; 18 ones (19 planes only).
 *   This is CPUGameStates.get_nn_features 'basic' (python/mcts/cpu/cpu_game_states.py:430-494);
 *   18 planes leaves out its last, all-ones plane.
 * - dtype OMQ_DTYPE_F32 or OMQ_DTYPE_BF16; layout OMQ_LAYOUT_NCHW or OMQ_LAYOUT_NHWC. out is
 *   aligned to two elements (8 bytes for float32, 4 for bfloat16).
 * Replaces the per-state feature extraction of CPUGameStates.get_nn_features, which the CPU
 * driver feeds its evaluator (python/mcts/cpu/optimized_wave_search.py:337). The reference's
 * GPU builder, GPUGameStates.get_nn_features (python/mcts/gpu/gpu_game_states.py:534-664),
 * has the same role with another plane layout. */
int omq_leaf_features(const omq_forest* f, const omq_wave* w, const int8_t* root_boards,
                      const int32_t* root_player, const int32_t* root_moves, int32_t planes,
                      int32_t dtype, int32_t layout, void* out, void* stream);

/* Subtree reuse.  For every tree t with 0 < new_roots[t] < num_nodes[t], node new_roots[t]
 * becomes the root, and its subtree is kept. Other values leave tree t unchanged.
 * - Numbering.  Kept nodes are renumbered breadth-first from the new root, children in row
 *   order. This is the order in which CSRTree.shift_root assigns the new indices.
 * - Copied fields.  N, W and P are copied, and parents and rows are remapped. The new root has
 *   parent -1 and action -1 and keeps its N, W and P.
 * - Dropped nodes.  Every other node is dropped, and num_nodes[t] becomes the subtree size.
 * - Layout.  Children stay consecutive (child of edge e = node e+1), so the tree is ready for
 *   the next omq_select.
 * - Inconsistent trees.  A tree with a row outside [0, num_nodes) is left unchanged.
 * - Workspace.  A device array of at least
 *   OMQ_SHIFT_WORKSPACE_PER_NODE * num_trees * capacity int32 entries, owned by the caller.
 * The caller updates what lives outside the forest arrays: the root key, the root legal mask
 * and the root board.
 * Replaces CSRTree.shift_root (python/mcts/gpu/csr_tree.py:1020-1229) as used by
 * TreeOperations.apply_subtree_reuse (python/mcts/core/tree_operations.py:53-133) and the
 * reuse kernels of mcts_kernels.cu:2095-2337. */
int omq_shift_root(const omq_forest* f, const int32_t* new_roots, int32_t* workspace,
                   int64_t workspace_ints, void* stream);

/* omq_shift_root without a caller workspace, and without any allocation: the workspace is a
 * device array of the library (OMQ_NOALLOC_SHIFT_INTS int32, 32 MiB, one per GPU the library
 * runs on, held until the process ends).  Same semantics and results as omq_shift_root.
 * - Limit.  num_trees * capacity * OMQ_SHIFT_WORKSPACE_PER_NODE must not exceed
 *   OMQ_NOALLOC_SHIFT_INTS (num_trees * capacity <= 1,048,576 nodes); larger forests get
 *   OMQ_E_LIMIT and nothing is launched.
 * - No allocation.  The entry point calls no hipMalloc, hipFree or allocating library routine;
 *   its first call on a device looks the array's address up (hipGetSymbolAddress).
 * - Sharing.  Every call on one GPU uses that GPU's array: calls that overlap on one GPU (two
 *   streams, two threads) race, and must be ordered by the caller.
 * No counterpart in the reference: this entry point is for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid allocation). */
int omq_shift_root_noalloc(const omq_forest* f, const int32_t* new_roots, void* stream);

/* Root visit-count policy of every tree into policy[t*num_actions + a] (double):
 * N(child_a) / (sum of the root's children's N). When the root has no children, the policy
 * is uniform over the action space. When it has children but no visits, it is uniform over
 * the children's actions.
 * Replaces MCTS._extract_policy (python/mcts/core/mcts.py:1069-1137). */
int omq_root_policy(const omq_forest* f, double* policy, void* stream);

/* Move selection per tree from policy rows (as omq_root_policy writes them) into actions[t].
 * - temperature 0 takes the first maximum.
 * - Otherwise w_a = p_a^(1/temperature), with w = p at temperature 1 and 0 where p = 0. The
 *   action is the first a whose normalised cumulative sum of w_a / sum(w) exceeds a uniform
 *   draw u in [0, 1).
 * u comes from a SplitMix64 stream keyed by (seed, counter, tree), in place of numpy's global
 * generator; one (seed, counter) pair gives one reproducible draw per tree. The power is
 * evaluated as exp(log(p)/T) with the library's own log and exp.
 * Replaces MCTS.select_action (python/mcts/core/mcts.py:1167-1203). */
int omq_sample_actions(const omq_forest* f, const double* policy, double temperature,
                       uint64_t seed, uint64_t counter, int32_t* actions, void* stream);

/* Root Dirichlet noise on the device. Row t of noise ([T*num_actions], double) receives a
 * Dirichlet(alpha, ..., alpha) draw over the root's L legal actions: entry i belongs to the
 * i-th legal action (the layout omq_expand reads), and entries i >= L are 0. L is the root
 * legal mask's popcount for board models and the sparse-model count of the root key otherwise.
 * - Gamma variates: Marsaglia-Tsang. Shape < 1 is boosted by U^(1/alpha).
 * - Normal variates: Marsaglia's polar method.
 * - log and exp: the library's own.
 * - Uniforms: a SplitMix64 stream keyed by (seed, counter, tree, action index).
 * Replaces np.random.dirichlet at root expansion (python/mcts/cpu/optimized_wave_search.py:387-392)
 * and the Dirichlet kernel of mcts_kernels.cu:649-754. */
int omq_root_dirichlet(const omq_forest* f, double alpha, uint64_t seed, uint64_t counter,
                       double* noise, void* stream);

/* Reference-style path backup over an explicit path matrix (no group log needed):
 * paths[b*max_depth + d], d < min(path_len[b], max_depth), root first; values[b] is the leaf
 * value; N[x] += 1, W[x] += sign * values[b] with float atomics, the sign taken from the
 * distance to the leaf (path_len[b]-1-d) or the depth d; tree index tree_of[b] (tree 0 for
 * all when tree_of is NULL).  Entries outside [0, capacity) (-1 padding) are skipped, as in
 * the reference kernel; a row whose tree index is outside [0, num_trees) is skipped.  Only
 * num_trees, capacity, visit_counts and value_sums of the forest are read.
 * Replaces vectorized_backup (mcts_kernels.cu:121-158 / torch_custom_ops.py mcts::vectorized_backup). */
int omq_paths_backup(const omq_forest* f, const int32_t* paths, const int32_t* path_len,
                     const int32_t* tree_of, const float* values, int32_t batch, int32_t max_depth,
                     int32_t sign_mode, void* stream);

/* Reference-style virtual loss on a node list: visit_counts[tree_of[i]*capacity + nodes[i]]
 * += delta (atomic).  delta > 0 applies, delta < 0 reverts (no clamp at zero: every revert
 * pairs with an apply).  Entries whose node or tree index is out of range (including -1
 * padding) are skipped.  Only num_trees, capacity and visit_counts of the forest are read.
 * Replaces batch_apply_virtual_loss / batch_remove_virtual_loss (mcts_kernels.cu:845-860,934-953). */
int omq_virtual_loss(const omq_forest* f, const int32_t* nodes, const int32_t* tree_of,
                     int32_t count, int32_t delta, void* stream);

/* Reference fused UCB selection over explicit CSR edges.  For b < batch, parent
 * p = node_indices[b] with row [children_start[p], children_end[p]) of children[] / priors[]:
 *     ucb_i = (visit_counts[c_i] > 0 ? q_values[c_i] : 0)
 *             + c_puct * priors_i * sqrtf((float)visit_counts[p]) / (1 + visit_counts[c_i])
 * in float32 (left to right), and selected[b] = the row position of the first maximum above
 * -1e10 (strict '>'), or -1 for an empty row.  Unvisited children get q = 0 and no priority
 * (this is not omq_select's rule).  The index arrays are trusted: every index must lie in its
 * array (as in the reference).
 * Replaces mcts::fused_ucb_selection (python/mcts/gpu/torch_custom_ops.py:108-193) and its
 * kernel fused_ucb_selection_adapter_kernel (python/mcts/gpu/mcts_kernels.cu:1466-1512). */
int omq_fused_ucb_selection(const int32_t* node_indices, int32_t batch,
                            const int32_t* children_start, const int32_t* children_end,
                            const int32_t* children, const float* q_values,
                            const int32_t* visit_counts, const float* priors, float c_puct,
                            int32_t* selected, void* stream);

/* The reference accelerator's remaining operators (MCTSGPUAccelerator,
 * python/mcts/gpu/mcts_gpu_accelerator.py:81-207, over the pybind module of
 * python/mcts/gpu/mcts_kernels.cu:2342-2410).  Their trees are the reference's GPU variant: a
 * dense children table children[num_nodes * max_children] (a row ends at its first negative
 * entry) and explicit CSR edges.  Index arrays are trusted as in the reference, except where a
 * check is stated. */

/* Paths whose current node needs expansion: for s < wave_size with valid_mask[s] != 0 and
 * 0 <= current_nodes[s] < num_nodes, the node when its table row holds no child and its visit
 * count is 0.  The nodes are written to out_nodes in path order (a node reached by two paths is
 * written twice, as in the reference) and their number to out_count[0] (device memory);
 * out_nodes holds wave_size entries, all of which the call may write.
 * Replaces find_expansion_nodes_cuda (mcts_kernels.cu:46-87,1329-1362), which writes them in
 * the order its atomics land and bounds the node index by the number of paths. */
int omq_find_expansion_nodes(const int32_t* current_nodes, const uint8_t* valid_mask,
                             int32_t wave_size, const int32_t* children, int32_t max_children,
                             const int32_t* visit_counts, int32_t num_nodes, int32_t* out_nodes,
                             int32_t* out_count, void* stream);

/* UCB selection over CSR rows: for row b < batch, edges [row_ptr[b], row_ptr[b+1]) of
 * col_indices / priors, child c_i = col_indices[i]:
 *     ucb_i = (visit_counts[c_i] > 0 ? q_values[c_i] : 0)
 *             + c_puct * priors[i] * sqrtf((float)parent_visits[b] + 1) / (1 + visit_counts[c_i])
 * in float32, left to right; an edge is skipped when c_i < 0, and also (the reference reads
 * past its arrays there) when i >= num_children or c_i >= num_children.  selected[b] = the row
 * position of the first maximum above -1e10 (strict '>'), 0 when no score is above it or when
 * row_ptr[b] < 0 or row_ptr[b+1] < row_ptr[b], and -1 for an empty row; scores[b] (when not
 * NULL) that maximum (-1e10 without one, 0 for the last three cases).
 * Replaces batched_ucb_selection_cuda (mcts_kernels.cu:240-318,1412-1464). */
int omq_batched_ucb_selection(const float* q_values, const int32_t* visit_counts,
                              int32_t num_children, const int32_t* parent_visits,
                              const float* priors, const int32_t* row_ptr,
                              const int32_t* col_indices, int32_t batch, float c_puct,
                              int32_t* selected, float* scores, void* stream);

/* Selection down the dense children table, one path per root: from roots[w], while depth <
 * max_depth - 1, an expanded node (is_expanded) scores its children (up to the first negative
 * entry): an unvisited child +inf, else q_values[c] + c_puct * prior_probs[c] *
 * sqrtf((float)visit_counts[node]) / (1 + visit_counts[c]) (float32, left to right); the first
 * maximum (strict '>' from -inf) is next.  A node that is not expanded, has no child or no
 * child above -inf ends the path: expand_nodes[w] = node, needs_expansion[w] = 1,
 * path_lengths[w] = depth + 1.  A path that reaches depth max_depth - 1 leaves path_lengths[w],
 * expand_nodes[w] and needs_expansion[w] at 0, as the reference's kernel does.
 * paths[w * max_depth + i] holds the path's nodes and -1 after its last.  The children table
 * has num_nodes rows: a child entry >= num_nodes ends its row as a negative one does, and a
 * root outside [0, num_nodes) is a path of one node that needs expansion (the reference reads
 * past its arrays in both cases).  max_depth >= 1.
 * Replaces fused_select_expand_cuda (mcts_kernels.cu:451-544,2002-2045). */
int omq_fused_select_expand(const int32_t* roots, int32_t num_paths, const int32_t* children,
                            int32_t num_nodes, int32_t max_children,
                            const int32_t* visit_counts, const float* q_values,
                            const float* prior_probs, const uint8_t* is_expanded,
                            int32_t max_depth, float c_puct, int32_t* paths,
                            int32_t* path_lengths, int32_t* expand_nodes,
                            uint8_t* needs_expansion, void* stream);

/* The reference's second form of the same descent: from roots[w], while depth < max_depth - 1
 * and depth < 32, a node with visit_counts[node] == 0 ends the path; otherwise its children (up
 * to the first negative entry) score
 *     q = n > 0 ? value_sums[c] * (1 / ((float)n + 1e-8f)) : 0,   n = visit_counts[c]
 *     ucb = q + c_puct * priors[c] * sqrt_parent * (1 / (1 + (float)n))
 * with correctly rounded float32 reciprocals and sqrt_parent = 1 / sqrt(r), r = 1 / (float)(N +
 * 1) in float32, the square root and its reciprocal taken in float64 and rounded once to float32
 * (the reference's rsqrtf is an approximation with no published rounding); the first maximum
 * (strict '>' from -inf) is next, and a node with no such child ends the path.
 * path_lengths[w] = depth + 1 always; paths as above; ucb_scores[w * max_children + i] = the
 * root's score of child i (0 past the row's end, or when the root is not scored).  Bounds as
 * above.  Replaces fused_select_expand_optimized_cuda (mcts_kernels.cu:546-640,2047-2083). */
int omq_fused_select_expand_optimized(const int32_t* roots, int32_t num_paths,
                                      const int32_t* children, int32_t num_nodes,
                                      int32_t max_children, const int32_t* visit_counts,
                                      const float* value_sums, const float* priors,
                                      int32_t max_depth, float c_puct, float* ucb_scores,
                                      int32_t* paths, int32_t* path_lengths, void* stream);

/* Children appended for a batch of parents, in batch order.  Parent b with 0 <=
 * parent_indices[b] < max_nodes and n = num_children[b] > 0 takes nodes [node_counter[0],
 * + n) and edges [edge_counter[0], + n) (both counters advance by n); when either range passes
 * max_nodes / max_edges nothing is written for it (the counters still advance, as the
 * reference's atomic bump does).  For i < min(n, max_children), child c = first node + i and
 * edge e = first edge + i: parent_indices_out[c] = p, parent_actions_out[c] = actions[b *
 * max_children + i], node_priors_out[c] = priors[b * max_children + i], visit_counts_out[c] =
 * 0, value_sums_out[c] = 0, children[p * max_children + i] = c (when that slot is below
 * max_nodes * max_children), col_indices[e] = c, edge_actions[e] and edge_priors[e] as the
 * child's.  child_indices[b * max_children + i] = c for every child written, -1 otherwise.
 * Two items with the same parent write the same children-table slots, and which lands last is
 * not specified (nor is it in the reference).  max_children >= 1.
 * Replaces batched_add_children_cuda (mcts_kernels.cu:1122-1189,1679-1733), which allocates in
 * the order its threads' atomics land (batch order is one of them) and returns the index
 * tensor unfilled. */
int omq_batched_add_children(const int32_t* parent_indices, int32_t batch,
                             const int32_t* actions, const float* priors,
                             const int32_t* num_children, int32_t* node_counter,
                             int32_t* edge_counter, int32_t* children,
                             int32_t* parent_indices_out, int32_t* parent_actions_out,
                             float* node_priors_out, int32_t* visit_counts_out,
                             float* value_sums_out, int32_t* col_indices, int32_t* edge_actions,
                             float* edge_priors, int32_t max_nodes, int32_t max_children,
                             int32_t max_edges, int32_t* child_indices, void* stream);

/* ---- more of the reference pybind module's operators (mcts_kernels.cu:2342-2410) ---------- */

/* Per-simulation selection over a parent's row of the dense children table with virtual-loss
 * counts (parallel_select_with_virtual_loss_enhanced_cuda, python/mcts/gpu/mcts_kernels.cu:
 * 1936-2000, kernel :962-1053; bound at :2371-2384, probed by
 * python/mcts/gpu/wave_search.py:1193).  Simulation s scores the children of
 * p = parent_nodes[s] at table positions [0, max_children) of row p (stride children_stride),
 * skipping entries < 0 or >= num_nodes: n = N[c] + VL[c], value = W[c] + VL[c] * vl (float),
 * Q = value / n for n > 0 else 0, ucb = Q + c_puct * P * sqrt(N[p] + 1) / (1 + n), with
 * P = priors[c], or priors[s * priors_stride + c] when priors_stride > 0 (per-simulation
 * priors; children >= priors_stride skipped).  With legal_masks ([num_sims,
 * action_space_size] bytes; NULL: none), a child of a parent other than node 0 whose action
 * child_actions[c] is in [0, action_space_size) and illegal for s is skipped.  The child of
 * the first maximum above -inf (strict '>') is written to selected_children[s], else -1 (also
 * for p < 0 or p outside the rows or arrays).  Then virtual_loss_counts[c] += 1 for every
 * selection (after all of them).  The reference's dirichlet_noise / dirichlet_epsilon
 * arguments are ignored by it (priors come pre-mixed) and are not taken here. */
int omq_parallel_select_with_virtual_loss(
    const int32_t* parent_nodes, int32_t num_sims, const int32_t* children, int32_t num_rows,
    int32_t max_children, int32_t children_stride, const int32_t* visit_counts,
    int32_t* virtual_loss_counts, const float* value_sums, int32_t num_nodes,
    const float* priors, int32_t priors_stride, const uint8_t* legal_masks,
    int32_t action_space_size, const int32_t* child_actions, float c_puct,
    float virtual_loss_value, int32_t* selected_children, void* stream);

/* Root selection with per-simulation Dirichlet-mixed priors (fused_ucb_with_noise_cuda,
 * python/mcts/gpu/mcts_kernels.cu:1791-1823, kernel :760-797; MCTSGPUAccelerator.
 * fused_ucb_with_noise, python/mcts/gpu/mcts_gpu_accelerator.py:326-327): for simulation s,
 * P' = (1 - eps) P[c] + eps * noise[s, c] and ucb = q[c] + c_puct * P' * parent_visits_sqrt /
 * (1 + N[c]); selected[s] = the position of the first maximum above -1e10, or 0. */
int omq_fused_ucb_with_noise(const float* q_values, const int32_t* visit_counts,
                             const float* priors, int32_t num_children,
                             const float* dirichlet_noise, int32_t num_sims,
                             float parent_visits_sqrt, float c_puct, float epsilon,
                             int32_t* selected, void* stream);

/* UCB selection over dense per-item slots (batched_ucb_selection_dense_cuda,
 * python/mcts/gpu/mcts_kernels.cu:1563-1598, kernel :1364-1409): item b's slots with
 * valid_mask set and child c in [0, num_valid_children) score
 * (N[c] > 0 ? V[c] : 0) + c_puct * P[b, slot] * sqrt(pv[b] + 1) / (1 + N[c]); selected[b] = the
 * child of the first maximum above -1e10, or -1. */
int omq_batched_ucb_selection_dense(const int32_t* batch_children, const float* batch_priors,
                                    const int32_t* parent_visits, const uint8_t* valid_mask,
                                    int32_t batch, int32_t max_children,
                                    const int32_t* child_visits, const float* child_values,
                                    int32_t num_valid_children, float c_puct,
                                    int32_t* selected, void* stream);

/* Rows of Dirichlet(alpha) noise (batched_dirichlet_noise_cuda, python/mcts/gpu/
 * mcts_kernels.cu:1735-1790, kernels :649-754; MCTSGPUAccelerator.batched_dirichlet_noise,
 * mcts_gpu_accelerator.py:323-324): noise[s, a] = g[s, a] / sum_a g[s, a] with
 * g ~ Gamma(alpha, 1), 0 for a row whose sum is 0.  The draws come from the counter-based
 * stream of omq_root_dirichlet keyed by (seed, counter, row, entry) in place of the
 * reference's time-seeded cuRAND states; the gammas and the row sum are float64, each quotient
 * is rounded to float32 once. */
int omq_batched_dirichlet_noise(int32_t num_sims, int32_t num_actions, double alpha,
                                uint64_t seed, uint64_t counter, float* noise, void* stream);

/* optimized_backup_scatter_cuda (python/mcts/gpu/mcts_kernels.cu:1825-1870;
 * MCTSGPUAccelerator.optimized_backup_scatter, mcts_gpu_accelerator.py:329-330): the reference
 * prepares per-entry updates it never reads and then runs vectorized_backup_kernel, so this is
 * omq_paths_backup with the leaf-positive sign over plain arrays of num_nodes counts. */
int omq_optimized_backup_scatter(const int32_t* paths, const int32_t* path_lengths,
                                 const float* values, int32_t batch, int32_t max_depth,
                                 int32_t* visit_counts, float* value_sums, int32_t num_nodes,
                                 void* stream);

/* int32 workspace entries of omq_parallel_bfs_subtree and omq_extract_subtree_edges */
#define OMQ_BFS_WORKSPACE_INTS(max_nodes) (3 * (int64_t)(max_nodes) + 1)
#define OMQ_EDGES_WORKSPACE_INTS(num_nodes) \
  ((int64_t)(num_nodes) + ((int64_t)(num_nodes) + 1023) / 1024 + 1)

/* Breadth-first subtree of root_idx in a CSR graph (parallel_bfs_subtree_cuda,
 * python/mcts/gpu/mcts_kernels.cu:2246-2287, kernel :2095-2194; bound at :2396-2401; called
 * from python/mcts/gpu/gpu_bfs.py:49).  row_ptr holds max_nodes + 1 offsets into
 * col_indices [num_edges] (rows clamped to it).  Writes in_subtree [max_nodes] (0/1),
 * node_remap [max_nodes] (the new index, -1 outside) and *subtree_count.  New indices follow
 * a FIFO breadth-first walk: levels in order, each node's children in row order, a child at
 * its first occurrence (the order of the reference's fallback, gpu_bfs.py:70-127); children
 * outside [0, max_nodes) are skipped.  *subtree_count = -1 when a level's rows add up past
 * 2^31 - 1 (overlapping rows).  One workgroup; workspace: OMQ_BFS_WORKSPACE_INTS(max_nodes)
 * int32 owned by the caller. */
int omq_parallel_bfs_subtree(const int32_t* row_ptr, const int32_t* col_indices,
                             int32_t num_edges, int32_t root_idx, int32_t max_nodes,
                             uint8_t* in_subtree, int32_t* node_remap, int32_t* subtree_count,
                             int32_t* workspace, int64_t workspace_ints, void* stream);

/* The edges of a subtree found by omq_parallel_bfs_subtree (extract_subtree_edges_cuda,
 * python/mcts/gpu/mcts_kernels.cu:2289-2337, kernel :2201-2244; bound at :2402-2408; called
 * from python/mcts/gpu/gpu_bfs.py:149).  For every node i < num_nodes with in_subtree[i], in
 * ascending i, the edges e of its row (in row order) whose child c is in [0, num_nodes) and in
 * the subtree give (node_remap[i], node_remap[c], edge_actions[e] or 0 when edge_actions is
 * NULL), written in that order up to max_edges entries; *edge_count = the number of such edges
 * (it can exceed max_edges: the caller checks).  Workspace:
 * OMQ_EDGES_WORKSPACE_INTS(num_nodes) int32 owned by the caller. */
int omq_extract_subtree_edges(const int32_t* row_ptr, const int32_t* col_indices,
                              const int16_t* edge_actions, int32_t num_edges,
                              const uint8_t* in_subtree, const int32_t* node_remap,
                              int32_t num_nodes, int32_t max_edges, int32_t* edge_parents,
                              int32_t* edge_children, int16_t* edge_actions_out,
                              int32_t* edge_count, int32_t* workspace, int64_t workspace_ints,
                              void* stream);

#ifdef __cplusplus
}
#endif
#endif /* OMQ_TREE_OPS_H */
