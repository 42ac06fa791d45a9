// C ABI of libomq_tree_ops.so: argument checks, error reporting, launches.
// Declarations and the reference functions each entry point replaces: include/omq_tree_ops.h.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "omq_tree_ops.h"

namespace omq {
hipError_t launch_select(const omq_forest& f, const omq_wave& w, int W, float c_puct,
                         float virtual_loss, int max_depth, int vl_atomic, hipStream_t stream);
void select_set_options(int spin_limit);
int select_spin_limit();
hipError_t launch_leaf_info(const omq_forest& f, const omq_wave& w, int W, hipStream_t st);
hipError_t launch_synth_eval(const omq_forest& f, const omq_wave& w, int W, float scale,
                             hipStream_t st);
hipError_t launch_expand(const omq_forest& f, const omq_wave& w, int W, float virtual_loss,
                         int policy, const double* noise, double eps, hipStream_t st);
hipError_t launch_backup(const omq_forest& f, const omq_wave& w, int W, float virtual_loss,
                         int sign_mode, int w_mode, hipStream_t st);
bool expand_backup_fusable(const omq_forest& f, int policy, int w_mode);
hipError_t launch_expand_backup(const omq_forest& f, const omq_wave& w, int W,
                                float virtual_loss, const double* noise, double eps,
                                int sign_mode, hipStream_t st);
hipError_t launch_paths_backup(const omq_forest& f, const int32_t* paths, const int32_t* plen,
                               const int32_t* tree_of, const float* values, int batch,
                               int max_depth, int sign_mode, hipStream_t st);
hipError_t launch_virtual_loss(const omq_forest& f, const int32_t* nodes, const int32_t* tree_of,
                               int count, int delta, hipStream_t st);
hipError_t launch_reset(const omq_forest& f, hipStream_t st);
hipError_t launch_shift_root(const omq_forest& f, const int32_t* new_roots, int32_t* ws,
                             hipStream_t st);
hipError_t shift_scratch(int32_t** out);
hipError_t launch_root_policy(const omq_forest& f, double* pol, hipStream_t st);
hipError_t launch_sample_actions(const omq_forest& f, const double* pol, double temperature,
                                 uint64_t seed, uint64_t counter, int32_t* actions,
                                 hipStream_t st);
hipError_t launch_root_dirichlet(const omq_forest& f, double alpha, uint64_t seed,
                                 uint64_t counter, double* noise, hipStream_t st);
hipError_t launch_gomoku_terminal(const omq_forest& f, const omq_wave& w, const int8_t* boards,
                                  const int32_t* root_player, int rule, int bs, int32_t* uterm,
                                  hipStream_t st);
hipError_t launch_go_rules(const omq_forest& f, const omq_wave& w, const int8_t* boards,
                           const int32_t* root_player, const int32_t* root_passes,
                           const int32_t* root_ko, int flags, int bs, int32_t* uterm,
                           hipStream_t st);
hipError_t launch_leaf_features(const omq_forest& f, const omq_wave& w, const int8_t* boards,
                                const int32_t* root_player, const int32_t* root_moves, int bs,
                                int planes, int dtype, int nhwc, void* out, hipStream_t st);
hipError_t launch_fused_ucb(const int32_t* node_indices, int batch, const int32_t* starts,
                            const int32_t* ends, const int32_t* children, const float* q,
                            const int32_t* visits, const float* priors, float c_puct,
                            int32_t* selected, hipStream_t st);
hipError_t launch_find_expansion_nodes(const int32_t* current_nodes, const uint8_t* valid_mask,
                                       int wave_size, const int32_t* children, int max_children,
                                       const int32_t* visit_counts, int num_nodes,
                                       int32_t* out_nodes, int32_t* out_count, hipStream_t st);
hipError_t launch_batched_ucb(const float* q_values, const int32_t* visit_counts,
                              int num_children, const int32_t* parent_visits,
                              const float* priors, const int32_t* row_ptr,
                              const int32_t* col_indices, int batch, float c_puct,
                              int32_t* selected, float* scores, hipStream_t st);
hipError_t launch_fused_select_expand(const int32_t* roots, int num_paths,
                                      const int32_t* children, int num_nodes, int max_children,
                                      const int32_t* visit_counts, const float* q_values,
                                      const float* prior_probs, const uint8_t* is_expanded,
                                      int max_depth, float c_puct, int32_t* paths,
                                      int32_t* path_lengths, int32_t* expand_nodes,
                                      uint8_t* needs_expansion, hipStream_t st);
hipError_t launch_fused_select_expand_opt(const int32_t* roots, int num_paths,
                                          const int32_t* children, int num_nodes,
                                          int max_children, const int32_t* visit_counts,
                                          const float* value_sums, const float* priors,
                                          int max_depth, float c_puct, float* ucb_scores,
                                          int32_t* paths, int32_t* path_lengths,
                                          hipStream_t st);
hipError_t launch_parallel_select_vl(const int32_t* parent_nodes, int num_sims,
                                     const int32_t* children, int num_rows, int max_children,
                                     int children_stride, const int32_t* visit_counts,
                                     const int32_t* vl_counts, const float* value_sums,
                                     int num_nodes, const float* priors, int priors_stride,
                                     const uint8_t* legal_masks, int action_space,
                                     const int32_t* child_actions, float c_puct, float vl_value,
                                     int32_t* selected, hipStream_t st);
hipError_t launch_fused_ucb_noise(const float* q_values, const int32_t* visit_counts,
                                  const float* priors, int num_children, const float* noise,
                                  int num_sims, float parent_visits_sqrt, float c_puct,
                                  float epsilon, int32_t* selected, hipStream_t st);
hipError_t launch_batched_ucb_dense(const int32_t* batch_children, const float* batch_priors,
                                    const int32_t* parent_visits, const uint8_t* valid_mask,
                                    int batch, int max_children, const int32_t* child_visits,
                                    const float* child_values, int num_valid, float c_puct,
                                    int32_t* selected, hipStream_t st);
hipError_t launch_batched_dirichlet(int num_sims, int num_actions, double alpha, uint64_t seed,
                                    uint64_t counter, float* noise, hipStream_t st);
hipError_t launch_bfs_subtree(const int32_t* row_ptr, const int32_t* col, int num_edges,
                              int root, int max_nodes, uint8_t* in_subtree, int32_t* remap,
                              int32_t* count, int32_t* ws, hipStream_t st);
hipError_t launch_extract_edges(const int32_t* row_ptr, const int32_t* col, const int16_t* actions,
                                int num_edges, const uint8_t* in_subtree, const int32_t* remap,
                                int num_nodes, int max_edges, int32_t* out_parent,
                                int32_t* out_child, int16_t* out_action, int32_t* edge_count,
                                int32_t* ws, hipStream_t st);
hipError_t launch_batched_add_children(
    const int32_t* parent_indices, int batch, const int32_t* actions, const float* priors,
    const int32_t* num_children, int32_t* node_counter, int32_t* edge_counter,
    int32_t* children, int32_t* parent_indices_out, int32_t* parent_actions_out,
    float* node_priors_out, int32_t* visit_counts_out, float* value_sums_out,
    int32_t* col_indices, int32_t* edge_actions, float* edge_priors, int max_nodes,
    int max_children, int max_edges, int32_t* child_indices, hipStream_t st);
size_t leaf_lds_per_wave_host(const omq_forest& f);
}  // namespace omq

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return OMQ_OK;
  return fail(OMQ_E_LAUNCH, "%s: %s", what, hipGetErrorString(e));
}

int check_forest(const omq_forest* f) {
  if (!f) return fail(OMQ_E_ARG, "forest is null");
  if (f->num_trees <= 0 || f->capacity <= 0)
    return fail(OMQ_E_ARG, "num_trees (%d) and capacity (%d) must be positive", f->num_trees,
                f->capacity);
  if (f->num_actions <= 0 || f->num_actions > OMQ_MAX_ACTIONS)
    return fail(OMQ_E_LIMIT, "num_actions %d outside [1, %d]", f->num_actions, OMQ_MAX_ACTIONS);
  if (f->game != OMQ_GAME_BOARD && f->game != OMQ_GAME_GO && f->game != OMQ_GAME_SPARSE)
    return fail(OMQ_E_ARG, "unknown game model %d", f->game);
  if (f->game != OMQ_GAME_SPARSE) {
    if (f->legal_words != (f->num_actions + 31) / 32)
      return fail(OMQ_E_ARG, "legal_words %d != ceil(num_actions/32) = %d", f->legal_words,
                  (f->num_actions + 31) / 32);
    if (f->num_actions > OMQ_MAX_ROW + (f->game == OMQ_GAME_GO ? 1 : 0))
      return fail(OMQ_E_LIMIT, "board with %d actions exceeds the row limit %d", f->num_actions,
                  OMQ_MAX_ROW);
  } else {
    if (f->min_legal < 1 || f->max_legal < f->min_legal || f->max_legal > 64 ||
        f->max_legal > f->num_actions)
      return fail(OMQ_E_ARG, "sparse legal range [%d, %d] must lie in [1, min(64, A)]",
                  f->min_legal, f->max_legal);
  }
  if (!f->visit_counts || !f->value_sums || !f->priors || !f->parents || !f->first_child ||
      !f->num_children || !f->actions || !f->num_nodes || !f->root_keys)
    return fail(OMQ_E_ARG, "forest has a null array");
  if (f->game != OMQ_GAME_SPARSE && !f->root_legal)
    return fail(OMQ_E_ARG, "board forest without root_legal");
  return OMQ_OK;
}

// The reference-style primitives touch visit_counts (and value_sums) only.
int check_forest_nw(const omq_forest* f, bool need_w) {
  if (!f) return fail(OMQ_E_ARG, "forest is null");
  if (f->num_trees <= 0 || f->capacity <= 0)
    return fail(OMQ_E_ARG, "num_trees (%d) and capacity (%d) must be positive", f->num_trees,
                f->capacity);
  if (!f->visit_counts || (need_w && !f->value_sums))
    return fail(OMQ_E_ARG, "forest has a null array");
  return OMQ_OK;
}

int check_wave(const omq_forest* f, const omq_wave* w, int wave_size) {
  if (!w) return fail(OMQ_E_ARG, "wave buffers are null");
  if (w->max_wave <= 0 || w->max_wave > OMQ_MAX_WAVE)
    return fail(OMQ_E_LIMIT, "max_wave %d outside [1, %d]", w->max_wave, OMQ_MAX_WAVE);
  if (w->max_depth <= 0 || w->max_depth > OMQ_MAX_DEPTH)
    return fail(OMQ_E_LIMIT, "max_depth %d outside [1, %d]", w->max_depth, OMQ_MAX_DEPTH);
  if (wave_size <= 0 || wave_size > w->max_wave)
    return fail(OMQ_E_ARG, "wave_size %d outside [1, max_wave=%d]", wave_size, w->max_wave);
  if (!w->paths || !w->path_len || !w->leaves || !w->sim_uid || !w->uleaf || !w->ufirst ||
      !w->ucount || !w->glog || !w->gcount || !w->gmembers || !w->ukey || !w->ulegal ||
      !w->uedge || !w->unew || !w->policy || !w->values || !w->sim_value || !w->stats ||
      !w->status || !w->sel_scratch)
    return fail(OMQ_E_ARG, "wave buffers have a null array");
  (void)f;
  return OMQ_OK;
}

int check_leaf_lds(const omq_forest* f) {
  if (omq::leaf_lds_per_wave_host(*f) > 64 * 1024)
    return fail(OMQ_E_LIMIT, "per-leaf LDS need %zu bytes exceeds 64 KiB",
                omq::leaf_lds_per_wave_host(*f));
  return OMQ_OK;
}

}  // namespace

extern "C" {

int omq_abi_version(void) { return OMQ_ABI_VERSION; }

const char* omq_last_error(void) { return g_err.c_str(); }

int omq_forest_reset(const omq_forest* f, void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  return hip_status(omq::launch_reset(*f, (hipStream_t)stream), "omq_forest_reset");
}

int omq_select(const omq_forest* f, const omq_wave* w, int32_t wave_size, float c_puct,
               float virtual_loss, int32_t max_depth, int32_t vl_atomic, void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  rc = check_wave(f, w, wave_size);
  if (rc) return rc;
  if (max_depth <= 0 || max_depth > w->max_depth)
    return fail(OMQ_E_ARG, "max_depth %d outside [1, wave max_depth=%d]", max_depth,
                w->max_depth);
  if (!(virtual_loss >= 0.0f) || virtual_loss > 1048576.0f)
    return fail(OMQ_E_ARG, "virtual_loss %g must be in [0, 2^20]", (double)virtual_loss);
  return hip_status(omq::launch_select(*f, *w, wave_size, c_puct, virtual_loss, max_depth,
                                       vl_atomic ? 1 : 0, (hipStream_t)stream),
                    "omq_select");
}

int omq_select_options(int32_t spin_limit) {
  if (spin_limit < 0) return fail(OMQ_E_ARG, "spin_limit %d < 0", spin_limit);
  omq::select_set_options(spin_limit);
  return OMQ_OK;
}

int32_t omq_select_spin_limit(void) { return omq::select_spin_limit(); }

int omq_wall_clock_khz(int32_t* khz) {
  if (khz == nullptr) return fail(OMQ_E_ARG, "khz is null");
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&v, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
    return fail(OMQ_E_LAUNCH, "hipDeviceGetAttribute(WallClockRate) failed");
  *khz = v;
  return OMQ_OK;
}

int omq_leaf_info(const omq_forest* f, const omq_wave* w, void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  rc = check_wave(f, w, w ? w->max_wave : 1);
  if (rc) return rc;
  rc = check_leaf_lds(f);
  if (rc) return rc;
  return hip_status(omq::launch_leaf_info(*f, *w, w->max_wave, (hipStream_t)stream),
                    "omq_leaf_info");
}

int omq_gomoku_terminal(const omq_forest* f, const omq_wave* w, const int8_t* root_boards,
                        const int32_t* root_player, int32_t rule, int32_t* uterminal,
                        void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  rc = check_wave(f, w, w ? w->max_wave : 1);
  if (rc) return rc;
  if (f->game != OMQ_GAME_BOARD)
    return fail(OMQ_E_ARG, "omq_gomoku_terminal needs a board forest (game %d)", f->game);
  int bs = 0;
  while ((bs + 1) * (bs + 1) <= f->num_actions) ++bs;
  if (bs * bs != f->num_actions)
    return fail(OMQ_E_ARG, "num_actions %d is not a square board", f->num_actions);
  if (!root_boards) return fail(OMQ_E_ARG, "root_boards is null");
  if (rule != OMQ_RULE_FREESTYLE && rule != OMQ_RULE_RENJU)
    return fail(OMQ_E_ARG, "unknown gomoku rule %d", rule);
  return hip_status(omq::launch_gomoku_terminal(*f, *w, root_boards, root_player, rule, bs,
                                                uterminal, (hipStream_t)stream),
                    "omq_gomoku_terminal");
}

int omq_go_rules(const omq_forest* f, const omq_wave* w, const int8_t* root_boards,
                 const int32_t* root_player, const int32_t* root_passes, const int32_t* root_ko,
                 int32_t flags, int32_t* uterminal, void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  rc = check_wave(f, w, w ? w->max_wave : 1);
  if (rc) return rc;
  if (f->game != OMQ_GAME_GO)
    return fail(OMQ_E_ARG, "omq_go_rules needs a Go forest (game %d)", f->game);
  int bs = 0;
  while ((bs + 1) * (bs + 1) <= f->num_actions - 1) ++bs;
  if (bs * bs + 1 != f->num_actions)
    return fail(OMQ_E_ARG, "num_actions %d is not a square board plus the pass", f->num_actions);
  if (!root_boards) return fail(OMQ_E_ARG, "root_boards is required");
  if (!w->umask) return fail(OMQ_E_ARG, "omq_go_rules writes the wave's umask: it is null");
  if (flags & ~(OMQ_GO_KO | OMQ_GO_SUICIDE)) return fail(OMQ_E_ARG, "unknown Go flags %d", flags);
  return hip_status(omq::launch_go_rules(*f, *w, root_boards, root_player, root_passes, root_ko,
                                         flags, bs, uterminal, (hipStream_t)stream),
                    "omq_go_rules");
}

int omq_leaf_features(const omq_forest* f, const omq_wave* w, const int8_t* root_boards,
                      const int32_t* root_player, const int32_t* root_moves, int32_t planes,
                      int32_t dtype, int32_t layout, void* out, void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  rc = check_wave(f, w, w ? w->max_wave : 1);
  if (rc) return rc;
  if (f->game != OMQ_GAME_BOARD)
    return fail(OMQ_E_ARG, "omq_leaf_features needs a board forest (game %d)", f->game);
  int bs = 0;
  while ((bs + 1) * (bs + 1) <= f->num_actions) ++bs;
  if (bs * bs != f->num_actions)
    return fail(OMQ_E_ARG, "num_actions %d is not a square board", f->num_actions);
  if (!root_boards || !out) return fail(OMQ_E_ARG, "root_boards and out are required");
  if (planes != 18 && planes != 19) return fail(OMQ_E_ARG, "planes %d is not 18 or 19", planes);
  if (dtype != OMQ_DTYPE_F32 && dtype != OMQ_DTYPE_BF16)
    return fail(OMQ_E_ARG, "unknown feature dtype %d", dtype);
  if (layout != OMQ_LAYOUT_NCHW && layout != OMQ_LAYOUT_NHWC)
    return fail(OMQ_E_ARG, "unknown feature layout %d", layout);
  const uintptr_t align = dtype == OMQ_DTYPE_F32 ? 8 : 4;
  if ((uintptr_t)out % align != 0)
    return fail(OMQ_E_ARG, "out must be aligned to %d bytes", (int)align);
  return hip_status(omq::launch_leaf_features(*f, *w, root_boards, root_player, root_moves, bs,
                                              planes, dtype, layout == OMQ_LAYOUT_NHWC, out,
                                              (hipStream_t)stream),
                    "omq_leaf_features");
}

int omq_shift_root(const omq_forest* f, const int32_t* new_roots, int32_t* workspace,
                   int64_t workspace_ints, void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  if (!new_roots || !workspace) return fail(OMQ_E_ARG, "new_roots and workspace are required");
  const int64_t need = (int64_t)OMQ_SHIFT_WORKSPACE_PER_NODE * f->num_trees * f->capacity;
  if (workspace_ints < need)
    return fail(OMQ_E_ARG, "workspace holds %lld int32, omq_shift_root needs %lld",
                (long long)workspace_ints, (long long)need);
  return hip_status(omq::launch_shift_root(*f, new_roots, workspace, (hipStream_t)stream),
                    "omq_shift_root");
}

int omq_shift_root_noalloc(const omq_forest* f, const int32_t* new_roots, void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  if (!new_roots) return fail(OMQ_E_ARG, "new_roots is required");
  const int64_t need = (int64_t)OMQ_SHIFT_WORKSPACE_PER_NODE * f->num_trees * f->capacity;
  if (need > (int64_t)OMQ_NOALLOC_SHIFT_INTS)
    return fail(OMQ_E_LIMIT,
                "omq_shift_root_noalloc: %d trees x capacity %d needs %lld workspace int32, the "
                "library's own workspace holds %d (use omq_shift_root with a workspace)",
                f->num_trees, f->capacity, (long long)need, OMQ_NOALLOC_SHIFT_INTS);
  int32_t* ws = nullptr;
  rc = hip_status(omq::shift_scratch(&ws), "omq_shift_root_noalloc (workspace lookup)");
  if (rc) return rc;
  return hip_status(omq::launch_shift_root(*f, new_roots, ws, (hipStream_t)stream),
                    "omq_shift_root_noalloc");
}

int omq_root_policy(const omq_forest* f, double* policy, void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  if (!policy) return fail(OMQ_E_ARG, "policy is null");
  return hip_status(omq::launch_root_policy(*f, policy, (hipStream_t)stream), "omq_root_policy");
}

int omq_sample_actions(const omq_forest* f, const double* policy, double temperature,
                       uint64_t seed, uint64_t counter, int32_t* actions, void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  if (!policy || !actions) return fail(OMQ_E_ARG, "policy and actions are required");
  if (!(temperature >= 0.0) || temperature > 1e6)
    return fail(OMQ_E_ARG, "temperature %g outside [0, 1e6]", temperature);
  return hip_status(omq::launch_sample_actions(*f, policy, temperature, seed, counter, actions,
                                               (hipStream_t)stream),
                    "omq_sample_actions");
}

int omq_root_dirichlet(const omq_forest* f, double alpha, uint64_t seed, uint64_t counter,
                       double* noise, void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  if (!noise) return fail(OMQ_E_ARG, "noise is null");
  if (!(alpha > 0.0) || alpha > 1e6) return fail(OMQ_E_ARG, "alpha %g outside (0, 1e6]", alpha);
  return hip_status(omq::launch_root_dirichlet(*f, alpha, seed, counter, noise,
                                               (hipStream_t)stream),
                    "omq_root_dirichlet");
}

int omq_synthetic_evaluate(const omq_forest* f, const omq_wave* w, float logit_scale,
                           void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  rc = check_wave(f, w, w ? w->max_wave : 1);
  if (rc) return rc;
  rc = check_leaf_lds(f);
  if (rc) return rc;
  return hip_status(
      omq::launch_synth_eval(*f, *w, w->max_wave, logit_scale, (hipStream_t)stream),
      "omq_synthetic_evaluate");
}

int omq_expand(const omq_forest* f, const omq_wave* w, int32_t wave_size, float virtual_loss,
               int32_t expand_policy, const double* root_noise, double dirichlet_epsilon,
               void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  rc = check_wave(f, w, wave_size);
  if (rc) return rc;
  rc = check_leaf_lds(f);
  if (rc) return rc;
  if (expand_policy != OMQ_EXPAND_FULL && expand_policy != OMQ_EXPAND_REFERENCE_PW)
    return fail(OMQ_E_ARG, "unknown expansion policy %d", expand_policy);
  if (!(dirichlet_epsilon >= 0.0 && dirichlet_epsilon <= 1.0))
    return fail(OMQ_E_ARG, "dirichlet_epsilon %g outside [0, 1]", dirichlet_epsilon);
  return hip_status(omq::launch_expand(*f, *w, wave_size, virtual_loss, expand_policy,
                                       root_noise, dirichlet_epsilon, (hipStream_t)stream),
                    "omq_expand");
}

int omq_backup(const omq_forest* f, const omq_wave* w, int32_t wave_size, float virtual_loss,
               int32_t sign_mode, int32_t w_mode, void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  rc = check_wave(f, w, wave_size);
  if (rc) return rc;
  if (sign_mode != OMQ_SIGN_LEAF_POSITIVE && sign_mode != OMQ_SIGN_ROOT_POSITIVE)
    return fail(OMQ_E_ARG, "unknown sign mode %d", sign_mode);
  if (w_mode != OMQ_WACC_ORDERED && w_mode != OMQ_WACC_ATOMIC)
    return fail(OMQ_E_ARG, "unknown W accumulation mode %d", w_mode);
  return hip_status(omq::launch_backup(*f, *w, wave_size, virtual_loss, sign_mode, w_mode,
                                       (hipStream_t)stream),
                    "omq_backup");
}

int omq_expand_backup(const omq_forest* f, const omq_wave* w, int32_t wave_size,
                      float virtual_loss, int32_t expand_policy, const double* root_noise,
                      double dirichlet_epsilon, int32_t sign_mode, int32_t w_mode,
                      void* stream) {
  int rc = check_forest(f);
  if (rc) return rc;
  rc = check_wave(f, w, wave_size);
  if (rc) return rc;
  rc = check_leaf_lds(f);
  if (rc) return rc;
  if (expand_policy != OMQ_EXPAND_FULL && expand_policy != OMQ_EXPAND_REFERENCE_PW)
    return fail(OMQ_E_ARG, "unknown expansion policy %d", expand_policy);
  if (!(dirichlet_epsilon >= 0.0 && dirichlet_epsilon <= 1.0))
    return fail(OMQ_E_ARG, "dirichlet_epsilon %g outside [0, 1]", dirichlet_epsilon);
  if (sign_mode != OMQ_SIGN_LEAF_POSITIVE && sign_mode != OMQ_SIGN_ROOT_POSITIVE)
    return fail(OMQ_E_ARG, "unknown sign mode %d", sign_mode);
  if (w_mode != OMQ_WACC_ORDERED && w_mode != OMQ_WACC_ATOMIC)
    return fail(OMQ_E_ARG, "unknown W accumulation mode %d", w_mode);
  if (omq::expand_backup_fusable(*f, expand_policy, w_mode))
    return hip_status(omq::launch_expand_backup(*f, *w, wave_size, virtual_loss, root_noise,
                                                dirichlet_epsilon, sign_mode,
                                                (hipStream_t)stream),
                      "omq_expand_backup");
  rc = hip_status(omq::launch_expand(*f, *w, wave_size, virtual_loss, expand_policy, root_noise,
                                     dirichlet_epsilon, (hipStream_t)stream),
                  "omq_expand_backup");
  if (rc) return rc;
  return hip_status(omq::launch_backup(*f, *w, wave_size, virtual_loss, sign_mode, w_mode,
                                       (hipStream_t)stream),
                    "omq_expand_backup");
}

int omq_paths_backup(const omq_forest* f, const int32_t* paths, const int32_t* path_len,
                     const int32_t* tree_of, const float* values, int32_t batch,
                     int32_t max_depth, int32_t sign_mode, void* stream) {
  int rc = check_forest_nw(f, true);
  if (rc) return rc;
  if (batch < 0 || max_depth <= 0) return fail(OMQ_E_ARG, "batch/max_depth out of range");
  if (batch == 0) return OMQ_OK;
  if (!paths || !path_len || !values) return fail(OMQ_E_ARG, "null path arrays");
  if (sign_mode != OMQ_SIGN_LEAF_POSITIVE && sign_mode != OMQ_SIGN_ROOT_POSITIVE)
    return fail(OMQ_E_ARG, "unknown sign mode %d", sign_mode);
  return hip_status(omq::launch_paths_backup(*f, paths, path_len, tree_of, values, batch,
                                             max_depth, sign_mode, (hipStream_t)stream),
                    "omq_paths_backup");
}

int omq_virtual_loss(const omq_forest* f, const int32_t* nodes, const int32_t* tree_of,
                     int32_t count, int32_t delta, void* stream) {
  int rc = check_forest_nw(f, false);
  if (rc) return rc;
  if (count < 0) return fail(OMQ_E_ARG, "count %d < 0", count);
  if (count == 0) return OMQ_OK;
  if (!nodes) return fail(OMQ_E_ARG, "null node list");
  return hip_status(omq::launch_virtual_loss(*f, nodes, tree_of, count, delta,
                                             (hipStream_t)stream),
                    "omq_virtual_loss");
}

int omq_fused_ucb_selection(const int32_t* node_indices, int32_t batch,
                            const int32_t* children_start, const int32_t* children_end,
                            const int32_t* children, const float* q_values,
                            const int32_t* visit_counts, const float* priors, float c_puct,
                            int32_t* selected, void* stream) {
  if (batch < 0) return fail(OMQ_E_ARG, "batch %d < 0", batch);
  if (batch == 0) return OMQ_OK;
  if (!node_indices || !children_start || !children_end || !children || !q_values ||
      !visit_counts || !priors || !selected)
    return fail(OMQ_E_ARG, "omq_fused_ucb_selection: a null array");
  return hip_status(omq::launch_fused_ucb(node_indices, batch, children_start, children_end,
                                          children, q_values, visit_counts, priors, c_puct,
                                          selected, (hipStream_t)stream),
                    "omq_fused_ucb_selection");
}

int omq_find_expansion_nodes(const int32_t* current_nodes, const uint8_t* valid_mask,
                             int32_t wave_size, const int32_t* children, int32_t max_children,
                             const int32_t* visit_counts, int32_t num_nodes, int32_t* out_nodes,
                             int32_t* out_count, void* stream) {
  if (wave_size < 0 || max_children < 0 || num_nodes < 0)
    return fail(OMQ_E_ARG, "omq_find_expansion_nodes: wave_size %d, max_children %d, "
                "num_nodes %d must not be negative", wave_size, max_children, num_nodes);
  if (!out_count) return fail(OMQ_E_ARG, "omq_find_expansion_nodes: null count");
  if (wave_size > 0 && (!current_nodes || !valid_mask || !out_nodes ||
                        (num_nodes > 0 && (!visit_counts || (max_children > 0 && !children)))))
    return fail(OMQ_E_ARG, "omq_find_expansion_nodes: a null array");
  return hip_status(omq::launch_find_expansion_nodes(current_nodes, valid_mask, wave_size,
                                                     children, max_children, visit_counts,
                                                     num_nodes, out_nodes, out_count,
                                                     (hipStream_t)stream),
                    "omq_find_expansion_nodes");
}

int omq_batched_ucb_selection(const float* q_values, const int32_t* visit_counts,
                              int32_t num_children, const int32_t* parent_visits,
                              const float* priors, const int32_t* row_ptr,
                              const int32_t* col_indices, int32_t batch, float c_puct,
                              int32_t* selected, float* scores, void* stream) {
  if (batch < 0 || num_children < 0)
    return fail(OMQ_E_ARG, "omq_batched_ucb_selection: batch %d, num_children %d < 0", batch,
                num_children);
  if (batch == 0) return OMQ_OK;
  if (!parent_visits || !row_ptr || !selected ||
      (num_children > 0 && (!q_values || !visit_counts || !priors || !col_indices)))
    return fail(OMQ_E_ARG, "omq_batched_ucb_selection: a null array");
  return hip_status(omq::launch_batched_ucb(q_values, visit_counts, num_children, parent_visits,
                                            priors, row_ptr, col_indices, batch, c_puct,
                                            selected, scores, (hipStream_t)stream),
                    "omq_batched_ucb_selection");
}

int omq_fused_select_expand(const int32_t* roots, int32_t num_paths, const int32_t* children,
                            int32_t num_nodes, int32_t max_children,
                            const int32_t* visit_counts, const float* q_values,
                            const float* prior_probs, const uint8_t* is_expanded,
                            int32_t max_depth, float c_puct, int32_t* paths,
                            int32_t* path_lengths, int32_t* expand_nodes,
                            uint8_t* needs_expansion, void* stream) {
  if (num_paths < 0 || num_nodes < 0 || max_children < 0 || max_depth < 1)
    return fail(OMQ_E_ARG, "omq_fused_select_expand: num_paths %d, num_nodes %d, "
                "max_children %d must not be negative and max_depth %d >= 1", num_paths,
                num_nodes, max_children, max_depth);
  if (num_paths == 0) return OMQ_OK;
  if (!roots || !paths || !path_lengths || !expand_nodes || !needs_expansion ||
      (num_nodes > 0 && (!visit_counts || !q_values || !prior_probs || !is_expanded ||
                         (max_children > 0 && !children))))
    return fail(OMQ_E_ARG, "omq_fused_select_expand: a null array");
  return hip_status(omq::launch_fused_select_expand(roots, num_paths, children, num_nodes,
                                                    max_children, visit_counts, q_values,
                                                    prior_probs, is_expanded, max_depth,
                                                    c_puct, paths, path_lengths, expand_nodes,
                                                    needs_expansion, (hipStream_t)stream),
                    "omq_fused_select_expand");
}

int omq_fused_select_expand_optimized(const int32_t* roots, int32_t num_paths,
                                      const int32_t* children, int32_t num_nodes,
                                      int32_t max_children, const int32_t* visit_counts,
                                      const float* value_sums, const float* priors,
                                      int32_t max_depth, float c_puct, float* ucb_scores,
                                      int32_t* paths, int32_t* path_lengths, void* stream) {
  if (num_paths < 0 || num_nodes < 0 || max_children < 0 || max_depth < 1)
    return fail(OMQ_E_ARG, "omq_fused_select_expand_optimized: num_paths %d, num_nodes %d, "
                "max_children %d must not be negative and max_depth %d >= 1", num_paths,
                num_nodes, max_children, max_depth);
  if (num_paths == 0) return OMQ_OK;
  if (!roots || !paths || !path_lengths || (max_children > 0 && !ucb_scores) ||
      (num_nodes > 0 && (!visit_counts || !value_sums || !priors ||
                         (max_children > 0 && !children))))
    return fail(OMQ_E_ARG, "omq_fused_select_expand_optimized: a null array");
  return hip_status(omq::launch_fused_select_expand_opt(roots, num_paths, children, num_nodes,
                                                        max_children, visit_counts, value_sums,
                                                        priors, max_depth, c_puct, ucb_scores,
                                                        paths, path_lengths,
                                                        (hipStream_t)stream),
                    "omq_fused_select_expand_optimized");
}

int omq_batched_add_children(const int32_t* parent_indices, int32_t batch,
                             const int32_t* actions, const float* priors,
                             const int32_t* num_children, int32_t* node_counter,
                             int32_t* edge_counter, int32_t* children,
                             int32_t* parent_indices_out, int32_t* parent_actions_out,
                             float* node_priors_out, int32_t* visit_counts_out,
                             float* value_sums_out, int32_t* col_indices, int32_t* edge_actions,
                             float* edge_priors, int32_t max_nodes, int32_t max_children,
                             int32_t max_edges, int32_t* child_indices, void* stream) {
  if (batch < 0 || max_nodes < 0 || max_edges < 0 || max_children < 1)
    return fail(OMQ_E_ARG, "omq_batched_add_children: batch %d, max_nodes %d, max_edges %d "
                "must not be negative and max_children %d >= 1", batch, max_nodes, max_edges,
                max_children);
  if (batch == 0) return OMQ_OK;
  if (!parent_indices || !actions || !priors || !num_children || !node_counter ||
      !edge_counter || !child_indices ||
      (max_nodes > 0 && (!children || !parent_indices_out || !parent_actions_out ||
                         !node_priors_out || !visit_counts_out || !value_sums_out)) ||
      (max_edges > 0 && (!col_indices || !edge_actions || !edge_priors)))
    return fail(OMQ_E_ARG, "omq_batched_add_children: a null array");
  return hip_status(omq::launch_batched_add_children(
                        parent_indices, batch, actions, priors, num_children, node_counter,
                        edge_counter, children, parent_indices_out, parent_actions_out,
                        node_priors_out, visit_counts_out, value_sums_out, col_indices,
                        edge_actions, edge_priors, max_nodes, max_children, max_edges,
                        child_indices, (hipStream_t)stream),
                    "omq_batched_add_children");
}

}  // extern "C"

int omq_parallel_select_with_virtual_loss(
    const int32_t* parent_nodes, int32_t num_sims, const int32_t* children, int32_t num_rows,
    int32_t max_children, int32_t children_stride, const int32_t* visit_counts,
    int32_t* virtual_loss_counts, const float* value_sums, int32_t num_nodes,
    const float* priors, int32_t priors_stride, const uint8_t* legal_masks,
    int32_t action_space_size, const int32_t* child_actions, float c_puct,
    float virtual_loss_value, int32_t* selected_children, void* stream) {
  const char* who = "omq_parallel_select_with_virtual_loss";
  if (num_sims < 0 || num_rows < 0 || max_children < 0 || num_nodes < 0 || priors_stride < 0 ||
      action_space_size < 0 || children_stride < max_children)
    return fail(OMQ_E_ARG, "%s: num_sims %d, num_rows %d, max_children %d, num_nodes %d, "
                "priors_stride %d, action_space_size %d must not be negative and "
                "children_stride %d >= max_children", who, num_sims, num_rows, max_children,
                num_nodes, priors_stride, action_space_size, children_stride);
  if (num_sims == 0) return OMQ_OK;
  if (!parent_nodes || !selected_children ||
      (num_nodes > 0 && (!visit_counts || !virtual_loss_counts || !value_sums || !priors)) ||
      (num_rows > 0 && max_children > 0 && !children) ||
      (legal_masks && (!child_actions || action_space_size == 0)))
    return fail(OMQ_E_ARG, "%s: a null array", who);
  hipStream_t st = (hipStream_t)stream;
  int rc = hip_status(omq::launch_parallel_select_vl(parent_nodes, num_sims, children, num_rows,
                                                     max_children, children_stride,
                                                     visit_counts, virtual_loss_counts,
                                                     value_sums, num_nodes, priors,
                                                     priors_stride, legal_masks,
                                                     action_space_size, child_actions, c_puct,
                                                     virtual_loss_value, selected_children, st),
                      who);
  if (rc || num_nodes == 0) return rc;
  // the virtual loss of every selection, after all of them (selected ids outside the counts,
  // -1 included, are skipped)
  omq_forest vf{};
  vf.num_trees = 1;
  vf.capacity = num_nodes;
  vf.visit_counts = virtual_loss_counts;
  return hip_status(omq::launch_virtual_loss(vf, selected_children, nullptr, num_sims, 1, st),
                    who);
}

int omq_fused_ucb_with_noise(const float* q_values, const int32_t* visit_counts,
                             const float* priors, int32_t num_children,
                             const float* dirichlet_noise, int32_t num_sims,
                             float parent_visits_sqrt, float c_puct, float epsilon,
                             int32_t* selected, void* stream) {
  if (num_sims < 0 || num_children < 0)
    return fail(OMQ_E_ARG, "omq_fused_ucb_with_noise: num_sims %d, num_children %d < 0",
                num_sims, num_children);
  if (num_sims == 0) return OMQ_OK;
  if (!selected || (num_children > 0 && (!q_values || !visit_counts || !priors ||
                                         !dirichlet_noise)))
    return fail(OMQ_E_ARG, "omq_fused_ucb_with_noise: a null array");
  return hip_status(omq::launch_fused_ucb_noise(q_values, visit_counts, priors, num_children,
                                                dirichlet_noise, num_sims, parent_visits_sqrt,
                                                c_puct, epsilon, selected, (hipStream_t)stream),
                    "omq_fused_ucb_with_noise");
}

int omq_batched_ucb_selection_dense(const int32_t* batch_children, const float* batch_priors,
                                    const int32_t* parent_visits, const uint8_t* valid_mask,
                                    int32_t batch, int32_t max_children,
                                    const int32_t* child_visits, const float* child_values,
                                    int32_t num_valid_children, float c_puct,
                                    int32_t* selected, void* stream) {
  if (batch < 0 || max_children < 0 || num_valid_children < 0)
    return fail(OMQ_E_ARG, "omq_batched_ucb_selection_dense: batch %d, max_children %d, "
                "num_valid_children %d < 0", batch, max_children, num_valid_children);
  if (batch == 0) return OMQ_OK;
  if (!parent_visits || !selected ||
      (max_children > 0 && (!batch_children || !batch_priors || !valid_mask)) ||
      (num_valid_children > 0 && (!child_visits || !child_values)))
    return fail(OMQ_E_ARG, "omq_batched_ucb_selection_dense: a null array");
  return hip_status(omq::launch_batched_ucb_dense(batch_children, batch_priors, parent_visits,
                                                  valid_mask, batch, max_children, child_visits,
                                                  child_values, num_valid_children, c_puct,
                                                  selected, (hipStream_t)stream),
                    "omq_batched_ucb_selection_dense");
}

int omq_batched_dirichlet_noise(int32_t num_sims, int32_t num_actions, double alpha,
                                uint64_t seed, uint64_t counter, float* noise, void* stream) {
  if (num_sims < 0 || num_actions < 0)
    return fail(OMQ_E_ARG, "omq_batched_dirichlet_noise: num_sims %d, num_actions %d < 0",
                num_sims, num_actions);
  if (!(alpha > 0.0) || !(alpha < 1e300))
    return fail(OMQ_E_ARG, "omq_batched_dirichlet_noise: alpha %g must be positive and finite",
                alpha);
  if ((int64_t)num_sims * num_actions == 0) return OMQ_OK;
  if (!noise) return fail(OMQ_E_ARG, "omq_batched_dirichlet_noise: null output");
  return hip_status(omq::launch_batched_dirichlet(num_sims, num_actions, alpha, seed, counter,
                                                  noise, (hipStream_t)stream),
                    "omq_batched_dirichlet_noise");
}

int omq_optimized_backup_scatter(const int32_t* paths, const int32_t* path_lengths,
                                 const float* values, int32_t batch, int32_t max_depth,
                                 int32_t* visit_counts, float* value_sums, int32_t num_nodes,
                                 void* stream) {
  if (batch < 0 || max_depth <= 0 || num_nodes < 0)
    return fail(OMQ_E_ARG, "omq_optimized_backup_scatter: batch %d, num_nodes %d >= 0 and "
                "max_depth %d >= 1", batch, num_nodes, max_depth);
  if (batch == 0 || num_nodes == 0) return OMQ_OK;
  if (!paths || !path_lengths || !values || !visit_counts || !value_sums)
    return fail(OMQ_E_ARG, "omq_optimized_backup_scatter: a null array");
  omq_forest vf{};
  vf.num_trees = 1;
  vf.capacity = num_nodes;
  vf.visit_counts = visit_counts;
  vf.value_sums = value_sums;
  return hip_status(omq::launch_paths_backup(vf, paths, path_lengths, nullptr, values, batch,
                                             max_depth, OMQ_SIGN_LEAF_POSITIVE,
                                             (hipStream_t)stream),
                    "omq_optimized_backup_scatter");
}

int omq_parallel_bfs_subtree(const int32_t* row_ptr, const int32_t* col_indices,
                             int32_t num_edges, int32_t root_idx, int32_t max_nodes,
                             uint8_t* in_subtree, int32_t* node_remap, int32_t* subtree_count,
                             int32_t* workspace, int64_t workspace_ints, void* stream) {
  const char* who = "omq_parallel_bfs_subtree";
  if (max_nodes <= 0 || num_edges < 0)
    return fail(OMQ_E_ARG, "%s: max_nodes %d must be positive and num_edges %d >= 0", who,
                max_nodes, num_edges);
  if (root_idx < 0 || root_idx >= max_nodes)
    return fail(OMQ_E_ARG, "%s: root_idx %d outside [0, %d)", who, root_idx, max_nodes);
  if (!row_ptr || !in_subtree || !node_remap || !subtree_count || !workspace ||
      (num_edges > 0 && !col_indices))
    return fail(OMQ_E_ARG, "%s: a null array", who);
  const int64_t need = OMQ_BFS_WORKSPACE_INTS((int64_t)max_nodes);
  if (workspace_ints < need)
    return fail(OMQ_E_ARG, "%s: workspace holds %lld int32, it needs %lld", who,
                (long long)workspace_ints, (long long)need);
  return hip_status(omq::launch_bfs_subtree(row_ptr, col_indices, num_edges, root_idx, max_nodes,
                                            in_subtree, node_remap, subtree_count, workspace,
                                            (hipStream_t)stream),
                    who);
}

int omq_extract_subtree_edges(const int32_t* row_ptr, const int32_t* col_indices,
                              const int16_t* edge_actions, int32_t num_edges,
                              const uint8_t* in_subtree, const int32_t* node_remap,
                              int32_t num_nodes, int32_t max_edges, int32_t* edge_parents,
                              int32_t* edge_children, int16_t* edge_actions_out,
                              int32_t* edge_count, int32_t* workspace, int64_t workspace_ints,
                              void* stream) {
  const char* who = "omq_extract_subtree_edges";
  if (num_nodes < 0 || num_edges < 0 || max_edges < 0)
    return fail(OMQ_E_ARG, "%s: num_nodes %d, num_edges %d, max_edges %d < 0", who, num_nodes,
                num_edges, max_edges);
  if (!edge_count || !workspace || (num_nodes > 0 && (!row_ptr || !in_subtree || !node_remap)) ||
      (num_edges > 0 && !col_indices) ||
      (max_edges > 0 && (!edge_parents || !edge_children || !edge_actions_out)))
    return fail(OMQ_E_ARG, "%s: a null array", who);
  const int64_t need = OMQ_EDGES_WORKSPACE_INTS((int64_t)num_nodes);
  if (workspace_ints < need)
    return fail(OMQ_E_ARG, "%s: workspace holds %lld int32, it needs %lld", who,
                (long long)workspace_ints, (long long)need);
  return hip_status(omq::launch_extract_edges(row_ptr, col_indices, edge_actions, num_edges,
                                              in_subtree, node_remap, num_nodes, max_edges,
                                              edge_parents, edge_children, edge_actions_out,
                                              edge_count, workspace, (hipStream_t)stream),
                    who);
}
