// The torch operators of the tree library, registered from C++ (libomq_torch_ops.so, loaded with
// torch.ops.load_library): each checks its tensors and calls the C ABI (omq_tree_ops.h) on the
// caller's current HIP stream, so that a torch.ops call does not pass through Python.
//
//   omq::vectorized_backup, omq::warp_vectorized_backup      the reference's mcts:: operators
//   omq::fused_ucb_selection                                 (torch_custom_ops.py:26,71,108)
//   omq::batch_apply_virtual_loss, omq::batch_remove_virtual_loss
//                                      (batch_apply/remove_virtual_loss, mcts_kernels.cu:845-953)
//   omq::_alias_mcts(name)            registers the operator `name` under the reference's own
//                                     namespace as well (mcts::name), for a name no module took;
//                                     omq::_mcts_aliased(name) says whether it did
//
// Tensors must be contiguous and on one HIP device; host tensors are refused (the library has
// no CPU implementation).  The Meta kernels give the shapes only (no device work).
#include <torch/library.h>

#include <ATen/core/Tensor.h>
#include <ATen/ops/empty.h>
#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>

#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "omq_tree_ops.h"

namespace {

void check_rc(int rc, const char* what) {
  TORCH_CHECK(rc == OMQ_OK, what, ": ", omq_last_error());
}

// The tensors' common device (a HIP device); every tensor contiguous.
c10::Device check_tensors(const char* name, std::initializer_list<const at::Tensor*> ts) {
  const c10::Device dev = (*ts.begin())->device();
  TORCH_CHECK(dev.is_cuda(), "omq::", name, ": tensors must be on a HIP device (got ", dev, ")");
  for (const at::Tensor* t : ts) {
    TORCH_CHECK(t->device() == dev, "omq::", name, ": all tensors must be on ", dev);
    TORCH_CHECK(t->is_contiguous(), "omq::", name, ": tensors must be contiguous");
  }
  return dev;
}

void check_dtype(const char* name, const char* arg, const at::Tensor& t, at::ScalarType want) {
  TORCH_CHECK(t.scalar_type() == want, "omq::", name, ": ", arg, " must be ", want, ", not ",
              t.scalar_type());
}

void* stream_of(c10::Device dev) { return c10::hip::getCurrentHIPStream(dev.index()).stream(); }

// A one-tree forest over a count array (and a value-sum array): what omq_paths_backup and
// omq_virtual_loss read.
omq_forest count_forest(const at::Tensor& counts, const at::Tensor* sums) {
  omq_forest f{};
  f.num_trees = 1;
  f.capacity = (int32_t)counts.numel();
  f.visit_counts = counts.data_ptr<int32_t>();
  if (sums != nullptr) f.value_sums = sums->data_ptr<float>();
  return f;
}

void backup_impl(const char* name, const at::Tensor& paths, const at::Tensor& path_lengths,
                 const at::Tensor& values, const at::Tensor& visit_counts,
                 const at::Tensor& value_sums) {
  const c10::Device dev =
      check_tensors(name, {&paths, &path_lengths, &values, &visit_counts, &value_sums});
  TORCH_CHECK(paths.dim() == 2 && paths.scalar_type() == at::kInt &&
                  path_lengths.scalar_type() == at::kInt,
              "omq::", name, ": paths int32 [B, D], path_lengths int32 [B]");
  TORCH_CHECK(values.scalar_type() == at::kFloat && visit_counts.scalar_type() == at::kInt &&
                  value_sums.scalar_type() == at::kFloat,
              "omq::", name, ": values/value_sums float32, visit_counts int32");
  const int64_t B = paths.size(0), D = paths.size(1);
  TORCH_CHECK(path_lengths.numel() == B && values.numel() == B, "omq::", name,
              ": one length and one value per path");
  TORCH_CHECK(visit_counts.numel() == value_sums.numel(), "omq::", name,
              ": visit_counts and value_sums differ in size");
  if (B == 0 || visit_counts.numel() == 0) return;
  const c10::hip::HIPGuard guard(dev.index());
  const omq_forest f = count_forest(visit_counts, &value_sums);
  check_rc(omq_paths_backup(&f, paths.data_ptr<int32_t>(), path_lengths.data_ptr<int32_t>(),
                            nullptr, values.data_ptr<float>(), (int32_t)B,
                            (int32_t)std::max<int64_t>(D, 1), OMQ_SIGN_LEAF_POSITIVE,
                            stream_of(dev)),
           "omq_paths_backup");
}

// mcts_kernels.cu:121-158 (sign by distance from the leaf); the warp variant
// (mcts_kernels.cu:164-230) never leaves out a lane, so it adds the same terms
void vectorized_backup(const at::Tensor& paths, const at::Tensor& path_lengths,
                       const at::Tensor& values, const at::Tensor& visit_counts,
                       const at::Tensor& value_sums) {
  backup_impl("vectorized_backup", paths, path_lengths, values, visit_counts, value_sums);
}

void warp_vectorized_backup(const at::Tensor& paths, const at::Tensor& path_lengths,
                            const at::Tensor& values, const at::Tensor& visit_counts,
                            const at::Tensor& value_sums) {
  backup_impl("warp_vectorized_backup", paths, path_lengths, values, visit_counts, value_sums);
}

void virtual_loss_impl(const char* name, const at::Tensor& node_indices,
                       const at::Tensor& counts, int delta) {
  const c10::Device dev = check_tensors(name, {&node_indices, &counts});
  TORCH_CHECK(node_indices.scalar_type() == at::kInt && counts.scalar_type() == at::kInt,
              "omq::", name, ": node_indices and virtual_loss_counts must be int32");
  const int64_t n = node_indices.numel();
  if (n == 0 || counts.numel() == 0) return;
  const c10::hip::HIPGuard guard(dev.index());
  const omq_forest f = count_forest(counts, nullptr);
  check_rc(omq_virtual_loss(&f, node_indices.data_ptr<int32_t>(), nullptr, (int32_t)n, delta,
                            stream_of(dev)),
           "omq_virtual_loss");
}

void batch_apply_virtual_loss(const at::Tensor& node_indices,
                              const at::Tensor& virtual_loss_counts) {
  virtual_loss_impl("batch_apply_virtual_loss", node_indices, virtual_loss_counts, 1);
}

void batch_remove_virtual_loss(const at::Tensor& node_indices,
                               const at::Tensor& virtual_loss_counts) {
  virtual_loss_impl("batch_remove_virtual_loss", node_indices, virtual_loss_counts, -1);
}

// torch_custom_ops.py:108-193 (kernel mcts_kernels.cu:1466-1512): per parent, the row position
// of the first maximum of q + c*P*sqrt(N_parent)/(1+n), q = 0 for an unvisited child
at::Tensor fused_ucb_selection(const at::Tensor& node_indices, const at::Tensor& children_start,
                               const at::Tensor& children_end, const at::Tensor& children,
                               const at::Tensor& q_values, const at::Tensor& visit_counts,
                               const at::Tensor& priors, double c_puct) {
  const char* name = "fused_ucb_selection";
  const c10::Device dev = check_tensors(name, {&node_indices, &children_start, &children_end,
                                               &children, &q_values, &visit_counts, &priors});
  check_dtype(name, "node_indices", node_indices, at::kInt);
  check_dtype(name, "children_start", children_start, at::kInt);
  check_dtype(name, "children_end", children_end, at::kInt);
  check_dtype(name, "children", children, at::kInt);
  check_dtype(name, "q_values", q_values, at::kFloat);
  check_dtype(name, "visit_counts", visit_counts, at::kInt);
  check_dtype(name, "priors", priors, at::kFloat);
  at::Tensor selected =
      at::empty({node_indices.numel()}, node_indices.options().dtype(at::kInt));
  const c10::hip::HIPGuard guard(dev.index());
  check_rc(omq_fused_ucb_selection(node_indices.data_ptr<int32_t>(),
                                   (int32_t)node_indices.numel(),
                                   children_start.data_ptr<int32_t>(),
                                   children_end.data_ptr<int32_t>(),
                                   children.data_ptr<int32_t>(), q_values.data_ptr<float>(),
                                   visit_counts.data_ptr<int32_t>(), priors.data_ptr<float>(),
                                   (float)c_puct, selected.data_ptr<int32_t>(), stream_of(dev)),
           "omq_fused_ucb_selection");
  return selected;
}

// Meta kernels: shapes only
void backup_meta(const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                 const at::Tensor&) {}
void virtual_loss_meta(const at::Tensor&, const at::Tensor&) {}
at::Tensor fused_ucb_meta(const at::Tensor& node_indices, const at::Tensor&, const at::Tensor&,
                          const at::Tensor&, const at::Tensor&, const at::Tensor&,
                          const at::Tensor&, double) {
  return at::empty({node_indices.numel()}, node_indices.options().dtype(at::kInt));
}

constexpr const char* kBackupSchema =
    "(Tensor paths, Tensor path_lengths, Tensor values, Tensor(a!) visit_counts, "
    "Tensor(b!) value_sums) -> ()";
constexpr const char* kVirtualLossSchema =
    "(Tensor node_indices, Tensor(a!) virtual_loss_counts) -> ()";
constexpr const char* kFusedUcbSchema =
    "(Tensor node_indices, Tensor children_start, Tensor children_end, Tensor children, "
    "Tensor q_values, Tensor visit_counts, Tensor priors, float c_puct) -> Tensor";

// Defines `name` in library m and registers its kernels (host and HIP tensors reach the same
// function, which refuses host tensors; Meta gives the shapes).
template <class Fn, class Meta>
void define(torch::Library& m, const char* name, const char* schema, Fn fn, Meta meta) {
  m.def((std::string(name) + schema).c_str());
  m.impl(name, torch::dispatch(c10::DispatchKey::CUDA, fn));
  m.impl(name, torch::dispatch(c10::DispatchKey::CPU, fn));
  m.impl(name, torch::dispatch(c10::DispatchKey::Meta, meta));
}

void define_op(torch::Library& m, const std::string& name) {
  if (name == "vectorized_backup")
    define(m, "vectorized_backup", kBackupSchema, vectorized_backup, backup_meta);
  else if (name == "warp_vectorized_backup")
    define(m, "warp_vectorized_backup", kBackupSchema, warp_vectorized_backup, backup_meta);
  else if (name == "fused_ucb_selection")
    define(m, "fused_ucb_selection", kFusedUcbSchema, fused_ucb_selection, fused_ucb_meta);
  else if (name == "batch_apply_virtual_loss")
    define(m, "batch_apply_virtual_loss", kVirtualLossSchema, batch_apply_virtual_loss,
           virtual_loss_meta);
  else if (name == "batch_remove_virtual_loss")
    define(m, "batch_remove_virtual_loss", kVirtualLossSchema, batch_remove_virtual_loss,
           virtual_loss_meta);
  else
    TORCH_CHECK(false, "omq::_alias_mcts: no operator ", name);
}

// The mcts:: registrations made by _alias_mcts (kept for the life of the process).
std::mutex g_alias_mutex;
std::vector<std::unique_ptr<torch::Library>> g_aliases;
std::vector<std::string> g_aliased;

// Registers omq::name under the reference's namespace too.  The caller checks first that no
// module (the reference's own, imported first) took mcts::name.  Returns false when this
// library registered it already.
bool alias_mcts(const std::string& name) {
  const std::lock_guard<std::mutex> lock(g_alias_mutex);
  for (const std::string& n : g_aliased)
    if (n == name) return false;
  auto lib = std::make_unique<torch::Library>(torch::Library::FRAGMENT, "mcts", std::nullopt,
                                              __FILE__, __LINE__);
  define_op(*lib, name);
  g_aliases.push_back(std::move(lib));
  g_aliased.push_back(name);
  return true;
}

// Whether _alias_mcts registered mcts::name.
bool mcts_aliased(const std::string& name) {
  const std::lock_guard<std::mutex> lock(g_alias_mutex);
  for (const std::string& n : g_aliased)
    if (n == name) return true;
  return false;
}

}  // namespace

TORCH_LIBRARY(omq, m) {
  for (const char* name : {"vectorized_backup", "warp_vectorized_backup", "fused_ucb_selection",
                           "batch_apply_virtual_loss", "batch_remove_virtual_loss"})
    define_op(m, name);
  m.def("_alias_mcts(str name) -> bool", &alias_mcts);
  m.def("_mcts_aliased(str name) -> bool", &mcts_aliased);
}
