// PyTorch operator registration for the MI355X alignment library.
//
// Registers fast_forced_aligner_cuda::align and ::emission_validity with the
// schemas of the reference (src/fast_forced_aligner/csrc/alignment.cu:1064-1070),
// so a Python layer written against the reference's operators works unchanged.
// This file only adapts tensors to the C ABI of include/ffa.h: it checks
// arguments, builds the descriptor table in pinned host memory, uploads it
// asynchronously, allocates outputs and scratch from PyTorch's caching
// allocator, and enqueues the HIP kernels on the current stream. It never
// synchronizes the host.
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPCachingAllocatorMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <climits>
#include <optional>
#include <tuple>
#include <vector>

#include "ffa.h"

namespace {

using c10::hip::HIPCachingAllocatorMasqueradingAsCUDA::recordStreamMasqueradingAsCUDA;
using c10::hip::HIPStreamMasqueradingAsCUDA;

void check_ffa(int rc) {
  TORCH_CHECK(rc == FFA_OK, "fast_forced_aligner: ", ffa_last_error());
}

// emission_validity (alignment.cu:893-917).
at::Tensor emission_validity(at::TensorList emissions) {
  const int64_t count = emissions.size();
  TORCH_CHECK(count > 0 && count <= FFA_MAX_BATCH, "provide 1..65535 emission tensors");
  TORCH_CHECK(emissions[0].is_cuda(), "CUDA emissions required");
  const auto device = emissions[0].device();
  c10::hip::HIPGuardMasqueradingAsCUDA guard(device);
  const HIPStreamMasqueradingAsCUDA stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(device.index());
  auto host = at::empty({count, 2}, at::TensorOptions().dtype(at::kLong).device(at::kCPU).pinned_memory(true));
  auto* descriptors = host.data_ptr<int64_t>();
  for (int64_t i = 0; i < count; ++i) {
    const auto& e = emissions[i];
    TORCH_CHECK(e.device() == device && e.scalar_type() == at::kFloat && e.dim() == 2 && e.is_contiguous() &&
                    e.size(0) > 0 && e.size(0) <= INT_MAX && e.size(1) > 0 && e.size(1) <= FFA_MAX_VOCAB,
                "emissions must be contiguous CUDA FP32 [T,V] on one device with supported dimensions");
    descriptors[2 * i] = reinterpret_cast<int64_t>(e.data_ptr<float>());
    descriptors[2 * i + 1] = e.numel();
    recordStreamMasqueradingAsCUDA(e.storage().data_ptr(), stream);
  }
  auto resident = host.to(device, /*non_blocking=*/true);
  auto result = at::empty({count}, emissions[0].options().dtype(at::kBool));
  check_ffa(ffa_emission_validity_launch(resident.data_ptr<int64_t>(), count,
                                         reinterpret_cast<uint8_t*>(result.data_ptr<bool>()), stream.stream()));
  return result;
}

// align (alignment.cu:919-1061).
std::tuple<std::vector<at::Tensor>, std::vector<int64_t>> align(
    at::TensorList emissions, at::TensorList targets, at::IntArrayRef blanks, int64_t chunk_frames, int64_t mode,
    int64_t threads, int64_t repair_rounds, int64_t optimization_pass, int64_t variant,
    int64_t repair_budget_frames, int64_t repair_threads, bool compact_alphabet, bool parallel_traceback,
    bool overlap_fallback, int64_t trace_min_frames, int64_t repair_min_frames, bool frontier_reuse,
    int64_t frontier_min_frames, const std::optional<at::Tensor>& emission_validity, bool check_inputs) {
  const int64_t count = emissions.size();
  TORCH_CHECK_VALUE(count > 0 && count <= FFA_MAX_BATCH && (int64_t)targets.size() == count,
                    "provide 1..65535 matching emissions and targets");
  TORCH_CHECK_VALUE((int64_t)blanks.size() == count, "provide one blank ID per record");
  TORCH_CHECK(emissions[0].is_cuda(), "CUDA emissions required");
  const auto device = emissions[0].device();
  c10::hip::HIPGuardMasqueradingAsCUDA guard(device);
  const HIPStreamMasqueradingAsCUDA stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(device.index());
  const uint8_t* mask = nullptr;
  if (emission_validity.has_value()) {
    const auto& m = *emission_validity;
    TORCH_CHECK_VALUE(m.device() == device && m.scalar_type() == at::kBool && m.dim() == 1 && m.numel() == count &&
                          m.is_contiguous(),
                      "emission_validity must be contiguous CUDA bool [batch] on the input device");
    recordStreamMasqueradingAsCUDA(m.storage().data_ptr(), stream);
    mask = reinterpret_cast<const uint8_t*>(m.data_ptr<bool>());
  }
  ffa_align_options o;
  ffa_default_options(mode != 0, &o);
  o.chunk_frames = chunk_frames;
  o.mode = mode;
  o.threads = threads;
  o.repair_rounds = repair_rounds;
  o.optimization_pass = optimization_pass;
  o.variant = variant;
  o.repair_budget_frames = repair_budget_frames;
  o.repair_threads = repair_threads;
  o.compact_alphabet = compact_alphabet;
  o.parallel_traceback = parallel_traceback;
  o.overlap_fallback = overlap_fallback;
  o.trace_min_frames = trace_min_frames;
  o.repair_min_frames = repair_min_frames;
  o.frontier_reuse = frontier_reuse;
  o.frontier_min_frames = frontier_min_frames;
  o.check_inputs = check_inputs;
  std::vector<ffa_record> records(count);
  std::vector<int64_t> sizes(count);
  for (int64_t i = 0; i < count; ++i) {
    const auto& e = emissions[i];
    const auto& t = targets[i];
    // the per-record metadata contract of alignment.py:243-251, raised as ValueError
    TORCH_CHECK_VALUE(e.is_cuda() && e.device() == device && t.device() == device && e.scalar_type() == at::kFloat &&
                          t.scalar_type() == at::kLong && e.dim() == 2 && t.dim() == 1 && e.is_contiguous() &&
                          t.is_contiguous(),
                      "inputs must be contiguous CUDA float32 [T,V] and int64 [U] on one device");
    TORCH_CHECK_VALUE(e.size(0) > 0 && e.size(0) <= INT_MAX && e.size(1) > 0 && e.size(1) <= FFA_MAX_VOCAB &&
                          2 * t.numel() + 1 <= FFA_MAX_STATES && blanks[i] >= 0 && blanks[i] < e.size(1),
                      "unsupported frame count, vocabulary, target length, or blank ID");
    records[i].emissions = e.data_ptr<float>();
    records[i].targets = t.numel() ? t.data_ptr<int64_t>() : nullptr;
    records[i].frames = e.size(0);
    records[i].vocab = e.size(1);
    records[i].tokens = t.numel();
    records[i].blank = blanks[i];
    sizes[i] = e.size(0);
    // the kernels read raw addresses: keep the sources alive for this stream (alignment.cu:977-980)
    recordStreamMasqueradingAsCUDA(e.storage().data_ptr(), stream);
    if (t.numel()) recordStreamMasqueradingAsCUDA(t.storage().data_ptr(), stream);
  }
  ffa_align_plan plan;
  check_ffa(ffa_align_plan_batch(records.data(), count, &o, &plan));
  auto host = at::empty({plan.table_bytes}, at::TensorOptions().dtype(at::kByte).device(at::kCPU).pinned_memory(true));
  check_ffa(ffa_align_describe(&plan, records.data(), host.data_ptr(), plan.table_bytes));
  auto table = host.to(device, /*non_blocking=*/true);
  const auto options = emissions[0].options();
  auto empty = [&](at::IntArrayRef shape, at::ScalarType type) { return at::empty(shape, options.dtype(type)); };
  auto labels = empty({plan.total_frames}, at::kLong);
  auto scores = empty({plan.total_frames}, at::kFloat);
  auto status = empty({count}, at::kInt);
  auto objective = empty({count}, at::kFloat);
  auto stitched = empty({count}, at::kInt);
  auto repair_passes = empty({count}, at::kInt);
  auto repaired_frames = empty({count}, at::kLong);
  auto shortcut_stats = empty({count, 3}, at::kLong);
  auto routing_stats = empty({count, 3}, at::kInt);
  auto reuse_stats = empty({plan.reuse_rows, 4}, at::kLong);
  auto workspace = empty({plan.workspace_bytes}, at::kByte);
  ffa_align_outputs out;
  out.labels = labels.data_ptr<int64_t>();
  out.scores = scores.data_ptr<float>();
  out.status = status.data_ptr<int32_t>();
  out.objective = objective.data_ptr<float>();
  out.stitched = stitched.data_ptr<int32_t>();
  out.repair_passes = repair_passes.data_ptr<int32_t>();
  out.repaired_frames = repaired_frames.data_ptr<int64_t>();
  out.shortcut_stats = shortcut_stats.data_ptr<int64_t>();
  out.routing_stats = routing_stats.data_ptr<int32_t>();
  out.reuse_stats = plan.reuse_rows ? reuse_stats.data_ptr<int64_t>() : nullptr;
  check_ffa(ffa_align_launch(&plan, &o, table.data_ptr(), mask, &out, workspace.data_ptr(), stream.stream()));
  return {{labels, scores, status, objective, stitched, repair_passes, repaired_frames, shortcut_stats,
           routing_stats, reuse_stats},
          std::move(sizes)};
}

}  // namespace

TORCH_LIBRARY(fast_forced_aligner_cuda, m) {
  m.def("emission_validity(Tensor[] emissions) -> Tensor");
  m.def("align(Tensor[] emissions, Tensor[] targets, int[] blanks, int chunk_frames, int mode, "
        "int threads, int repair_rounds, int optimization_pass, int variant, "
        "int repair_budget_frames, int repair_threads, bool compact_alphabet, bool parallel_traceback, "
        "bool overlap_fallback, int trace_min_frames, int repair_min_frames, bool frontier_reuse, "
        "int frontier_min_frames, Tensor? emission_validity=None, bool check_inputs=True) -> (Tensor[], int[])");
}

TORCH_LIBRARY_IMPL(fast_forced_aligner_cuda, CUDA, m) {
  m.impl("align", &align);
  m.impl("emission_validity", &emission_validity);
}
