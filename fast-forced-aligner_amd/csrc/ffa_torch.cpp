// PyTorch adaptor for the MI355X alignment library.
//
// Registers fast_forced_aligner_cuda::align and ::emission_validity with the
// schemas of the reference (src/fast_forced_aligner/csrc/alignment.cu:1064-1070),
// so a Python layer written against the reference's operators works unchanged,
// and exposes the same alignment as a Python function (module _ffa_torch,
// function align) that the package's own align() calls: it reads the Python
// lists directly and skips the dispatcher's boxing of two tensor lists and
// twenty arguments.
//
// Both entry points share one implementation that only adapts tensors to the
// C ABI of include/ffa.h: it checks arguments, writes the descriptor table
// (passed in the kernel arguments, or uploaded from pinned host memory for
// batches of more than 64 records), allocates the scratch and the outputs from
// PyTorch's caching allocator (one block each), and enqueues the HIP kernels on
// the current stream. It never synchronizes the host.
#include <ATen/ATen.h>
#include <ATen/core/CachingHostAllocator.h>
#include <ATen/hip/impl/HIPCachingAllocatorMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <c10/core/InferenceMode.h>
#include <torch/csrc/autograd/python_variable.h>
#include <torch/library.h>
#include <pybind11/pybind11.h>

#include <algorithm>
#include <climits>
#include <optional>
#include <tuple>
#include <vector>

#include "ffa.h"

namespace py = pybind11;

namespace {

using c10::hip::HIPCachingAllocatorMasqueradingAsCUDA::recordStreamMasqueradingAsCUDA;
using c10::hip::HIPStreamMasqueradingAsCUDA;

void check_ffa(int rc) {
  TORCH_CHECK(rc == FFA_OK, "fast_forced_aligner: ", ffa_last_error());
}

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

// The workspace of a call on `stream`: kept per thread and stream between calls
// up to 64 MiB (the kernels of calls on one stream run in order, so the next
// call may reuse it; workspaces past the cap, and calls under graph capture,
// allocate per call). The cache is never destroyed: tensors must not be freed
// after the allocator at exit.
at::Tensor workspace_for(const at::TensorOptions& options, int64_t bytes, hipStream_t stream) {
  constexpr int64_t kCap = int64_t(64) << 20;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  // under graph capture the workspace comes from the graph's own pool, as before
  if (bytes > kCap || hipStreamIsCapturing(stream, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone)
    return at::empty({bytes}, options.dtype(at::kByte));
  struct Entry {
    c10::DeviceIndex device;
    hipStream_t stream;
    at::Tensor buffer;
  };
  static thread_local auto* cache = new std::vector<Entry>();
  const c10::DeviceIndex device = options.device().index();
  for (Entry& e : *cache)
    if (e.device == device && e.stream == stream) {
      if (e.buffer.numel() < bytes) e.buffer = at::empty({bytes}, options.dtype(at::kByte));
      return e.buffer;
    }
  cache->push_back({device, stream, at::empty({bytes}, options.dtype(at::kByte))});
  return cache->back().buffer;
}

// A tensor over bytes [offset, offset + numel*itemsize) of `block`: shares the
// block's storage (one allocation serves every output of a call).
at::Tensor view_of(const at::Tensor& block, int64_t offset, at::ScalarType type, c10::IntArrayRef sizes) {
  const auto meta = c10::scalarTypeToTypeMeta(type);
  auto t = at::detail::make_tensor<c10::TensorImpl>(c10::Storage(block.storage()), block.key_set(), meta);
  t.unsafeGetTensorImpl()->set_storage_offset(offset / (int64_t)meta.itemsize());
  t.unsafeGetTensorImpl()->set_sizes_contiguous(sizes);
  return t;
}

// The alignment of one batch (alignment.cu:919-1061). `emission(i)` /
// `target(i)` return the i-th input tensors, `blank(i)` its blank id.
// Metadata errors raise ValueError with the reference Python layer's messages
// (alignment.py:233-252); knob errors raise RuntimeError as the operator does.
template <class E, class Y, class L>
std::tuple<std::vector<at::Tensor>, std::vector<int64_t>> run_align(int64_t count, E emission, Y target, L blank,
                                                                    const ffa_align_options& o,
                                                                    const at::Tensor* validity) {
  TORCH_CHECK_VALUE(count > 0 && count <= FFA_MAX_BATCH, "provide 1..65535 matching emissions and targets");
  const at::Tensor& e0 = emission(0);
  TORCH_CHECK_VALUE(e0.is_cuda(), "inputs must be contiguous CUDA float32 [T,V] and int64 [U] on one device");
  const auto device = e0.device();
  c10::hip::HIPGuardMasqueradingAsCUDA guard(device);
  const HIPStreamMasqueradingAsCUDA stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(device.index());
  std::vector<ffa_record> records(count);
  std::vector<int64_t> sizes(count);
  const void* last_e = nullptr;
  const void* last_y = nullptr;
  for (int64_t i = 0; i < count; ++i) {
    const at::Tensor& e = emission(i);
    const at::Tensor& t = target(i);
    const int64_t b = blank(i);
    // the per-record metadata contract of alignment.py:243-251
    TORCH_CHECK_VALUE(e.is_cuda() && e.device() == device && t.device() == device && e.scalar_type() == at::kFloat &&
                          t.scalar_type() == at::kLong && e.dim() == 2 && t.dim() == 1 && e.is_contiguous() &&
                          t.is_contiguous(),
                      "inputs must be contiguous CUDA float32 [T,V] and int64 [U] on one device");
    TORCH_CHECK_VALUE(e.size(0) > 0 && e.size(0) <= INT_MAX && e.size(1) > 0 && e.size(1) <= FFA_MAX_VOCAB &&
                          2 * t.numel() + 1 <= FFA_MAX_STATES && b >= 0 && b < e.size(1),
                      "unsupported frame count, vocabulary, target length, or blank ID");
    records[i].emissions = static_cast<const float*>(e.data_ptr());
    records[i].targets = t.numel() ? static_cast<const int64_t*>(t.data_ptr()) : nullptr;
    records[i].frames = e.size(0);
    records[i].vocab = e.size(1);
    records[i].tokens = t.numel();
    records[i].blank = b;
    sizes[i] = e.size(0);
    // the kernels read raw addresses: keep the sources alive for this stream
    // (alignment.cu:977-980); consecutive views of one block are recorded once
    const void* es = e.storage().data_ptr().get();
    if (es != last_e) recordStreamMasqueradingAsCUDA(e.storage().data_ptr(), stream);
    last_e = es;
    if (t.numel()) {
      const void* ys = t.storage().data_ptr().get();
      if (ys != last_y) recordStreamMasqueradingAsCUDA(t.storage().data_ptr(), stream);
      last_y = ys;
    }
  }
  const uint8_t* mask = nullptr;  // checked after the records, as alignment.py:486-492 follows _metadata
  if (validity) {
    const at::Tensor& m = *validity;
    TORCH_CHECK_VALUE(m.device() == device && m.scalar_type() == at::kBool && m.dim() == 1 && m.numel() == count &&
                          m.is_contiguous(),
                      "emission_validity must be contiguous CUDA bool [batch] on the input device");
    recordStreamMasqueradingAsCUDA(m.storage().data_ptr(), stream);
    mask = reinterpret_cast<const uint8_t*>(m.data_ptr());
  }
  ffa_align_plan plan;
  check_ffa(ffa_align_plan_batch(records.data(), count, &o, &plan));
  // descriptor table: batches of at most FFA_TABLE_ARG_RECORDS records pass it
  // in the kernel arguments (a host buffer reused once the launch returns);
  // larger ones are uploaded by the launch from a pinned block, which must not
  // be reused before the copy ran
  thread_local std::vector<unsigned char> arg_table;
  c10::DataPtr host;
  void* table = nullptr;
  at::HostAllocator* host_alloc = nullptr;
  if (plan.table_uploaded) {
    host_alloc = at::getHostAllocator(at::kCUDA);
    host = host_alloc->allocate(plan.table_bytes);
    table = host.get();
  } else {
    arg_table.resize(plan.table_bytes);
    table = arg_table.data();
  }
  check_ffa(ffa_align_describe(&plan, records.data(), table, plan.table_bytes));
  const auto options = e0.options();
  auto scratch = workspace_for(options, plan.workspace_bytes, stream.stream());
  // outputs: one allocation, ten views (alignment.cu:1059 order)
  const int64_t N = plan.total_frames, B = count, R = plan.reuse_rows;
  int64_t off = 0;
  auto place = [&](int64_t bytes) { const int64_t at = off; off += align256(bytes); return at; };
  const int64_t o_labels = place(8 * N), o_scores = place(4 * N), o_status = place(4 * B), o_objective = place(4 * B),
                o_stitched = place(4 * B), o_passes = place(4 * B), o_repaired = place(8 * B),
                o_shortcut = place(24 * B), o_routing = place(12 * B), o_reuse = place(32 * R);
  auto block = at::empty({off}, options.dtype(at::kByte));
  auto labels = view_of(block, o_labels, at::kLong, {N});
  auto scores = view_of(block, o_scores, at::kFloat, {N});
  auto status = view_of(block, o_status, at::kInt, {B});
  auto objective = view_of(block, o_objective, at::kFloat, {B});
  auto stitched = view_of(block, o_stitched, at::kInt, {B});
  auto repair_passes = view_of(block, o_passes, at::kInt, {B});
  auto repaired_frames = view_of(block, o_repaired, at::kLong, {B});
  auto shortcut_stats = view_of(block, o_shortcut, at::kLong, {B, 3});
  auto routing_stats = view_of(block, o_routing, at::kInt, {B, 3});
  auto reuse_stats = view_of(block, o_reuse, at::kLong, {R, 4});
  auto* base = static_cast<uint8_t*>(block.data_ptr());
  ffa_align_outputs out;
  out.labels = reinterpret_cast<int64_t*>(base + o_labels);
  out.scores = reinterpret_cast<float*>(base + o_scores);
  out.status = reinterpret_cast<int32_t*>(base + o_status);
  out.objective = reinterpret_cast<float*>(base + o_objective);
  out.stitched = reinterpret_cast<int32_t*>(base + o_stitched);
  out.repair_passes = reinterpret_cast<int32_t*>(base + o_passes);
  out.repaired_frames = reinterpret_cast<int64_t*>(base + o_repaired);
  out.shortcut_stats = reinterpret_cast<int64_t*>(base + o_shortcut);
  out.routing_stats = reinterpret_cast<int32_t*>(base + o_routing);
  out.reuse_stats = R ? reinterpret_cast<int64_t*>(base + o_reuse) : nullptr;
  check_ffa(ffa_align_launch(&plan, &o, table, mask, &out, scratch.data_ptr(), stream.stream()));
  if (plan.table_uploaded) host_alloc->record_event(host.get(), host.get_context(), stream.unwrap());
  return {{labels, scores, status, objective, stitched, repair_passes, repaired_frames, shortcut_stats,
           routing_stats, reuse_stats},
          std::move(sizes)};
}

// The emission scan shared by the operator and the package's Python entry
// (replaces alignment.cu:893-917 and the Python checks of alignment.py:312-343):
// every record must be a contiguous fp32 [T, V] tensor on the first record's
// device with 0 < T <= INT_MAX and 0 < V <= 8192; their {address, numel}
// descriptors go into a caching-host-allocator block, one asynchronous upload
// on the current stream, one workgroup per record. `item(i)` returns the i-th
// tensor or nullptr when the i-th object is not a tensor; `reject(message)`
// raises the caller's exception type.
template <class Item, class Reject>
at::Tensor scan_emissions(int64_t count, Item item, Reject reject, const char* shape_message) {
  if (count <= 0 || count > FFA_MAX_BATCH) reject("provide 1..65535 emission tensors");
  const at::Tensor* first = item(0);
  if (!first || !first->is_cuda()) reject(shape_message);
  const auto device = first->device();
  c10::hip::HIPGuardMasqueradingAsCUDA guard(device);
  const HIPStreamMasqueradingAsCUDA stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(device.index());
  auto* host_alloc = at::getHostAllocator(at::kCUDA);
  const int64_t bytes = 16 * count;
  c10::DataPtr host = host_alloc->allocate(bytes);
  auto* descriptors = static_cast<int64_t*>(host.get());
  const void* last = nullptr;
  for (int64_t i = 0; i < count; ++i) {
    const at::Tensor* e = item(i);
    if (!e || !(e->is_cuda() && e->device() == device && e->scalar_type() == at::kFloat && e->dim() == 2 &&
                e->is_contiguous() && e->size(0) > 0 && e->size(0) <= INT_MAX && e->size(1) > 0 &&
                e->size(1) <= FFA_MAX_VOCAB))
      reject(shape_message);
    descriptors[2 * i] = reinterpret_cast<int64_t>(e->data_ptr());
    descriptors[2 * i + 1] = e->numel();
    const void* storage = e->storage().data_ptr().get();
    if (storage != last) recordStreamMasqueradingAsCUDA(e->storage().data_ptr(), stream);
    last = storage;
  }
  const auto options = first->options();
  auto table = at::empty({align256(bytes)}, options.dtype(at::kByte));
  const hipError_t copied = hipMemcpyAsync(table.data_ptr(), host.get(), bytes, hipMemcpyHostToDevice, stream.stream());
  TORCH_CHECK(copied == hipSuccess, "fast_forced_aligner: descriptor upload failed: ", hipGetErrorString(copied));
  host_alloc->record_event(host.get(), host.get_context(), stream.unwrap());
  auto result = at::empty({count}, options.dtype(at::kBool));
  check_ffa(ffa_emission_validity_launch(static_cast<const int64_t*>(table.data_ptr()), count,
                                         reinterpret_cast<uint8_t*>(result.data_ptr()), stream.stream()));
  return result;
}

// emission_validity operator (the reference schema of alignment.cu:1065):
// argument errors raise RuntimeError, as the reference operator's checks do.
at::Tensor emission_validity_op(at::TensorList emissions) {
  return scan_emissions(
      (int64_t)emissions.size(),
      [&](int64_t i) -> const at::Tensor* { return &emissions[i]; },
      [](const char* message) { TORCH_CHECK(false, message); },
      "emissions must be contiguous CUDA FP32 [T,V] on one device with supported dimensions");
}

// align operator (alignment.cu:919-1061): the reference schema and return order.
std::tuple<std::vector<at::Tensor>, std::vector<int64_t>> align_op(
    at::TensorList emissions, at::TensorList targets, at::IntArrayRef blanks, int64_t chunk_frames, int64_t mode,
    int64_t threads, int64_t repair_rounds, int64_t optimization_pass, int64_t variant,
    int64_t repair_budget_frames, int64_t repair_threads, bool compact_alphabet, bool parallel_traceback,
    bool overlap_fallback, int64_t trace_min_frames, int64_t repair_min_frames, bool frontier_reuse,
    int64_t frontier_min_frames, const std::optional<at::Tensor>& emission_validity, bool check_inputs) {
  const int64_t count = emissions.size();
  TORCH_CHECK_VALUE(count > 0 && count <= FFA_MAX_BATCH && (int64_t)targets.size() == count,
                    "provide 1..65535 matching emissions and targets");
  TORCH_CHECK_VALUE((int64_t)blanks.size() == count, "provide one blank ID per record");
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
  return run_align(
      count, [&](int64_t i) -> const at::Tensor& { return emissions[i]; },
      [&](int64_t i) -> const at::Tensor& { return targets[i]; }, [&](int64_t i) { return blanks[i]; }, o,
      emission_validity.has_value() ? &*emission_validity : nullptr);
}

// Python entry of the package's align(): emissions / targets are Python
// sequences of tensors, blank_id an int or a sequence of ints, and the knob
// vector is the public API's (alignment.py:496-501). Returns the ten output
// tensors and the record lengths. Outputs are inference tensors, as under the
// reference's @torch.inference_mode.
py::tuple align_py(py::handle emissions, py::handle targets, py::handle blank_id, bool optimized,
                   bool check_inputs, py::handle validity, bool logits) {
  c10::InferenceMode inference;
  py::object es_seq = py::reinterpret_steal<py::object>(PySequence_Fast(emissions.ptr(), "emissions"));
  py::object ys_seq = py::reinterpret_steal<py::object>(PySequence_Fast(targets.ptr(), "targets"));
  if (!es_seq || !ys_seq) throw py::error_already_set();
  const int64_t count = PySequence_Fast_GET_SIZE(es_seq.ptr());
  if (count <= 0 || count > FFA_MAX_BATCH || PySequence_Fast_GET_SIZE(ys_seq.ptr()) != count)
    throw py::value_error("provide 1..65535 matching emissions and targets");
  PyObject** es = PySequence_Fast_ITEMS(es_seq.ptr());
  PyObject** ys = PySequence_Fast_ITEMS(ys_seq.ptr());
  for (int64_t i = 0; i < count; ++i)
    if (!THPVariable_Check(es[i]) || !THPVariable_Check(ys[i]))
      throw py::value_error("inputs must be contiguous CUDA float32 [T,V] and int64 [U] on one device");
  int64_t single = 0;
  std::vector<int64_t> blanks;
  auto as_blank = [](PyObject* x, int64_t* value) {  // an int, not a bool (alignment.py:250)
    if (!PyLong_Check(x) || PyBool_Check(x)) return false;
    int overflow = 0;
    *value = PyLong_AsLongLongAndOverflow(x, &overflow);
    return overflow == 0 && !(*value == -1 && PyErr_Occurred());
  };
  const bool uniform = PyLong_Check(blank_id.ptr()) && !PyBool_Check(blank_id.ptr());
  if (uniform) {
    if (!as_blank(blank_id.ptr(), &single)) {
      PyErr_Clear();
      throw py::value_error("unsupported frame count, vocabulary, target length, or blank ID");
    }
  } else {
    py::object bs = py::reinterpret_steal<py::object>(PySequence_Fast(blank_id.ptr(), "blank_id"));
    if (!bs) throw py::error_already_set();
    if (PySequence_Fast_GET_SIZE(bs.ptr()) != count) throw py::value_error("provide one blank ID per record");
    blanks.resize(count);
    PyObject** items = PySequence_Fast_ITEMS(bs.ptr());
    for (int64_t i = 0; i < count; ++i)
      if (!as_blank(items[i], &blanks[i])) {
        PyErr_Clear();
        throw py::value_error("unsupported frame count, vocabulary, target length, or blank ID");
      }
  }
  const at::Tensor* mask = nullptr;
  if (!validity.is_none()) {
    if (!THPVariable_Check(validity.ptr()))
      throw py::value_error("emission_validity must be contiguous CUDA bool [batch] on the input device");
    mask = &THPVariable_Unpack(validity.ptr());
  }
  ffa_align_options o;
  ffa_default_options(optimized ? 1 : 0, &o);
  o.check_inputs = check_inputs;
  o.logits = logits ? 1 : 0;
  std::tuple<std::vector<at::Tensor>, std::vector<int64_t>> result;
  try {
    result = run_align(
        count, [&](int64_t i) -> const at::Tensor& { return THPVariable_Unpack(es[i]); },
        [&](int64_t i) -> const at::Tensor& { return THPVariable_Unpack(ys[i]); },
        [&](int64_t i) { return uniform ? single : blanks[i]; }, o, mask);
  } catch (const c10::ValueError& error) {
    throw py::value_error(error.what_without_backtrace());
  } catch (const c10::Error& error) {
    throw std::runtime_error(error.what_without_backtrace());
  }
  const auto& tensors = std::get<0>(result);
  const auto& lengths = std::get<1>(result);
  py::tuple outs(tensors.size());
  for (size_t i = 0; i < tensors.size(); ++i)
    outs[i] = py::reinterpret_steal<py::object>(THPVariable_Wrap(tensors[i]));
  py::tuple lens(lengths.size());
  for (size_t i = 0; i < lengths.size(); ++i) lens[i] = py::int_(lengths[i]);
  return py::make_tuple(outs, lens);
}

// Python entry of the package's emission_validity(): the operator's scan, with
// the Python layer's ValueError for malformed arguments (alignment.py:312-343).
py::object emission_validity_py(py::handle emissions) {
  c10::InferenceMode inference;
  py::object seq = py::reinterpret_steal<py::object>(PySequence_Fast(emissions.ptr(), "emissions"));
  if (!seq) throw py::error_already_set();
  PyObject** items = PySequence_Fast_ITEMS(seq.ptr());
  at::Tensor result = scan_emissions(
      (int64_t)PySequence_Fast_GET_SIZE(seq.ptr()),
      [&](int64_t i) -> const at::Tensor* {
        return THPVariable_Check(items[i]) ? &THPVariable_Unpack(items[i]) : nullptr;
      },
      [](const char* message) { throw py::value_error(message); },
      "emissions must be contiguous CUDA float32 [T,V] with supported dimensions on one device");
  return py::reinterpret_steal<py::object>(THPVariable_Wrap(result));
}

// Row log-softmax of raw logits (ffa_log_softmax_launch): the values the
// fused logits path of align() works on, materialized. `logits` is a sequence
// of contiguous CUDA float32 [T, V] tensors on one device; returns one tensor
// per record, views of one allocation, enqueued on the current stream.
py::list log_softmax_py(py::handle logits_obj) {
  c10::InferenceMode inference;
  py::object seq = py::reinterpret_steal<py::object>(PySequence_Fast(logits_obj.ptr(), "logits"));
  if (!seq) throw py::error_already_set();
  const int64_t count = PySequence_Fast_GET_SIZE(seq.ptr());
  if (count <= 0 || count > FFA_MAX_BATCH) throw py::value_error("provide 1..65535 logit tensors");
  PyObject** items = PySequence_Fast_ITEMS(seq.ptr());
  const char* bad = "logits must be contiguous CUDA float32 [T,V] with supported dimensions on one device";
  if (!THPVariable_Check(items[0]) || !THPVariable_Unpack(items[0]).is_cuda()) throw py::value_error(bad);
  const auto device = THPVariable_Unpack(items[0]).device();
  c10::hip::HIPGuardMasqueradingAsCUDA guard(device);
  const HIPStreamMasqueradingAsCUDA stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(device.index());
  std::vector<int64_t> offsets(count);
  int64_t total = 0, max_frames = 0;
  for (int64_t i = 0; i < count; ++i) {
    if (!THPVariable_Check(items[i])) throw py::value_error(bad);
    const at::Tensor& x = THPVariable_Unpack(items[i]);
    if (!(x.is_cuda() && x.device() == device && x.scalar_type() == at::kFloat && x.dim() == 2 && x.is_contiguous() &&
          x.size(0) > 0 && x.size(0) <= INT_MAX && x.size(1) > 0 && x.size(1) <= FFA_MAX_VOCAB))
      throw py::value_error(bad);
    offsets[i] = total;
    total += align256(4 * x.numel());
    max_frames = std::max<int64_t>(max_frames, x.size(0));
  }
  const auto options = THPVariable_Unpack(items[0]).options();
  auto block = at::empty({total}, options.dtype(at::kByte));
  auto* base = static_cast<uint8_t*>(block.data_ptr());
  auto* host_alloc = at::getHostAllocator(at::kCUDA);
  const int64_t table_bytes = count * (int64_t)sizeof(ffa_logits_record);
  c10::DataPtr host = host_alloc->allocate(table_bytes);
  auto* recs = static_cast<ffa_logits_record*>(host.get());
  py::list outs(count);
  for (int64_t i = 0; i < count; ++i) {
    const at::Tensor& x = THPVariable_Unpack(items[i]);
    recs[i] = ffa_logits_record{static_cast<const float*>(x.data_ptr()), reinterpret_cast<float*>(base + offsets[i]),
                                x.size(0), x.size(1)};
    recordStreamMasqueradingAsCUDA(x.storage().data_ptr(), stream);
    outs[i] = py::reinterpret_steal<py::object>(
        THPVariable_Wrap(view_of(block, offsets[i], at::kFloat, {x.size(0), x.size(1)})));
  }
  auto table = at::empty({align256(table_bytes)}, options.dtype(at::kByte));
  const hipError_t copied = hipMemcpyAsync(table.data_ptr(), host.get(), table_bytes, hipMemcpyHostToDevice,
                                           stream.stream());
  TORCH_CHECK(copied == hipSuccess, "fast_forced_aligner: record table upload failed: ", hipGetErrorString(copied));
  host_alloc->record_event(host.get(), host.get_context(), stream.unwrap());
  check_ffa(ffa_log_softmax_launch(static_cast<const ffa_logits_record*>(table.data_ptr()), count, max_frames,
                                   stream.stream()));
  return outs;
}

// Token spans of an alignment's paths (ffa_token_spans_launch): labels and
// status are align()'s outputs, lengths the frames and tokens the target
// length of each record, blank_id an int or one int per record. Returns int64
// [sum(tokens), 2] on the labels' device, enqueued on the current stream.
py::object token_spans_py(py::handle labels_obj, py::handle status_obj, py::handle lengths_obj,
                          py::handle tokens_obj, py::handle blank_id) {
  c10::InferenceMode inference;
  if (!THPVariable_Check(labels_obj.ptr()) || !THPVariable_Check(status_obj.ptr()))
    throw py::value_error("labels and status must be tensors from align()");
  const at::Tensor& labels = THPVariable_Unpack(labels_obj.ptr());
  const at::Tensor& status = THPVariable_Unpack(status_obj.ptr());
  py::object ls = py::reinterpret_steal<py::object>(PySequence_Fast(lengths_obj.ptr(), "lengths"));
  py::object ts = py::reinterpret_steal<py::object>(PySequence_Fast(tokens_obj.ptr(), "tokens"));
  if (!ls || !ts) throw py::error_already_set();
  const int64_t count = PySequence_Fast_GET_SIZE(ls.ptr());
  if (count <= 0 || count > FFA_MAX_BATCH || PySequence_Fast_GET_SIZE(ts.ptr()) != count)
    throw py::value_error("provide one frame count and one target length per record");
  if (!labels.is_cuda() || labels.scalar_type() != at::kLong || labels.dim() != 1 || !labels.is_contiguous() ||
      status.device() != labels.device() || status.scalar_type() != at::kInt || status.dim() != 1 ||
      status.numel() != count || !status.is_contiguous())
    throw py::value_error("labels must be contiguous CUDA int64 [N] and status CUDA int32 [batch] from align()");
  const bool uniform = PyLong_Check(blank_id.ptr()) && !PyBool_Check(blank_id.ptr());
  py::object bs;
  if (!uniform) {
    bs = py::reinterpret_steal<py::object>(PySequence_Fast(blank_id.ptr(), "blank_id"));
    if (!bs) throw py::error_already_set();
    if (PySequence_Fast_GET_SIZE(bs.ptr()) != count) throw py::value_error("provide one blank ID per record");
  }
  const auto device = labels.device();
  c10::hip::HIPGuardMasqueradingAsCUDA guard(device);
  const HIPStreamMasqueradingAsCUDA stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(device.index());
  auto* host_alloc = at::getHostAllocator(at::kCUDA);
  const int64_t table_bytes = count * (int64_t)sizeof(ffa_span_record);
  c10::DataPtr host = host_alloc->allocate(table_bytes);
  auto* recs = static_cast<ffa_span_record*>(host.get());
  int64_t frame = 0, span = 0;
  for (int64_t i = 0; i < count; ++i) {
    const int64_t T = py::cast<int64_t>(PySequence_Fast_GET_ITEM(ls.ptr(), i));
    const int64_t U = py::cast<int64_t>(PySequence_Fast_GET_ITEM(ts.ptr(), i));
    const int64_t b = uniform ? py::cast<int64_t>(blank_id) : py::cast<int64_t>(PySequence_Fast_GET_ITEM(bs.ptr(), i));
    if (T <= 0 || U < 0 || 2 * U + 1 > FFA_MAX_STATES || b < 0 || b >= FFA_MAX_VOCAB)
      throw py::value_error("unsupported frame count, target length, or blank ID");
    recs[i] = ffa_span_record{frame, T, span, (int32_t)U, (int32_t)b};
    frame += T;
    span += U;
  }
  if (frame != labels.numel()) throw py::value_error("frame counts do not add up to the labels' length");
  recordStreamMasqueradingAsCUDA(labels.storage().data_ptr(), stream);
  recordStreamMasqueradingAsCUDA(status.storage().data_ptr(), stream);
  auto table = at::empty({align256(table_bytes)}, labels.options().dtype(at::kByte));
  const hipError_t copied = hipMemcpyAsync(table.data_ptr(), host.get(), table_bytes, hipMemcpyHostToDevice,
                                           stream.stream());
  TORCH_CHECK(copied == hipSuccess, "fast_forced_aligner: span table upload failed: ", hipGetErrorString(copied));
  host_alloc->record_event(host.get(), host.get_context(), stream.unwrap());
  auto spans = at::empty({span, 2}, labels.options());
  if (span > 0)
    check_ffa(ffa_token_spans_launch(static_cast<const ffa_span_record*>(table.data_ptr()), count,
                                     static_cast<const int64_t*>(labels.data_ptr()),
                                     static_cast<const int32_t*>(status.data_ptr()),
                                     static_cast<int64_t*>(spans.data_ptr()), stream.stream()));
  return py::reinterpret_steal<py::object>(THPVariable_Wrap(spans));
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
  m.impl("align", &align_op);
  m.impl("emission_validity", &emission_validity_op);
}

PYBIND11_MODULE(_ffa_torch, m) {
  m.doc() = "MI355X CTC forced alignment: the package's direct entry to the HIP library";
  m.def("align", &align_py, py::arg("emissions"), py::arg("targets"), py::arg("blank_id"), py::arg("optimized"),
        py::arg("check_inputs"), py::arg("emission_validity"), py::arg("logits") = false);
  m.def("log_softmax", &log_softmax_py, py::arg("logits"));
  m.def("emission_validity", &emission_validity_py, py::arg("emissions"));
  m.def("token_spans", &token_spans_py, py::arg("labels"), py::arg("status"), py::arg("lengths"),
        py::arg("tokens"), py::arg("blank_id"));
}
