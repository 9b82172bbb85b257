/*
 * fast-forced-aligner for MI355X (gfx950): C ABI of the alignment hot path.
 *
 * The reference exposes this path as two PyTorch operators registered in
 * src/fast_forced_aligner/csrc/alignment.cu:1064-1070:
 *   fast_forced_aligner_cuda::emission_validity(Tensor[] emissions) -> Tensor
 *   fast_forced_aligner_cuda::align(Tensor[] emissions, Tensor[] targets, int[] blanks,
 *       <knobs>, Tensor? emission_validity, bool check_inputs) -> (Tensor[], int[])
 * This header is the same boundary with plain pointers and sizes: no torch types.
 * The build's torch extension (csrc/ffa_torch.cpp) registers those two operators
 * with identical schemas on top of these entry points; any other host (ctypes,
 * cgo, a C++ server) can call them directly.
 *
 * Conventions
 *   - Every pointer named "device" is HIP device memory on the current device.
 *   - Work is enqueued on `stream`; no entry point synchronizes the host.
 *   - Inputs are borrowed and never written. The caller keeps them alive, and
 *     unmodified, until the stream reaches the enqueued work.
 *   - Return value: FFA_OK, or a negative FFA_E_* code; ffa_last_error() then
 *     returns a message (thread-local, valid until the next call on the thread).
 */
#ifndef FFA_H
#define FFA_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FFA_OK 0
#define FFA_E_INVALID (-1)   /* argument outside the supported range (reference: TORCH_CHECK) */
#define FFA_E_HIP (-2)       /* a HIP launch or copy failed */
#define FFA_E_SIZE (-3)      /* a caller-provided buffer is too small */

#define FFA_MAX_BATCH 65535      /* alignment.cu:979, alignment.py:237 */
#define FFA_MAX_VOCAB 8192       /* alignment.cu:970, alignment.py:249 */
#define FFA_MAX_STATES 20479     /* 2U+1; the reference stops at 4096 (alignment.cu:970) */
#define FFA_TABLE_ARG_RECORDS 64 /* batches up to this size pass their record table as a kernel argument */

/* One record of the ragged batch (alignment.cu:961-988 reads the same facts
 * from each tensor pair). */
typedef struct ffa_record {
  const float* emissions;  /* device, contiguous row-major [frames][vocab] fp32 */
  const int64_t* targets;  /* device, contiguous [tokens] int64; may be NULL when tokens == 0 */
  int64_t frames;          /* T, 1 .. INT32_MAX */
  int64_t vocab;           /* V, 1 .. FFA_MAX_VOCAB */
  int64_t tokens;          /* U, 2U+1 <= FFA_MAX_STATES */
  int64_t blank;           /* 0 .. V-1 */
} ffa_record;

/* The operator's scalar arguments, same names and meaning as the schema at
 * alignment.cu:1066-1068. The public API always passes the vector at
 * alignment.py:496-501; ffa_default_options() returns it. */
typedef struct ffa_align_options {
  int64_t chunk_frames;          /* H (128); 1..512 here */
  int64_t mode;                  /* 0 conventional, 1 chunks without greedy, 2 optimized */
  int64_t threads;               /* 128|256|512; geometry only, validated like alignment.cu:932 */
  int64_t repair_rounds;         /* 0..2 */
  int64_t optimization_pass;     /* 2|3; result-identical variants */
  int64_t variant;               /* 0..2; result-identical input addressing */
  int64_t repair_budget_frames;  /* >= 0 */
  int64_t repair_threads;        /* 0|128|256|512; geometry only */
  int64_t trace_min_frames;      /* > 0; traceback strategy only */
  int64_t repair_min_frames;     /* >= 0 */
  int64_t frontier_min_frames;   /* >= 0 */
  int32_t compact_alphabet;      /* result-identical */
  int32_t parallel_traceback;    /* result-identical */
  int32_t overlap_fallback;
  int32_t frontier_reuse;
  int32_t check_inputs;
  /* 0: emissions are log-probabilities (the reference's input). 1: emissions
   * are raw fp32 logits and the path aligns their row log-softmax, computed
   * inside the kernels exactly as ffa_log_softmax_launch materializes it (no
   * counterpart in the reference, whose callers run log_softmax first:
   * examples/transformers_ctc/align.py:55-56). */
  int32_t logits;
} ffa_align_options;

/* Sizes the caller allocates before ffa_align_launch. */
typedef struct ffa_align_plan {
  int64_t count;            /* B */
  int64_t total_frames;     /* N = sum of T: length of labels and scores */
  int64_t table_bytes;      /* descriptor table, written on the host by ffa_align_describe */
  int64_t table_uploaded;   /* 0: the table travels in the kernel arguments (B <= FFA_TABLE_ARG_RECORDS)
                               and may be reused as soon as ffa_align_launch returns; 1: ffa_align_launch
                               copies it into the workspace on the stream, so it must stay unchanged until
                               the stream reaches the work (pinned memory keeps the copy asynchronous) */
  int64_t workspace_bytes;  /* device scratch for one call (the table's device copy included) */
  int64_t reuse_rows;       /* rows of reuse_stats: B when frontier reuse is active, else 0 */
  int64_t internal[32];     /* launch geometry; read by ffa_align_launch only */
} ffa_align_plan;

/* Device output buffers: the ten tensors align() returns, in the order of
 * alignment.cu:1059 / alignment.py:138-148. */
typedef struct ffa_align_outputs {
  int64_t* labels;           /* [N] */
  float* scores;             /* [N] */
  int32_t* status;           /* [B] */
  float* objective;          /* [B] */
  int32_t* stitched;         /* [B] */
  int32_t* repair_passes;    /* [B] */
  int64_t* repaired_frames;  /* [B] */
  int64_t* shortcut_stats;   /* [B][3] */
  int32_t* routing_stats;    /* [B][3] */
  int64_t* reuse_stats;      /* [reuse_rows][4]; may be NULL when reuse_rows == 0 */
} ffa_align_outputs;

/* The knob vector of alignment.py:496-501 for mode "optimized" (nonzero) or
 * "conventional" (zero). */
void ffa_default_options(int optimized, ffa_align_options* options);

/* Validates the batch and options like alignment.cu:924-989 and computes the
 * buffer sizes. Host only; touches no device memory. */
int ffa_align_plan_batch(const ffa_record* records, int64_t count, const ffa_align_options* options,
                         ffa_align_plan* plan);

/* Writes the descriptor table into host memory (the per-record metadata that
 * alignment.cu:996-1005 writes into pinned memory and uploads). */
int ffa_align_describe(const ffa_align_plan* plan, const ffa_record* records,
                       void* host_table, int64_t host_table_bytes);

/* Enqueues the alignment: replaces the descriptor upload and the kernel
 * sequence of alignment.cu:1005-1053 (pack_inputs + launch_alignment).
 * host_table holds the bytes written by ffa_align_describe (see
 * plan->table_uploaded for how long it must live); emission_validity is an
 * optional device bool[B] mask (alignment.cu:946-952); workspace is device
 * memory of plan->workspace_bytes.
 * Optimized-mode batches of log-probabilities with at most 1,024 chunks, at
 * most 4,096 states and no record of 2,048+ frames run as one kernel launch
 * (the chunk kernel finishes each record itself); for them the library holds
 * 128 KiB of arrival counters per (device, stream) (one per 128-byte line for
 * up to 1,024 records), allocated and zeroed on the stream's first such call
 * and kept until the process ends.
 * A stream under graph capture that has none yet takes the two-launch form.
 * Batches of log-probabilities with a transcript of more than 1,024 states
 * (conventional mode, or optimized mode with a record of 2,048+ frames; more
 * than 4,096 states in optimized mode without repair rounds) run
 * the full DP in bands of 256 states, one workgroup each; the launch first
 * zeroes the bands' control words and edge arrays, which the plan places in
 * the workspace (no kernel of this entry writes memory it does not own). */
int ffa_align_launch(const ffa_align_plan* plan, const ffa_align_options* options,
                     const void* host_table, const uint8_t* emission_validity,
                     const ffa_align_outputs* outputs, void* workspace, hipStream_t stream);

/* Allocation-free variant of ffa_align_launch. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The workspace (with the table's device copy) lives in a device array of
 * FFA_NOALLOC_MAX_BYTES that the library holds on each GPU it runs on until the
 * process ends. The caller passes the host table, inputs and outputs as for
 * ffa_align_launch; `stream` must belong to the current device. Nothing is
 * allocated or freed. Returns FFA_E_SIZE when plan->workspace_bytes exceeds
 * FFA_NOALLOC_MAX_BYTES (32 MiB: about 14 MiB serves 64
 * records of 250..1,750 frames and ~500 tokens; four 30,000-frame records of
 * 9,000 tokens need 580 MiB and must use ffa_align_launch).
 * Every call on a GPU shares that GPU's array: calls enqueued on one stream
 * are ordered, but calls that overlap on one GPU (several streams or threads)
 * race and corrupt each other's results. Batches that ffa_align_launch runs
 * as one launch run so here too, with their arrival counters in a second
 * device array of 128 KiB per GPU (zero when the library loads, left at zero
 * by every call). */
#define FFA_NOALLOC_MAX_BYTES (32u << 20)
int ffa_align_launch_noalloc(const ffa_align_plan* plan, const ffa_align_options* options, const void* host_table,
                             const uint8_t* emission_validity, const ffa_align_outputs* outputs,
                             hipStream_t stream);

/* Replaces emission_validity (alignment.cu:893-917 and its kernel :879-891).
 * device_descriptors: [count][2] int64 {device address of a float array, element
 * count}, the reference's descriptor layout. valid: device bool[count]. */
int ffa_emission_validity_launch(const int64_t* device_descriptors, int64_t count, uint8_t* valid,
                                 hipStream_t stream);

/* Token spans (the reference README's "Converting frame labels to timestamps",
 * stated only in prose there; this entry has no native counterpart in the
 * reference): for each record, the equal-label runs of its aligned path with
 * blank runs removed, as [start, end) frame pairs. A successful record (status
 * 0) has exactly `tokens` runs, written in order to spans[span_offset .. +tokens)
 * as int64 {start, end}; multiply by the model's frame stride for timestamps.
 * Records with a nonzero status get {-1, -1}. device_records: [count] records in
 * device memory; labels / status: align()'s outputs; spans: int64
 * [sum of tokens][2] in device memory. */
typedef struct ffa_span_record {
  int64_t frame_offset;  /* first frame of the record in labels */
  int64_t frames;        /* T */
  int64_t span_offset;   /* first span of the record */
  int32_t tokens;        /* U: spans of a successful record */
  int32_t blank;
} ffa_span_record;

int ffa_token_spans_launch(const ffa_span_record* device_records, int64_t count, const int64_t* labels,
                           const int32_t* status, int64_t* spans, hipStream_t stream);

/* Row log-softmax of raw logits (the producer step before alignment,
 * examples/transformers_ctc/align.py:55-56: logits.float().log_softmax(-1);
 * this entry has no native counterpart in the reference). Per row, with
 * m = max(x) (+0.0 for a zero maximum) and ls = logf(sum of expf(x - m)):
 * out = (x - m) - ls. The sum's order is fixed (lane l of a 64-lane wave adds
 * the terms of columns l, l+64, ... in turn from +0.0; the 64 partial sums then
 * combine as s[l] += s[l + o] for o = 32, 16, ..., 1), so the values equal,
 * bit for bit, the ones ffa_align_launch uses when options->logits is set.
 * device_records: [count] records in device memory; max_frames: the largest
 * `frames` among them (sizes the grid). */
typedef struct ffa_logits_record {
  const float* logits;  /* device, contiguous [frames][vocab] fp32 */
  float* log_probs;     /* device, contiguous [frames][vocab] fp32; may not overlap logits */
  int64_t frames;       /* 1 .. INT32_MAX */
  int64_t vocab;        /* 1 .. FFA_MAX_VOCAB */
} ffa_logits_record;

int ffa_log_softmax_launch(const ffa_logits_record* device_records, int64_t count, int64_t max_frames,
                           hipStream_t stream);

/* Message for the last failing call on this thread. */
const char* ffa_last_error(void);

/* Measurement hook (no counterpart in the reference; for benchmarks and
 * profilers). Arms two caller-created HIP events for the next
 * ffa_align_launch on the calling thread: `start` is recorded on that launch's
 * stream immediately before its dominant kernel (the full-record DP in
 * conventional mode, the chunk kernel in optimized mode) and `stop` right
 * after it. Passing NULL events disarms. */
int ffa_profile_next_launch(hipEvent_t start, hipEvent_t stop);

/* Measurement hook (no counterpart in the reference). Launches a kernel that
 * does nothing with `workgroups` x `threads` (1..1024) on `stream`: timed like
 * the dominant kernel, it gives the fixed cost of one dispatch under that
 * timing method, the floor beneath every kernel's measured duration. */
int ffa_launch_floor(int32_t workgroups, int32_t threads, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* FFA_H */
