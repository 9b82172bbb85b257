// CTC forced-alignment kernels for MI355X (gfx950) and the C ABI of include/ffa.h.
//
// One HIP source, no other backend. Reference behaviour is cited as
// "cu:<line>" (src/fast_forced_aligner/csrc/alignment.cu) and "py:<line>"
// (src/fast_forced_aligner/alignment.py).
//
// Work decomposition
//   conventional mode: one launch, one workgroup per record. The workgroup
//     validates the targets, runs the Viterbi recurrence over all T frames with
//     2-bit backpointers in HBM, picks the terminal, walks the path back and
//     writes labels and scores (cu:919-1061 sequence pack -> recurrence -> finish).
//   optimized mode: two launches.
//     chunk_kernel: one workgroup per 128-frame chunk. It stages and validates
//       the record's targets, then takes the greedy shortcut (cu:30-153) or
//       runs the relaxed chunk DP (cu:355-523), writing the chunk's labels and
//       scores directly plus a slot with its endpoints and objective.
//     tail_kernel: one workgroup per record: repair planning (cu:164-228),
//       repair DP, seam validation (cu:562-592), full-DP fallback with its
//       path, and all per-record outputs.
//
// DP layout: a workgroup of NT = 64*W threads owns the 2L+1 states of one
// record, K contiguous states per thread (state s = tid*K + k). The s-1 / s-2
// neighbours of a thread's first two states come from the previous lane via
// DPP wave_shr:1, and across waves through a double-buffered LDS slot with one
// barrier per frame. Emission gathers e[t][l[s]] are issued D frames ahead into
// registers. Backpointers are 2 bits per state, 16 states per 32-bit word,
// rows of 2*ceil(S/32) words.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "ffa.h"

namespace ffa {

constexpr float NEG_INF = -INFINITY;
// 16 bytes of -inf: the chunk kernel's loads of row quads past V read them
__device__ __align__(16) const float kNegInfQuad[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
constexpr int MAX_H = 512;          // chunk_frames supported by the LDS layout
constexpr int TAIL_SLOT_CAP = 512;  // record tails with more chunks plan in global memory
constexpr int YTOK_PAD = 72;        // sentinel entries after the staged targets
constexpr int EBLK_COLS = 64;       // widest row (V) staged in LDS blocks by the DP

// Record descriptor, 64 bytes. The first 32 bytes hold what a chunk
// workgroup needs to find its record and to request its rows and targets.
struct RecordDesc {
  const float* emissions;
  const int64_t* targets;
  int32_t frames;           // T <= INT32_MAX
  int32_t chunk_offset;     // first chunk of the record in the batch's chunk order
  int32_t vocab, tokens;
  int64_t frame_offset;     // into labels / scores
  int64_t bp_offset;        // 32-bit words into the backpointer scratch
  int64_t frontier_offset;  // floats into the frontier scratch; -1 when unused
  int32_t blank;
  int32_t flags;            // DESC_REUSE_COUNTED
};
static_assert(sizeof(RecordDesc) == 64, "descriptor layout");
// The record is one the reference would run with frontier reuse (T >=
// frontier_min_frames in a batch that enables it, alignment.cu:374): its
// reuse_stats row counts frontier writes and resumed frames. Records without
// the flag still save and resume frontiers when storage exists; results are
// the same either way.
constexpr int32_t DESC_REUSE_COUNTED = 1;

// The record table passed by value as a kernel argument (batches of at most
// FFA_TABLE_ARG_RECORDS records): the runtime copies it with the launch, so
// no upload, no copy kernel and no host synchronization object is needed, and
// a chunk workgroup finds its record in one round of loads. Larger batches
// upload the table into the workspace instead (NoTable kernels).
constexpr int ARG_RECORDS = FFA_TABLE_ARG_RECORDS;
struct alignas(16) ArgTable {
  RecordDesc rec[ARG_RECORDS];
};
struct NoTable {
  int32_t unused;
};
template <class TB>
constexpr bool kArgs = sizeof(TB) == sizeof(ArgTable);

struct Slot {  // per-chunk state of optimized mode (cu:1021-1029 buffers), 32 bytes
  int32_t a, b, start, end, frontier_end;
  float objective;
  int16_t flag;    // merged-interval flag of the repair rounds
  int16_t kind;    // 0 chunk DP, 1 greedy shortcut, 2 chunk DP after an ambiguous placement
  int16_t status;  // record status seen by the chunk (>= 2: rejected)
  int16_t skip_ok; // l[start] != blank && l[start] != l[start-2]: a +2 seam into start is legal
};
static_assert(sizeof(Slot) == 32, "slot layout");

// Per-chunk table entry of optimized mode, 16 bytes so that a whole batch's
// table usually stays small enough for the runtime's in-queue copy. It holds
// what the target loads need, so they are issued together with the record
// descriptor's load instead of after it:
//   lo bits 0-44 the targets' address / 8 (48-bit GPU addresses), 45-58 U,
//      59 the greedy fast path (V <= 32, V % 4 == 0, 16-byte aligned rows, at
//      most 128 frames, greedy shortcuts on), 60-62 V/4 - 1 (fast path)
//   hi bits 0-15 record, 16-24 frames in the chunk - 1, 25-55 chunk index.
struct ChunkEntry {
  uint64_t lo, hi;
};
static_assert(sizeof(ChunkEntry) == 16, "chunk entry layout");
constexpr int ENTRY_U_SHIFT = 45, ENTRY_FAST_SHIFT = 59, ENTRY_QUADS_SHIFT = 60;


struct Params {
  const RecordDesc* desc;
  const ChunkEntry* chunks;
  const uint8_t* validity;
  int64_t* labels;
  float* scores;
  int32_t* status;
  float* objective;
  int32_t* stitched;
  int32_t* repair_passes;
  int64_t* repaired_frames;
  int64_t* shortcut_stats;
  int32_t* routing_stats;
  int64_t* reuse_stats;
  uint32_t* bp;
  Slot* slots;
  float* frontiers;
  int64_t budget, repair_min, frontier_min;
  int32_t count, total_slots, H, mode, repair_rounds, check_inputs, overlap;
  int32_t tail_phase;  // TAIL_ALL, or a phase of the split tail (TAIL_PLAN0, TAIL_RESUME)
  int32_t u_cap, d_cap, v_words, lds_tail_slots;
  int32_t eblk_frames;  // frames per LDS emission block of the DP (0: rows read straight from HBM)
  int32_t logits;       // emissions are raw logits, aligned as their row log-softmax
  float2* stats;        // logits: per frame {row max, log of the row's exp-sum}, indexed like labels
  struct TailState* tstate;  // split tail: per-record state between its phases
  int32_t* arrivals;         // fused tail: per-record count of finished chunks, zero between calls
  int32_t* band_ctl;         // banded DP: ticket, late flag, per-record arrivals, terminal values (zeroed per call)
  uint64_t* edges;           // banded DP: per record and band boundary, one tagged value per frame
  int32_t band_stride;       // banded DP: edge arrays per frame of the batch (bands of the widest record - 1)
};
// Fused tail: at most this many chunks (so records) per batch, and one arrival
// counter per 128-byte line (the records' counters are hit by every chunk
// workgroup at nearly the same time; on shared lines the atomics queue).
constexpr int FUSED_MAX_CHUNKS = 1024;
constexpr int ARRIVAL_STRIDE = 32;

// ---------------------------------------------------------------------------
// Shared-memory layout. A fixed header followed by dynamic regions whose sizes
// come from the launch (all offsets are uniform).
// Per-record diagnostics of the tail kernel, kept in LDS by thread 0 so that
// they hold no registers across the tail's DP calls.
struct TailStats {
  int64_t sc_accepted, sc_frames, sc_ambiguous;  // shortcut_stats
  int64_t reuse[4];                              // reuse_stats
  int64_t repaired;                              // repaired_frames
  int early, rejected, maxprop, passes;          // routing_stats, repair_passes
};

// The record's tail state in global memory for the split tail (batches with
// records of at least 2,048 frames): the tail kernel plans the first repair
// round (TAIL_PLAN0), repair_kernel runs that round's DPs with one workgroup
// per merged interval (alignment.cu:727-760 gives each interval its own CTA
// the same way) or the early full fallback, and the record's last workgroup
// to finish runs the later rounds and the seam check (TAIL_RESUME).
struct TailState {
  TailStats ts;
  int32_t done;     // the record's outputs are written (rejected, or stitched on the fast path)
  int32_t status;   // after an early full fallback
  float objective;  // after an early full fallback
  int32_t work;     // first-round DPs planned for the record (repair intervals or the early fallback)
  int32_t pending;  // of those, not finished yet
  int32_t fallback;       // the seams failed: band_kernel runs the full fallback and writes the outputs
  int32_t fallback_from;  // chunk 0's frontier end for that fallback (0: none)
  int32_t pad;
};
static_assert(sizeof(TailState) % 16 == 0, "16-byte granules");

enum { TAIL_ALL = 0, TAIL_PLAN0 = 1, TAIL_RESUME = 2 };

struct StageWave {  // one wave's target staging summary (chunk kernel)
  int flags;      // 1 out-of-vocabulary id, 2 blank id among the targets
  int repeats;    // adjacent repeats
  uint32_t mask;  // alphabet mask (V <= 32)
  int pad;
};

struct Header {
  float xchg[2][16][2];  // DP neighbour values crossing wave boundaries
  float red_v[16];
  int red_i[16];
  int red_j[16];
  uint32_t red_m[16];
  float term_v[2];
  int ibuf[8];
  float fbuf[4];
  union {
    struct {
      int stg_f[16];       // per-wave staging flags: 1 out-of-vocabulary id, 2 blank id among the targets
      int stg_r[16];       // per-wave adjacent-repeat counts
      uint32_t stg_m[16];  // per-wave alphabet masks (V <= 32)
    };
    StageWave stg[12];     // the same per wave as one record (chunk kernel; 12 >= 10 waves + 2 read ahead)
  };
  int gbad[2];         // per-wave greedy rejection (fast path)
  int last;            // the record's outputs are written (tail fast path)
  int arrived;         // fused tail: this workgroup is the record's last chunk to finish
  TailStats ts;
};

struct Lds {
  Header* h;
  int16_t* ytok;   // targets as int16 (V <= 8192)
  uint16_t* key3;  // per target position j: key of y[j], y[j+1], y[j+2] (placement prefilter)
  float* eblk;     // DP emission blocks: 2 halves of eblk_frames rows of up to EBLK_COLS values
  int eblk_frames;
  // greedy region (aliased by the tail's slot copy)
  int32_t* g;
  float* fs;
  int32_t* r;
  int32_t* pd;
  int32_t* pc;
  int16_t* sym;
  uint32_t* bitmap;
  uint32_t* wpref;
  float2* st;      // logits: row statistics of the chunk's frames (chunk kernel)
  int32_t* cand;
  int32_t* candok;
  Slot* tslots;
};

__device__ inline size_t align16(size_t x) { return (x + 15) & ~size_t(15); }

// Entries of the per-frame greedy arrays: H rounded up to 32, at least 128
// (the fast path indexes them by lane across two waves).
__host__ __device__ inline int64_t greedy_frames(int64_t H) { return H < 128 ? 128 : (H + 31) & ~int64_t(31); }

// The sizes that fix the LDS layout (a subset of Params).
struct LdsShape {
  int32_t u_cap, eblk_frames, H, d_cap, v_words;
};

__device__ inline Lds carve(unsigned char* base, const Params& p);

__device__ inline LdsShape lds_shape(const Params& p) {
  return LdsShape{p.u_cap, p.eblk_frames, p.H, p.d_cap, p.v_words};
}

__device__ inline Lds carve(unsigned char* base, const LdsShape& p) {
  Lds L;
  size_t off = 0;
  L.h = reinterpret_cast<Header*>(base);
  off = align16(sizeof(Header));
  L.ytok = reinterpret_cast<int16_t*>(base + off);
  off = align16(off + 2 * ((size_t)p.u_cap + YTOK_PAD));
  L.key3 = reinterpret_cast<uint16_t*>(base + off);
  off = align16(off + 2 * ((size_t)p.u_cap + YTOK_PAD));
  L.eblk = p.eblk_frames ? reinterpret_cast<float*>(base + off) : nullptr;
  L.eblk_frames = p.eblk_frames;
  off += (size_t)8 * p.eblk_frames * EBLK_COLS;
  unsigned char* region = base + off;
  size_t g = 0;
  const size_t h32 = (size_t)greedy_frames(p.H);
  L.g = reinterpret_cast<int32_t*>(region + g); g += 4 * h32;
  L.fs = reinterpret_cast<float*>(region + g); g += 4 * h32;
  L.r = reinterpret_cast<int32_t*>(region + g); g += 4 * h32;
  L.pd = reinterpret_cast<int32_t*>(region + g); g += 4 * h32;
  L.pc = reinterpret_cast<int32_t*>(region + g); g += 4 * h32;
  L.cand = reinterpret_cast<int32_t*>(region + g); g += 4 * 256;
  L.candok = reinterpret_cast<int32_t*>(region + g); g += 4 * 256;
  L.sym = reinterpret_cast<int16_t*>(region + g); g = align16(g + 2 * (size_t)p.d_cap);
  L.bitmap = reinterpret_cast<uint32_t*>(region + g); g += 4 * (size_t)p.v_words;
  L.wpref = reinterpret_cast<uint32_t*>(region + g);
  g = align16(g + 4 * (size_t)p.v_words);
  L.st = reinterpret_cast<float2*>(region + g);
  L.tslots = reinterpret_cast<Slot*>(region);
  return L;
}

__device__ inline Lds carve(unsigned char* base, const Params& p) { return carve(base, lds_shape(p)); }

// Pointers read from the descriptor table or the parameter block are generic
// to the compiler, which would emit flat accesses; flat loads also count
// against lgkmcnt, so every LDS wait would stall on outstanding HBM reads.
// Device code therefore accesses global memory through address space 1.
#define GLB __attribute__((address_space(1)))
template <class T>
__device__ inline GLB T* glb(T* x) { return (GLB T*)x; }
template <class T>
__device__ inline const GLB T* glb(const T* x) { return (const GLB T*)x; }
__device__ inline float ldg_at(const GLB float* base, uint32_t byte_offset) {
  return *(const GLB float*)((const GLB char*)base + byte_offset);
}
typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef float v4f_t __attribute__((ext_vector_type(4)));
// Whole-struct copies to and from global memory (16-byte vector moves).
template <class T>
__device__ inline T load_pod(const GLB T* src) {
  static_assert(sizeof(T) % 16 == 0, "16-byte granules");
  v4i_t tmp[sizeof(T) / 16];
#pragma unroll
  for (size_t i = 0; i < sizeof(T) / 16; ++i) tmp[i] = ((const GLB v4i_t*)src)[i];
  T out;
  __builtin_memcpy(&out, tmp, sizeof(T));
  return out;
}
template <class T>
__device__ inline void store_pod(GLB T* dst, const T& value) {
  static_assert(sizeof(T) % 16 == 0, "16-byte granules");
  v4i_t tmp[sizeof(T) / 16];
  __builtin_memcpy(tmp, &value, sizeof(T));
#pragma unroll
  for (size_t i = 0; i < sizeof(T) / 16; ++i) ((GLB v4i_t*)dst)[i] = tmp[i];
}
// Agent-scope (relaxed atomic) stores and loads: the store is written through
// this XCD's L2, the load is served past it, so workgroups on other XCDs of the
// same kernel see the value without an L2 write-back or invalidation. With AG
// false they are ordinary accesses.
template <bool AG, class T>
__device__ inline void put(GLB T* dst, T value) {
  if constexpr (AG) __hip_atomic_store((T*)dst, value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else *dst = value;
}
template <class T>
__device__ inline void store_pod_agent(GLB T* dst, const T& value) {
  static_assert(sizeof(T) % 8 == 0, "8-byte words");
  uint64_t tmp[sizeof(T) / 8];
  __builtin_memcpy(tmp, &value, sizeof(T));
#pragma unroll
  for (size_t i = 0; i < sizeof(T) / 8; ++i)
    __hip_atomic_store((uint64_t*)dst + i, tmp[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ inline T load_pod_agent(const GLB T* src) {
  static_assert(sizeof(T) % 8 == 0, "8-byte words");
  uint64_t tmp[sizeof(T) / 8];
#pragma unroll
  for (size_t i = 0; i < sizeof(T) / 8; ++i)
    tmp[i] = __hip_atomic_load((const uint64_t*)src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  T out;
  __builtin_memcpy(&out, tmp, sizeof(T));
  return out;
}
// Waits until every earlier global store of this wave is complete (for
// agent-scope stores: visible to the whole GPU).
__device__ inline void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }


// ---------------------------------------------------------------------------
// Wave64 helpers.
__device__ inline float wave_shr1(float x, float fill) {
  // DPP wave_shr:1 - lane i receives lane i-1; lane 0 keeps `fill`.
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      __builtin_bit_cast(int, fill), __builtin_bit_cast(int, x), 0x138, 0xf, 0xf, false));
}

template <int CTRL, int ROW_MASK>
__device__ inline int dpp_add(int v) {
  return v + __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, false);
}

// Wave64 inclusive scan: row_shr 1/2/4/8 inside rows of 16 lanes, then
// row_bcast:15 and row_bcast:31 carry row totals forward (six DPP adds).
__device__ inline int wave_scan_dpp(int x) {
  x = dpp_add<0x111, 0xf>(x);
  x = dpp_add<0x112, 0xf>(x);
  x = dpp_add<0x114, 0xf>(x);
  x = dpp_add<0x118, 0xf>(x);
  x = dpp_add<0x142, 0xa>(x);
  x = dpp_add<0x143, 0xc>(x);
  return x;
}

__device__ inline int wave_shr1_int(int x, int fill) {
  return __builtin_amdgcn_update_dpp(fill, x, 0x138, 0xf, 0xf, false);
}

__device__ inline float readlane_f(float x, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}

__device__ inline uint32_t lanes_below(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Sequential fp32 sum ((x0 + x1) + x2) + ... of 128 LDS values by one thread:
// 16-byte reads issued ahead of the dependent chain of adds.
__device__ __attribute__((always_inline)) inline float serial_sum128(const float* x) {
  const v4f_t* x4 = reinterpret_cast<const v4f_t*>(x);
  float acc = 0.0f;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    v4f_t v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = x4[16 * half + i];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc = (half == 0 && i == 0) ? v[i].x : acc + v[i].x;
      acc += v[i].y;
      acc += v[i].z;
      acc += v[i].w;
    }
  }
  return acc;
}

// Sequential fp32 sum ((x0 + x1) + x2) + ... of an LDS array by one thread,
// reading 32 values ahead of the dependent adds. x must hold a multiple of 32.
__device__ __attribute__((always_inline)) inline float serial_sum(const float* x, int n) {
  float acc = x[0];
  for (int base = 0; base < n; base += 32) {
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = x[base + i];
#pragma unroll
    for (int i = 0; i < 32; ++i)
      if (base + i >= 1 && base + i < n) acc += v[i];
  }
  return acc;
}

// argmax with the reference's comparator (value desc, state asc; NaN never wins),
// cu:472-491.
__device__ inline void better(float& bv, int& bi, float ov, int oi) {
  if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}

__device__ inline void wave_argmax(float& bv, int& bi) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    better(bv, bi, ov, oi);
  }
}

__device__ inline int wave_incl_scan(int x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  return x;
}

// Block-wide inclusive scan of one int per thread (values beyond n are 0).
__device__ inline int block_incl_scan(int x, Header* h) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int v = wave_incl_scan(x);
  __syncthreads();
  if (lane == 63) h->red_i[wave] = v;
  __syncthreads();
  int carry = 0;
  for (int w = 0; w < wave; ++w) carry += h->red_i[w];
  (void)nw;
  __syncthreads();
  return v + carry;
}

__device__ inline int block_sum(int x, Header* h) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  __syncthreads();
  if (lane == 0) h->red_i[wave] = x;
  __syncthreads();
  int total = 0;
  for (int w = 0; w < nw; ++w) total += h->red_i[w];
  __syncthreads();
  return total;
}

__device__ inline int block_min(int x, Header* h) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = min(x, __shfl_xor(x, off, 64));
  __syncthreads();
  if (lane == 0) h->red_i[wave] = x;
  __syncthreads();
  int m = INT_MAX;
  for (int w = 0; w < nw; ++w) m = min(m, h->red_i[w]);
  __syncthreads();
  return m;
}

// ---------------------------------------------------------------------------
// Record view shared by all device routines.
struct Rec {
  const GLB float* e;
  const GLB int64_t* y;
  int64_t T;
  int32_t V, U, S, blank;
  int32_t stride;  // backpointer row, words
  GLB uint32_t* bp;
  GLB float* frontier;  // this record's frontier block, or nullptr
  GLB int64_t* labels;  // this record's output rows
  GLB float* scores;
  const int16_t* ytok;
  // Logits input: row statistics of frame t at st[t - st_first] (LDS in the
  // chunk kernel, global memory elsewhere); nullptr for log-probabilities.
  const float2* st;
  int64_t st_first;
};

// Log-softmax of a raw logit from its row statistics: (x - max) - log(sum).
__device__ inline float lsm(float x, float2 s) { return (x - s.x) - s.y; }

typedef float v2f_t __attribute__((ext_vector_type(2)));
__device__ inline void store_stats(GLB float2* dst, float2 v) { *(GLB v2f_t*)dst = v2f_t{v.x, v.y}; }

// Row statistics of the logits input: m = the row's maximum (a zero maximum is
// taken as +0.0) and ls = logf of the sum of expf(x - m), so that log_softmax
// is lsm(x, {m, ls}), the formula of torch's log_softmax. The sum has one fixed
// order shared by every routine below: lane l of a wave adds expf(x[l + 64k] - m)
// for k = 0, 1, ... in turn, starting from +0.0, then the 64 lane sums combine
// as s[l] += s[l + o] for o = 32, 16, 8, 4, 2, 1. A row of at most 32 values
// held by one lane gives the same bits (lanes 32-63 would add +0.0, which
// leaves every sum of exponentials unchanged).

// One lane, a row of V <= 32 values in registers (x[c] for c >= V unused).
__device__ __attribute__((always_inline)) inline float2 lane_row_stats(const float (&x)[32], int V) {
  float t[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) t[c] = fmaxf(2 * c < V ? x[2 * c] : NEG_INF, 2 * c + 1 < V ? x[2 * c + 1] : NEG_INF);
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
    for (int c = 0; c < w; ++c) t[c] = fmaxf(t[c], t[c + w]);
  const float m = t[0] + 0.0f;
  float e[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) e[c] = c < V ? expf(x[c] - m) : 0.0f;
#pragma unroll
  for (int w = 16; w >= 1; w >>= 1)
#pragma unroll
    for (int c = 0; c < w; ++c) e[c] = e[c] + e[c + w];
  return make_float2(m, logf(e[0]));
}

// R rows (rows_here <= R valid, stride V) by one wave; lane 0 returns the
// statistics. The R rows' loads are interleaved to keep several in flight.
template <int R>
__device__ __attribute__((always_inline)) inline void wave_row_stats(const GLB float* row0, int rows_here, int V,
                                                                      float2 (&out)[R]) {
  const int lane = threadIdx.x & 63;
  float m[R], sum[R];
#pragma unroll
  for (int q = 0; q < R; ++q) { m[q] = NEG_INF; sum[q] = 0.0f; }
  for (int c = lane; c < V; c += 64)
#pragma unroll
    for (int q = 0; q < R; ++q)
      if (q < rows_here) m[q] = fmaxf(m[q], row0[(int64_t)q * V + c]);
#pragma unroll
  for (int q = 0; q < R; ++q) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m[q] = fmaxf(m[q], __shfl_xor(m[q], off, 64));
    m[q] = m[q] + 0.0f;
  }
  for (int c = lane; c < V; c += 64)
#pragma unroll
    for (int q = 0; q < R; ++q)
      if (q < rows_here) sum[q] += expf(row0[(int64_t)q * V + c] - m[q]);
#pragma unroll
  for (int q = 0; q < R; ++q) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum[q] += __shfl_down(sum[q], off, 64);
    out[q] = make_float2(m[q], logf(sum[q]));
  }
}

// Statistics of n consecutive rows by the whole workgroup (waves take groups
// of four rows); lane 0 of each wave writes them to lds_out and / or glb_out.
__device__ __attribute__((always_inline)) inline void rows_stats(const GLB float* rows, int n, int V, float2* lds_out,
                                                                  GLB float2* glb_out) {
  constexpr int R = 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  for (int f0 = wave * R; f0 < n; f0 += nw * R) {
    float2 st[R];
    wave_row_stats<R>(rows + (int64_t)f0 * V, min(R, n - f0), V, st);
    if (lane == 0) {
#pragma unroll
      for (int q = 0; q < R; ++q)
        if (f0 + q < n) {
          if (lds_out) lds_out[f0 + q] = st[q];
          if (glb_out) store_stats(glb_out + f0 + q, st[q]);
        }
    }
  }
}

__device__ inline Rec make_rec(const RecordDesc& d, const Params& p, const Lds& L) {
  Rec r;
  r.e = glb(d.emissions);
  r.y = glb(d.targets);
  r.T = d.frames;
  r.V = d.vocab;
  r.U = d.tokens;
  r.S = 2 * d.tokens + 1;
  r.blank = d.blank;
  r.stride = 2 * ((r.S + 31) / 32);
  r.bp = glb(p.bp) + d.bp_offset;
  r.frontier = d.frontier_offset >= 0 ? glb(p.frontiers) + d.frontier_offset : nullptr;
  r.labels = glb(p.labels) + d.frame_offset;
  r.scores = glb(p.scores) + d.frame_offset;
  r.ytok = L.ytok;
  r.st = nullptr;  // set by kernels built for logits input
  r.st_first = 0;
  return r;
}

__device__ inline int label_of(const Rec& r, int s) { return (s & 1) ? (int)r.ytok[s >> 1] : r.blank; }

__device__ inline void load_tokens(const Rec& r, int16_t* ytok) {
  for (int j = threadIdx.x; j < r.U; j += blockDim.x) ytok[j] = (int16_t)r.y[j];
  __syncthreads();
}

__device__ inline void write_failed(const Rec& r, int64_t a, int64_t b) {  // cu:650-652
  for (int64_t t = a + threadIdx.x; t < b; t += blockDim.x) { r.labels[t] = -1; r.scores[t] = NEG_INF; }
}

// ---------------------------------------------------------------------------
// Viterbi over frames [a, b) of one record (recurrence_impl, cu:355-523).
struct DPOut {
  int terminal;
  float score;
  int start;  // state at frame a after traceback
};

enum { TRACE_NONE = 0, TRACE_ALWAYS = 1, TRACE_IF_FINITE = 2 };

template <int K>
__device__ inline void store_bits(GLB uint32_t* row, int tid, uint32_t bits) {
  if constexpr (K == 4) ((GLB uint8_t*)row)[tid] = (uint8_t)bits;
  else if constexpr (K == 8) ((GLB uint16_t*)row)[tid] = (uint16_t)bits;
  else if constexpr (K == 16) row[tid] = bits;
  else { row[2 * tid] = bits; }
}

template <int K>
struct BitsT { using type = uint32_t; };
template <>
struct BitsT<32> { using type = uint64_t; };

// Write-only target of the DP's backpointer stores from threads past a
// record's states (lane-indexed: at most 64 lanes x 8 bytes); never read.
__device__ uint32_t g_bp_sink[128];

template <int K>
__device__ inline void store_row(GLB uint32_t* row, int tid, typename BitsT<K>::type bits) {
  if constexpr (K == 32) {
    row[2 * tid] = (uint32_t)bits;
    row[2 * tid + 1] = (uint32_t)(bits >> 32);
  } else {
    store_bits<K>(row, tid, (uint32_t)bits);
  }
}

// Path walk from (b-1, terminal) down to a by wave 0 (finish, cu:642-667:
// writes labels and scores; returns the state at frame a).
//
// Batches of up to 64 frames, one per lane: lane i holds eight backpointer
// words (128 states) of frame t-i, from the window's top word down. The walk
// itself is serial and runs in scalar registers, in one of two forms chosen
// per batch by how far the previous batch moved:
//  * steps: groups of 8 frames; a group starts where the current state's word
//    and the one below it are both in the window (8 steps move at most 16
//    states) and resolves its steps from those two words joined into one
//    64-bit value, with the bit offset carried from step to step (no test or
//    branch per step); each step's state goes to its frame's lane. Halfway
//    through a full batch the next batch's words are requested around the
//    current state;
//  * runs (sparse paths, fewer than 8 state changes in the previous batch):
//    every lane reads its frame's move at the current state, a ballot finds
//    the first frame that moves, the frames up to it take the current state,
//    and the state then takes that frame's move: one round per state change
//    instead of one per frame. The next batch's words are requested when the
//    batch starts, with the same top word.
// A batch whose state leaves its window ends there and requests a new one. A
// batch's score gathers are stored during the next batch, so the walk does
// not wait for them.
__device__ __attribute__((always_inline)) inline int trace_path(const Rec& r, int64_t a, int64_t b, int terminal) {
  const int lane = threadIdx.x & 63;
  const int64_t stride = r.stride;
  constexpr int WW = 8;  // words per lane
  auto load_window = [&](int64_t t, int wb, uint32_t (&w)[WW]) {
    const int64_t ti = t - lane;
#pragma unroll
    for (int j = 0; j < WW; ++j) w[j] = 0;
    if (ti >= a) {
      const GLB uint32_t* row = r.bp + ti * stride;
#pragma unroll
      for (int j = 0; j < WW; ++j)
        if (wb - j >= 0) w[j] = row[wb - j];
    }
  };
  int64_t t = b - 1;
  int cur = terminal;
  int wb = cur >> 4;  // word of w[0]
  uint32_t w[WW], wn[WW];
  load_window(t, wb, w);
  // score of the previous batch's frame of this lane, stored during the next batch
  bool pend = false;
  int64_t pend_tf = 0;
  float pend_v = 0.0f;
  float2 pend_st = make_float2(0.0f, 0.0f);
  auto flush = [&] {
    if (pend) r.scores[pend_tf] = r.st ? lsm(pend_v, pend_st) : pend_v;
    pend = false;
  };
  bool runs = 8 * (int64_t)r.S < b - a;  // first batch: the record's states per frame
  while (t >= a) {
    const int lim = (int)min((int64_t)64, t - a + 1);
    const bool full = lim == 64 && t - 64 >= a;  // a next batch of frames follows
    const int from = cur;
    int mine = 0, pos = 0, wbn = -1;
    if (runs) {
      if (full) {
        wbn = wb;
        load_window(t - 64, wbn, wn);
      }
      const uint64_t live = lim == 64 ? ~0ull : (1ull << lim) - 1;
      int wsel = -1;
      uint32_t x = 0;  // this lane's word holding the current state
      bool flushed = false;
      while (pos < lim) {
        const int ws = cur >> 4;
        if (ws != wsel) {
          const int dw = wb - ws;
          if (dw > WW - 1) break;  // the state left the window: the batch ends here
          x = w[0];
#pragma unroll
          for (int j = 1; j < WW; ++j)
            if (dw == j) x = w[j];
          wsel = ws;
        }
        const uint32_t mv = (x >> (2 * (cur & 15))) & 3u;
        const uint64_t moving = __ballot(mv != 0) & live & (~0ull << pos);
        const int l = moving ? (int)__builtin_ctzll(moving) : lim - 1;  // last frame of the run
        if (lane >= pos && lane <= l) mine = cur;
        if (!flushed) { flush(); flushed = true; }
        pos = l + 1;
        if (!moving) break;
        cur -= __builtin_amdgcn_readlane((int)mv, l);
      }
    } else {
      for (int g = 0; g < lim; g += 8) {
        const int wsel = cur >> 4;
        const int dw = wb - wsel;  // w[dw] and w[dw + 1] hold the group's two words
        if (dw > WW - 2) break;
        uint32_t vh = w[0], vl = w[1];
#pragma unroll
        for (int j = 1; j <= WW - 2; ++j)
          if (dw == j) { vh = w[j]; vl = w[j + 1]; }
        int sh = 2 * (cur - (wsel - 1) * 16);  // bit offset of the state in {vh:vl}
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t hv = (uint32_t)__builtin_amdgcn_readlane((int)vh, g + j);
          const uint32_t lv = (uint32_t)__builtin_amdgcn_readlane((int)vl, g + j);
          const int mv = (int)(((uint64_t)hv << 32 | lv) >> sh) & 3;
          mine = lane == g + j ? cur : mine;
          cur -= mv;
          sh -= 2 * mv;
        }
        // frames past the interval read zero words: their steps do not move
        pos = min(g + 8, lim);
        if (g == 0) flush();
        if (g == 24 && full) {
          wbn = cur >> 4;
          load_window(t - 64, wbn, wn);
        }
      }
    }
    const int steps = pos;
    const int64_t tn = t - steps;
    if (tn >= a) {
      const int wfirst = cur >> 4;
      if (steps == 64 && wbn >= 0 && wbn - wfirst <= WW - 2) {
#pragma unroll
        for (int j = 0; j < WW; ++j) w[j] = wn[j];
        wb = wbn;
      } else {
        wb = wfirst;
        load_window(tn, wb, w);
      }
    }
    if (lane < steps) {
      const int64_t tf = t - lane;
      const int lab = label_of(r, mine);
      r.labels[tf] = lab;
      pend = true;
      pend_tf = tf;
      pend_v = r.e[tf * r.V + lab];
      if (r.st) pend_st = r.st[tf - r.st_first];
    }
    runs = 8 * (from - cur) < steps;
    t = tn;
  }
  flush();
  return cur;
}

// How the frame loop knows whether the workgroup has several waves: fixed
// at compile time (single / multi) or read at run time.
template <int MODE>
struct Waves {
  static constexpr int mode = MODE;  // 0 one wave, 1 several, 2 decided at run time
};

// LG: logits input (emission reads pass through lsm with r.st); a template
// parameter so that the log-probability build carries none of it. BYREC (the
// chunk and tail kernels): the K = 4 loops pick the one-wave form by the
// record's width, not the workgroup's (the conventional kernel keeps the
// workgroup test: its longest record sets its time and takes the same loop).
template <int K, int D, bool LG, bool BYREC = true>
__device__ __attribute__((always_inline)) DPOut dp_interval(const Rec& r, const Lds& L, int64_t a, int64_t b, bool record_end,
                             const GLB float* resume_from, int64_t start_t, GLB float* save_frontier, int trace) {
  using Bits = typename BitsT<K>::type;
  Header* h = L.h;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
  const int S = r.S;
  const int s0 = tid * K;
  const bool active = s0 < S;
  constexpr bool kMask = K == 32;
  uint32_t lab[K];  // byte offset of the state's label column within a frame row
  float skb[kMask ? 1 : K];  // 0 where the skip transition is legal, -inf elsewhere (cu:407)
  uint32_t skm = 0;          // the same as a bit mask when K == 32
  float al[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int s = s0 + k;
    const int ls = s < S ? label_of(r, s) : r.blank;
    lab[k] = 4u * (uint32_t)ls;
    const bool ok = s >= 2 && s < S && ls != r.blank && ls != label_of(r, s - 2);
    if constexpr (kMask) skm |= (uint32_t)ok << k;
    else skb[k] = ok ? 0.0f : NEG_INF;
  }
  const GLB float* e = r.e;
  const int64_t V = r.V;
  GLB uint32_t* bp = r.bp;
  // Exchange and store forms per state width, each the fastest measured
  // (the K = 8/16 loops slow down by 5% with any of the other forms, even
  // with only the slot numbering changed):
  //   K = 4:  exchanged value as the lane-0 fill of the DPP shift, sink store
  //           (threads without states store their unused frame bits into a
  //           sink instead of branching around the store every frame);
  //   K = 32, conventional kernel: DPP shifts independent of the exchange
  //           read, lane 0 selects it afterwards, sink store;
  //   K = 8, 16, and K = 32 in the chunk and tail kernels: lane 0 of waves
  //           past the first reads in a branch, stores only from threads with
  //           states (K = 32's chunk and tail kernels run at the register
  //           limit; the other forms move spills into their frame loops and
  //           made C3 optimized 55% slower).
  // Forms 1 and 2 read every lane's own wave slot: wave w's last states go
  // to slot w + 1 and slot 0 holds -inf for wave 0 (nothing writes it); the
  // branch form keeps wave w in slot w.
  constexpr int kRead = K == 4 ? 1 : (K == 32 && !BYREC) ? 2 : 0;
  constexpr bool kSink = kRead != 0;
  constexpr int kSlot = kRead != 0 ? 1 : 0;
  if (resume_from) {
#pragma unroll
    for (int k = 0; k < K; ++k) al[k] = (s0 + k < S) ? resume_from[s0 + k] : NEG_INF;
  } else {
    const GLB float* row = e + a * V;
    const float2 st_a = LG ? r.st[a - r.st_first] : make_float2(0.0f, 0.0f);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      float v = ldg_at(row, lab[k]);
      if (LG) v = lsm(v, st_a);
      al[k] = (s0 + k < S && (a > 0 || s0 + k < 2)) ? v : NEG_INF;  // cu:409
    }
    if (active) store_row<K>(bp + a * (int64_t)r.stride, tid, (Bits)0);  // cu:410
    start_t = a + 1;
  }
  if (nwaves > 1) {  // at most 10 waves: slots 0..10 of 16
    if constexpr (kSlot != 0)
      if (tid < 4) h->xchg[tid >> 1][0][tid & 1] = NEG_INF;
    if (lane == 63) {
      h->xchg[(start_t - 1) & 1][wave + kSlot][0] = al[K - 2];
      h->xchg[(start_t - 1) & 1][wave + kSlot][1] = al[K - 1];
    }
    __syncthreads();
  }
  // One frame of the recurrence (cu:438-444); strict '>' keeps stay > advance >
  // skip on ties. `evk` holds e[t][l[s]] for this thread's states. `waves`
  // (a Waves<> tag) says whether the workgroup has more than one wave; for
  // K = 4 the frame loops are compiled once for each case, so a single-wave
  // workgroup carries no cross-wave exchange code.
  auto frame = [&](auto waves, int64_t t, const float (&evk)[K]) {
    constexpr int WM = decltype(waves)::mode;
    const bool M = WM == 2 ? nwaves > 1 : WM == 1;
    // The skip into a thread's first state s0 (even, a blank state) is never
    // legal, so only the previous thread's last state is needed; the
    // multi-wave loops for K <= 16 exchange just that value across waves (the
    // other loops keep both, which measured faster for them).
    constexpr bool kOneUp = K <= 16 && WM == 1;
    float up1, up2;
    if constexpr (kRead == 1) {  // exchange value as the shift's lane-0 fill
      float fill1 = NEG_INF, fill2 = NEG_INF;
      if (M) {
        const int par = (int)((t - 1) & 1);
        fill1 = h->xchg[par][wave][1];
        if constexpr (!kOneUp) fill2 = h->xchg[par][wave][0];
      }
      up1 = wave_shr1(al[K - 1], fill1);
      up2 = kOneUp ? up1 : wave_shr1(al[K - 2], fill2);
    } else if constexpr (kRead == 2) {  // shifts independent of the read; lane 0 selects it
      up1 = wave_shr1(al[K - 1], NEG_INF);
      up2 = kOneUp ? up1 : wave_shr1(al[K - 2], NEG_INF);
      if (M) {
        const int par = (int)((t - 1) & 1);
        const float x1 = h->xchg[par][wave][1];
        if constexpr (!kOneUp) up2 = lane == 0 ? h->xchg[par][wave][0] : up2;
        up1 = lane == 0 ? x1 : up1;
      }
    } else {  // lane 0 of waves past the first reads in a branch
      up1 = wave_shr1(al[K - 1], NEG_INF);
      up2 = kOneUp ? up1 : wave_shr1(al[K - 2], NEG_INF);
      if (M && lane == 0 && wave > 0) {
        const int par = (int)((t - 1) & 1);
        if constexpr (!kOneUp) up2 = h->xchg[par][wave - 1][0];
        up1 = h->xchg[par][wave - 1][1];
      }
    }
    Bits bits = 0;
#pragma unroll
    for (int k = K - 1; k >= 0; --k) {
      const float stay = al[k];
      const float adv = k >= 1 ? al[k - 1] : up1;
      const float skp = k >= 2 ? al[k - 2] : (k == 1 ? up1 : up2);
      float best = stay;
      Bits j = 0;
      if (adv > best) { best = adv; j = 1; }
      // s0 = tid*K is even, so state s0+k is a blank state for even k and the
      // skip into it is never legal (cu:407): no comparison to make
      bool take = false;
      if ((k & 1) != 0) {
        if constexpr (kMask) take = ((skm >> k) & 1u) && skp > best;
        else take = skp + skb[k] > best;
      }
      if (take) { best = skp; j = 2; }
      al[k] = best + evk[k];
      bits |= j << (2 * k);
    }
    if constexpr (kSink)
      store_row<K>((active ? bp : glb(g_bp_sink)) + t * (active ? (int64_t)r.stride : 0), active ? tid : lane, bits);
    else if (active)
      store_row<K>(bp + t * (int64_t)r.stride, tid, bits);
    if (M) {
      if (lane == 63) {
        if constexpr (!kOneUp) h->xchg[t & 1][wave + kSlot][0] = al[K - 2];
        h->xchg[t & 1][wave + kSlot][1] = al[K - 1];
      }
      __syncthreads();
    }
  };
  const int64_t last = b - 1;
  // A record whose states all sit in wave 0 (at most 64 threads' worth) runs
  // the one-wave loop even in a wider workgroup: the other waves hold only
  // states past S, which nothing reads, and wave 0 receives from no wave, so
  // no exchange or barrier is needed per frame (the per-block barriers of the
  // staged path are still met by every wave).
  const bool multi = nwaves > 1 && (!BYREC || r.S > 64 * K);
  if (L.eblk && V <= EBLK_COLS) {
    // Emission rows staged in LDS, one block of F frames at a time (the block's
    // rows are one contiguous span of F*V floats in HBM, so every thread loads
    // plain coalesced dwords). Block k+1 is loaded into registers when block k
    // starts and written to the other half of the double buffer after block
    // k's frames are computed: each load has a whole block of frames to land,
    // and no load result is carried across a loop iteration.
    const int F = L.eblk_frames;
    constexpr int EB = K == 4 ? 32 : 11;  // per-thread values of one block (blockDim >= 64 for K = 4, >= 192 otherwise)
    const int NT = blockDim.x;
    float buf[EB];
    auto load_block = [&](int64_t tb) {
      const int total = (int)(min(tb + F, b) - tb) * (int)V;
      const GLB float* src = e + tb * V;
#pragma unroll
      for (int i = 0; i < EB; ++i) {
        const int idx = tid + i * NT;
        if (idx < total) buf[i] = src[idx];
      }
    };
    const float inv_v = 1.0f / (float)V;
    auto store_block = [&](int64_t tb, float* half) {
      const int total = (int)(min(tb + F, b) - tb) * (int)V;
#pragma unroll
      for (int i = 0; i < EB; ++i) {
        const int idx = tid + i * NT;
        if (idx < total) {
          float v = buf[i];
          if (LG) {  // frame of element idx: idx / V, exact in fp32 for idx < F * V <= 2048
            const int f = (int)(((float)idx + 0.5f) * inv_v);
            v = lsm(v, r.st[tb + f - r.st_first]);
          }
          half[idx] = v;
        }
      }
    };
    int half = 0;
    if (start_t <= last) {
      load_block(start_t);
      store_block(start_t, L.eblk);
      __syncthreads();
    }
    for (int64_t tb = start_t; tb <= last; tb += F) {
      const int64_t nb = tb + F;
      if (nb <= last) load_block(nb);
      const float* rows = L.eblk + half * F * EBLK_COLS;
      const int nf = (int)min((int64_t)F, last - tb + 1);
      auto frames = [&](auto waves) {
        auto one = [&](int f) {
          float evk[K];
          const float* row = rows + f * (int)V;
#pragma unroll
          for (int k = 0; k < K; ++k) evk[k] = *(const float*)((const char*)row + lab[k]);
          frame(waves, tb + f, evk);
        };
        for (int f = 0; f < nf; ++f) one(f);
      };
      // (K >= 8 only comes with more than 128 threads: always several waves;
      // K = 32 keeps a plain loop, which spills less in the chunk and tail kernels)
      if constexpr (K == 4) {
        if (multi) frames(Waves<1>{});
        else frames(Waves<0>{});
      } else if constexpr (K == 32) {
        for (int f = 0; f < nf; ++f) {
          float evk[K];
          const float* row = rows + f * (int)V;
#pragma unroll
          for (int k = 0; k < K; ++k) evk[k] = *(const float*)((const char*)row + lab[k]);
          frame(Waves<2>{}, tb + f, evk);
        }
      } else {
        frames(Waves<1>{});
      }
      if (nb <= last) store_block(nb, L.eblk + (half ^ 1) * F * EBLK_COLS);
      __syncthreads();  // the next block is in LDS; this block's reads are done
      half ^= 1;
    }
  } else {
  // Prefetch ring: the gathers of frame t are issued D frames ahead; loads past
  // the interval are clamped to its last row so every load is unconditional.
  // The main loop runs whole groups of D frames with no exits inside a group.
  float ev[D][K];
  // logits: the row statistics travel with the gathers and are applied when
  // the frame is computed
  float2 es[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int64_t t = min(start_t + d, last);
    const GLB float* row = e + t * V;
#pragma unroll
    for (int k = 0; k < K; ++k) ev[d][k] = ldg_at(row, lab[k]);
    es[d] = LG ? r.st[t - r.st_first] : make_float2(0.0f, 0.0f);
  }
  auto apply = [&](float (&evk)[K], float2 st) {
    if (LG) {
#pragma unroll
      for (int k = 0; k < K; ++k) evk[k] = lsm(evk[k], st);
    }
  };
  auto ring = [&](auto waves) {
    int64_t t0 = start_t;
    for (; t0 + D <= b; t0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        apply(ev[d], es[d]);
        frame(waves, t0 + d, ev[d]);
        const int64_t t = min(t0 + d + D, last);
        const GLB float* row = e + t * V;
#pragma unroll
        for (int k = 0; k < K; ++k) ev[d][k] = ldg_at(row, lab[k]);
        if (LG) es[d] = r.st[t - r.st_first];
      }
    }
    // remaining < D frames: their gathers are already in ev[0 .. b-t0-1]
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (t0 + d < b) {
        apply(ev[d], es[d]);
        frame(waves, t0 + d, ev[d]);
      }
  };
  if constexpr (K == 4) {
    if (multi) ring(Waves<1>{});
    else ring(Waves<0>{});
  } else if constexpr (K == 32) {  // plain loop (spills less in the chunk and tail kernels)
    int64_t t0 = start_t;
    for (; t0 + D <= b; t0 += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        apply(ev[d], es[d]);
        frame(Waves<2>{}, t0 + d, ev[d]);
        const int64_t t = min(t0 + d + D, last);
        const GLB float* row = e + t * V;
#pragma unroll
        for (int k = 0; k < K; ++k) ev[d][k] = ldg_at(row, lab[k]);
        if (LG) es[d] = r.st[t - r.st_first];
      }
    }
#pragma unroll
    for (int d = 0; d < D; ++d)
      if (t0 + d < b) {
        apply(ev[d], es[d]);
        frame(Waves<2>{}, t0 + d, ev[d]);
      }
  } else {
    ring(Waves<1>{});
  }
  }
  if (save_frontier) {  // cu:451-454
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (s0 + k < S) save_frontier[s0 + k] = al[k];
  }
  DPOut out;
  if (record_end) {  // cu:497-500
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int s = s0 + k;
      if (s == S - 1) h->term_v[1] = al[k];
      if (S > 1 && s == S - 2) h->term_v[0] = al[k];
    }
    __syncthreads();
    out.terminal = S - 1;
    out.score = h->term_v[1];
    if (S > 1 && h->term_v[0] >= h->term_v[1]) { out.terminal = S - 2; out.score = h->term_v[0]; }
  } else {  // lowest-index argmax with the NaN-at-state-0 rule, cu:462-492
    float bv = NEG_INF;
    int bi = INT_MAX;
#pragma unroll
    for (int k = 0; k < K; ++k)
      if (s0 + k < S) better(bv, bi, al[k], s0 + k);
    wave_argmax(bv, bi);
    if (lane == 0) { h->red_v[wave] = bv; h->red_i[wave] = bi; }
    if (tid == 0) h->fbuf[0] = al[0];
    __syncthreads();
    bv = h->red_v[0];
    bi = h->red_i[0];
    for (int w = 1; w < nwaves; ++w) better(bv, bi, h->red_v[w], h->red_i[w]);
    const float a0 = h->fbuf[0];
    if (isnan(a0)) { bi = 0; bv = a0; }
    out.terminal = bi;
    out.score = bv;
  }
  __syncthreads();  // backpointer stores and LDS reads complete before the walk / reuse
  out.start = 0;
  const bool do_trace = trace == TRACE_ALWAYS || (trace == TRACE_IF_FINITE && isfinite(out.score));
  if (do_trace) {
    if (wave == 0) {
      const int st = trace_path(r, a, b, out.terminal);
      if (lane == 0) h->ibuf[0] = st;
    }
    __syncthreads();
    out.start = h->ibuf[0];
    __syncthreads();
  }
  return out;
}

// ---------------------------------------------------------------------------
// Result of target staging (stage_targets below).
struct Staged {
  int status;
  uint32_t alpha32;
  int blank_in;  // some in-vocabulary target equals the blank id (only reachable unchecked)
};

enum { ALPHABET_NONE = 0, ALPHABET_MASK32 = 1, ALPHABET_BITMAP = 2 };

template <int CTRL, int ROW_MASK>
__device__ inline int dpp_or(int v) {
  return v | __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xf, false);
}

// Wave64 inclusive OR-scan (same DPP pattern as wave_scan_dpp); lane 63 holds
// the OR of all lanes.
__device__ inline int wave_or_scan_dpp(int x) {
  x = dpp_or<0x111, 0xf>(x);
  x = dpp_or<0x112, 0xf>(x);
  x = dpp_or<0x114, 0xf>(x);
  x = dpp_or<0x118, 0xf>(x);
  x = dpp_or<0x142, 0xa>(x);
  x = dpp_or<0x143, 0xc>(x);
  return x;
}

// Prefilter key of three consecutive targets: exact for V <= 32 (5 bits each),
// a 16-bit hash otherwise (candidates are always verified token by token).
__device__ inline uint32_t tri_key(int x0, int x1, int x2, bool small) {
  return small ? ((uint32_t)(x0 & 31) | (uint32_t)(x1 & 31) << 5 | (uint32_t)(x2 & 31) << 10)
               : (((uint32_t)x0 * 40503u + (uint32_t)x1 * 30011u + (uint32_t)x2 * 52511u) & 0xffffu);
}

// The first batch of a thread's targets, loaded before the values that the
// checks need (V, blank, T) are known. Thread k owns targets
// [k*per, (k+1)*per), per = ceil(U / threads), processed in batches of 8 with
// the one before (repeat count) and the two after (keys). Every thread loads
// with clamped indices and no branch, so the compiler can wait for these
// loads without waiting for loads issued after them (the chunk's rows). An
// empty transcript reads the descriptor table instead (values unused).
struct TargetLoads {
  const GLB int64_t* ys;
  int U, j0, j1, jlast;
  int64_t before;
  int64_t v[10];
};

__device__ __attribute__((always_inline)) inline void load_target_batch(TargetLoads& t, int jb) {
#pragma unroll
  for (int q = 0; q < 10; ++q) t.v[q] = t.ys[min(jb + q, t.jlast)];
}

__device__ __attribute__((always_inline)) inline TargetLoads issue_targets(const GLB int64_t* y, int U, const Params& p) {
  TargetLoads t;
  const int per = (U + (int)blockDim.x - 1) / (int)blockDim.x;
  t.U = U;
  t.j0 = threadIdx.x * per;
  t.j1 = min(U, t.j0 + per);
  t.ys = U > 0 ? y : (const GLB int64_t*)glb(p.desc);
  t.jlast = max(min(U, t.j1 + 2) - 1, 0);  // two past the range: the keys' lookahead
  t.before = t.ys[min(max(t.j0 - 1, 0), max(U - 1, 0))];  // compared only for j > 0
  load_target_batch(t, min(t.j0, t.jlast));
  return t;
}

// Checks and LDS staging of the loaded targets (see stage_targets),
// specialized for the alphabet form and the keys.
template <int ALPHABET, bool KEYS, bool PEEL = false>
__device__ __attribute__((always_inline)) Staged finish_targets(TargetLoads& t, int V, int blank, int64_t T, int rec,
                                                                 const Params& p, const Lds& L) {
  Header* h = L.h;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const int U = t.U, j0 = t.j0, j1 = t.j1;
  if constexpr (ALPHABET == ALPHABET_BITMAP) {
    for (int w = tid; w < (V + 31) / 32; w += blockDim.x) L.bitmap[w] = 0;
    __syncthreads();
    if (tid == 0) atomicOr(&L.bitmap[blank >> 5], 1u << (blank & 31));
  }
  bool oov = false, bin = false;
  int repeats = 0;
  uint32_t mask = 0;
  int64_t before = t.before;
  uint32_t before32 = (uint32_t)before;  // low word of the target before the current one (PEEL)
  // PEEL (chunk kernel): the first batch (loaded by issue_targets) is staged
  // outside the loop. As a loop-carried value it is copied between
  // registers, and the copy waits for every load in flight, the chunk's rows
  // included. The other kernels keep the loop form, which their DP loops'
  // code generation was measured with.
  auto batch = [&](int jb) {
    // 32-bit checks: a target is in the vocabulary iff its high word is zero
    // and its low word is below V (the int64 check of cu:860). Repeats
    // compare low words only; they differ from the int64 comparison only
    // when a target is out of the vocabulary, and then the status is 3
    // whatever the count (cu:861, cu:872-873).
    int tv[10];  // the staged int16 value of target jb+q: 0 when out of vocabulary, -1 past the end
    bool outq[10];
#pragma unroll
    for (int q = 0; q < 10; ++q) {
      const uint32_t lo = (uint32_t)t.v[q], hi = (uint32_t)((uint64_t)t.v[q] >> 32);
      outq[q] = (hi | (uint32_t)(lo >= (uint32_t)V)) != 0;
      tv[q] = jb + q < U ? (outq[q] ? 0 : (int)lo) : -1;
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int j = jb + q;
      if (j < j1) {
        const uint32_t lo = (uint32_t)t.v[q];
        const bool out = outq[q];
        oov |= out;
        bin |= !out && (int)lo == blank;
        repeats += j > 0 && lo == before32;
        before32 = lo;
        L.ytok[j] = (int16_t)tv[q];
        if constexpr (KEYS) L.key3[j] = (uint16_t)tri_key(tv[q], tv[q + 1], tv[q + 2], ALPHABET == ALPHABET_MASK32);
        if (!out) {
          if constexpr (ALPHABET == ALPHABET_BITMAP) atomicOr(&L.bitmap[lo >> 5], 1u << (lo & 31));
          if constexpr (ALPHABET == ALPHABET_MASK32) mask |= 1u << (lo & 31);
        }
      }
    }
  };
  if constexpr (PEEL) {
    // One wait for all of a batch's target loads on every path (they return
    // together). Otherwise the look-ahead targets that the branches below do
    // not read stay pending in the compiler's model, and it later waits for
    // every load in flight, the rows included, before reusing their registers.
    auto settle = [&] {
#pragma unroll
      for (int q = 0; q < 10; ++q) asm volatile("" ::"v"(t.v[q]));
    };
    asm volatile("" ::"v"(t.before));
    settle();
    if (j0 < j1) batch(j0);
    for (int jb = j0 + 8; jb < j1; jb += 8) {
      load_target_batch(t, jb);
      settle();
      batch(jb);
    }
  } else {
    for (int jb = j0; jb < j1; jb += 8) {
      if (jb > j0) load_target_batch(t, jb);
      int tv[10];  // the staged int16 value of target jb+q: 0 when out of vocabulary, -1 past the end
#pragma unroll
      for (int q = 0; q < 10; ++q) {
        const int64_t tok = t.v[q];
        tv[q] = jb + q < U ? ((tok < 0 || tok >= V) ? 0 : (int)tok) : -1;
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int j = jb + q;
        if (j < j1) {
          const int64_t tok = t.v[q];
          const bool out = tok < 0 || tok >= V;  // checked as int64 before narrowing (cu:860)
          oov |= out;
          bin |= !out && tok == blank;
          repeats += j > 0 && tok == before;  // cu:861
          before = tok;
          L.ytok[j] = (int16_t)tv[q];
          if constexpr (KEYS) L.key3[j] = (uint16_t)tri_key(tv[q], tv[q + 1], tv[q + 2], ALPHABET == ALPHABET_MASK32);
          if (!out) {
            if constexpr (ALPHABET == ALPHABET_BITMAP) atomicOr(&L.bitmap[tok >> 5], 1u << (tok & 31));
            if constexpr (ALPHABET == ALPHABET_MASK32) mask |= 1u << (tok & 31);
          }
        }
      }
    }
  }
  // sentinel padding after the targets: the placement prefilter reads ahead
  for (int j = U + tid; j < U + YTOK_PAD; j += blockDim.x) L.ytok[j] = -1;
  // wave reductions: ballots for the flags, DPP scans for the count and the mask
  const int wf = (__ballot(oov) != 0 ? 1 : 0) | (__ballot(bin) != 0 ? 2 : 0);
  const int wr = __builtin_amdgcn_readlane(wave_scan_dpp(repeats), 63);
  const int wm = ALPHABET == ALPHABET_MASK32 ? __builtin_amdgcn_readlane(wave_or_scan_dpp((int)mask), 63) : 0;
  int flags = 0, reps = 0;
  uint32_t m = ALPHABET == ALPHABET_MASK32 ? 1u << blank : 0u;
  if constexpr (PEEL) {
    if (lane == 0) h->stg[wave] = StageWave{wf, wr, (uint32_t)wm, 0};
    __syncthreads();
    for (int w0 = 0; w0 < nw; w0 += 4) {  // four records in flight (nw <= 10: reads past nw stay in the array, unused)
      StageWave sw[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) sw[k] = h->stg[w0 + k];
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (w0 + k < nw) {
          flags |= sw[k].flags;
          reps += sw[k].repeats;
          m |= sw[k].mask;
        }
    }
  } else {
    if (lane == 0) {
      h->stg_f[wave] = wf;
      h->stg_r[wave] = wr;
      h->stg_m[wave] = (uint32_t)wm;
    }
    __syncthreads();
    for (int w = 0; w < nw; ++w) {
      flags |= h->stg_f[w];
      reps += h->stg_r[w];
      m |= h->stg_m[w];
    }
  }
  Staged st;
  st.alpha32 = m;
  st.blank_in = (flags & 2) ? 1 : 0;
  if (flags & 1) st.status = 3;
  else if (p.check_inputs && (flags & 2)) st.status = 3;                // cu:872
  else if (p.check_inputs && (int64_t)U + reps > T) st.status = 4;      // cu:873
  else st.status = (p.validity && !glb(p.validity)[rec]) ? 2 : 0;     // cu:836
  return st;
}

// Target staging and validation (pack_inputs, cu:819-877), done by every
// workgroup that needs the record: copies the targets into LDS as int16,
// computes the status and the transcript alphabet (cu:53-58). For V <= 32 the
// alphabet is returned as a bit mask; otherwise it is left in L.bitmap. With
// `keys`, the placement prefilter keys of every target position are built too
// (from registers: each thread loads two targets past its range). Out-of-
// vocabulary ids are rejected (status 3) even unchecked: the reference reads
// out of bounds there (py:400-402); this build never reads outside the
// emission rows. One workgroup barrier.
template <int ALPHABET, bool KEYS>
__device__ __attribute__((always_inline)) Staged stage_targets(const GLB int64_t* y, int U, int V, int blank, int64_t T,
                                                                int rec, const Params& p, const Lds& L) {
  TargetLoads t = issue_targets(y, U, p);
  return finish_targets<ALPHABET, KEYS>(t, V, blank, T, rec, p, L);
}

template <int ALPHABET>
__device__ inline Staged stage_tokens(const RecordDesc& d, const Params& p, int rec, const Lds& L) {
  return stage_targets<ALPHABET, false>(glb(d.targets), d.tokens, d.vocab, d.blank, d.frames, rec, p, L);
}

__device__ inline bool legal_seam(const Rec& r, int start, int before) {  // cu:157-161
  const int jump = start - before;
  return jump == 0 || jump == 1 ||
         (jump == 2 && label_of(r, start) != r.blank && label_of(r, start) != label_of(r, start - 2));
}

// Literal placement test of the reference (cu:119-134), used when an
// in-vocabulary target equals the blank id (reachable only with
// check_inputs=False): the substring formulation below assumes blank labels sit
// at even states only. Every start state is checked against every label change
// of the chunk. Needs the greedy labels in L.g[0, n); fills L.pd / L.pc with the
// change offsets and labels. Workgroup-wide; returns the number of legal
// placements, *start (meaningful when exactly one) and *rlast.
__device__ __attribute__((always_inline)) int place_literal(const Lds& L, const int16_t* ytok, int n, int S, int blank, bool at_start, bool at_end,
                             int* start, int* rlast) {
  Header* h = L.h;
  const int tid = threadIdx.x, NT = blockDim.x;
  int carry = 0;  // r | changes << 16
  for (int base = 0; base < n; base += NT) {
    const int f = base + tid;
    int inc = 0, chg = 0;
    if (f < n && f > 0) {
      const int x = L.g[f], w = L.g[f - 1];
      chg = x != w;
      inc = x == w ? 0 : (x == blank || w == blank ? 1 : 2);  // cu:112-117
    }
    const int v = block_incl_scan(inc | (chg << 16), h) + carry;
    if (f < n) {
      L.r[f] = v & 0xffff;
      if (chg) {
        L.pd[v >> 16] = v & 0xffff;
        L.pc[v >> 16] = L.g[f];
      }
    }
    if (tid == NT - 1) h->ibuf[2] = v;
    __syncthreads();
    carry = h->ibuf[2];
    __syncthreads();
  }
  const int segs = (carry >> 16) + 1;
  const int rl = carry & 0xffff;
  const int g0 = L.g[0];
  if (tid == 0) h->ibuf[4] = -1;
  __syncthreads();
  int local = 0;
  for (int s = tid; s < S; s += NT) {
    const int ls = (s & 1) ? (int)ytok[s >> 1] : blank;
    const int terminal = s + rl;
    bool legal = ls == g0 && !(at_start && s > 1) && terminal < S && !(at_end && terminal < S - 2);
    for (int k = 1; k < segs && legal; ++k) {
      const int q = s + L.pd[k];
      legal = ((q & 1) ? (int)ytok[q >> 1] : blank) == L.pc[k];
    }
    if (legal) { ++local; h->ibuf[4] = s; }
  }
  const int matches = block_sum(local, h);
  *start = h->ibuf[4];
  *rlast = rl;
  __syncthreads();
  return matches;
}

// ---------------------------------------------------------------------------
// Greedy shortcut for chunk [a, b) (greedy_shortcuts, cu:30-153).
//
// Per frame: the unique maximum over the transcript alphabet (ties or a
// non-finite maximum reject the chunk). The greedy labels define a relative
// state walk r (0 same label, 1 when a blank is involved, 2 token to token).
// The token change points form a pattern c_1..c_m; a start state s is a legal
// placement iff the pattern equals the contiguous target substring
// y[j .. j+m) (s = 2j+1-r(first token)), plus the start/end constraints of the
// reference's placement loop. This is exactly the set the reference's O(S*H)
// loop accepts; here candidates are prefiltered on three tokens and the rest
// is checked with one comparison per (candidate, position) pair.
//
// Returns 1 when accepted (labels and scores written, *slot filled);
// *ambiguous is set when more than one placement is legal.
constexpr int CAND_CAP = 256;

// AG: labels and scores are written with agent-scope stores (fused tail).
template <bool AG>
__device__ __attribute__((always_inline)) int greedy_chunk(const Rec& r, const Lds& L, int64_t a, int64_t b, bool blank_in, Slot& out, int* ambiguous) {
  Header* h = L.h;
  const int tid = threadIdx.x, NT = blockDim.x;
  const int n = (int)(b - a);
  const int V = r.V, blank = r.blank, S = r.S, U = r.U;
  int bad = 0;
  {
    // general vocabulary: compact symbol list, then gathered loads per frame
    const int vw = (V + 31) >> 5;
    if (tid == 0) {
      uint32_t acc = 0;
      for (int w = 0; w < vw; ++w) { L.wpref[w] = acc; acc += __popc(L.bitmap[w]); }
      h->ibuf[1] = (int)acc;
    }
    __syncthreads();
    const int D = h->ibuf[1];
    for (int c = tid; c < V; c += NT) {
      const uint32_t word = L.bitmap[c >> 5];
      if (word >> (c & 31) & 1u) L.sym[L.wpref[c >> 5] + __popc(word & ((1u << (c & 31)) - 1u))] = (int16_t)c;
    }
    __syncthreads();
    for (int f = tid; f < n; f += NT) {
      const GLB float* row = r.e + (a + f) * (int64_t)V;
      const float2 st_f = r.st ? r.st[a + f - r.st_first] : make_float2(0.0f, 0.0f);
      float best = NEG_INF;
      int chosen = -1;
      bool dup = false;
      for (int base = 0; base < D; base += 8) {
        float v[8];
        int c[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          c[q] = L.sym[min(base + q, D - 1)];
          v[q] = ldg_at(row, 4u * (uint32_t)c[q]);
        }
        if (r.st) {
#pragma unroll
          for (int q = 0; q < 8; ++q) v[q] = lsm(v[q], st_f);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          if (base + q < D) {
            const bool gt = v[q] > best, eq = v[q] == best;
            best = gt ? v[q] : best;
            chosen = gt ? c[q] : chosen;
            dup = gt ? false : (dup || eq);
          }
        }
      }
      L.g[f] = chosen;
      L.fs[f] = best;
      bad |= !isfinite(best) || dup;
    }
  }
  bad = __syncthreads_or(bad);
  *ambiguous = 0;
  if (bad) { __syncthreads(); return 0; }
  const bool at_start = a == 0, at_end = b == r.T;
  int matches = 0, start = -1, rlast = 0;
  if (blank_in) {
    matches = place_literal(L, L.ytok, n, S, blank, at_start, at_end, &start, &rlast);
  } else {
  // relative walk and token pattern in one scan: low 16 bits r, high 16 bits
  // the running count of token change points
  int carry = 0;
  for (int base = 0; base < n; base += NT) {
    const int f = base + tid;
    int inc = 0, tc = 0, x = 0;
    if (f < n) {
      x = L.g[f];
      const int w = f > 0 ? L.g[f - 1] : -1;
      if (f > 0) inc = x == w ? 0 : (x == blank || w == blank ? 1 : 2);
      tc = x != blank && (f == 0 || x != w);
    }
    const int v = block_incl_scan(inc | (tc << 16), h) + carry;
    if (f < n) {
      L.r[f] = v & 0xffff;
      if (tc) {
        const int pos = (v >> 16) - 1;
        L.pc[pos] = x;
        L.pd[pos] = v & 0xffff;
      }
    }
    if (tid == NT - 1) h->ibuf[2] = v;
    __syncthreads();
    carry = h->ibuf[2];
    __syncthreads();
  }
  const int m = carry >> 16;
  rlast = L.r[n - 1];
  if (m == 0) {
    // all-blank chunk: even states, closed form of the placement loop (cu:119-134)
    if (at_start && at_end) { matches = (S == 1) ? 1 : 0; start = 0; }
    else if (at_start) { matches = 1; start = 0; }
    else if (at_end) { matches = 1; start = S - 1; }
    else { matches = (S + 1) / 2; start = 0; }
  } else {
    const int r1 = L.pd[0];
    const int pre = min(m, 3);
    // placement constraints of cu:119-123 for target position j (state s = 2j+1-r1)
    auto placeable = [&](int j) {
      const int s = 2 * j + 1 - r1;
      const int terminal = s + rlast;
      return !((at_start && s > 1) || terminal >= S || (at_end && terminal < S - 2));
    };
    if (tid == 0) h->ibuf[3] = 0;
    __syncthreads();
    for (int j = tid; j + m <= U; j += NT) {  // prefilter on the first three pattern tokens
      bool hit = L.ytok[j] == L.pc[0];
      for (int i = 1; i < pre && hit; ++i) hit = L.ytok[j + i] == L.pc[i];
      if (!hit || !placeable(j)) continue;
      const int k = atomicAdd(&h->ibuf[3], 1);
      if (k < CAND_CAP) { L.cand[k] = j; L.candok[k] = 1; }
    }
    __syncthreads();
    const int total = h->ibuf[3];
    if (total <= CAND_CAP) {
      const int width = m - pre;  // remaining positions, one comparison per (candidate, position)
      for (int q = tid; q < total * width; q += NT) {
        const int ci = q / width, i = pre + q % width;
        if (L.ytok[L.cand[ci] + i] != L.pc[i]) L.candok[ci] = 0;
      }
      __syncthreads();
      int local = 0, mine = -1;
      for (int ci = tid; ci < total; ci += NT)
        if (L.candok[ci]) { ++local; mine = L.cand[ci]; }
      matches = block_sum(local, h);
      if (local) h->ibuf[4] = 2 * mine + 1 - r1;
      __syncthreads();
      start = h->ibuf[4];
    } else {
      // more prefiltered candidates than the list holds: exact serial scan
      // (no realistic transcript repeats a three-token prefix this often)
      if (tid == 0) {
        int count = 0, found = -1;
        for (int j = 0; j + m <= U && count < 2; ++j) {
          bool hit = placeable(j);
          for (int i = 0; i < m && hit; ++i) hit = L.ytok[j + i] == L.pc[i];
          if (hit) { ++count; found = 2 * j + 1 - r1; }
        }
        h->ibuf[3] = count;
        h->ibuf[4] = found;
      }
      __syncthreads();
      matches = h->ibuf[3];
      start = h->ibuf[4];
    }
    __syncthreads();
  }
  }
  if (matches != 1) {
    *ambiguous = matches > 1;
    __syncthreads();
    return 0;
  }
  if (tid == 0) h->fbuf[1] = serial_sum(L.fs, n);  // serial fp32 chunk objective (cu:135-137)
  __syncthreads();
  const float score = h->fbuf[1];
  if (!isfinite(score)) { __syncthreads(); return 0; }  // cu:139
  for (int f = tid; f < n; f += NT) {  // finish's label/score gather collapses to g and fs here
    put<AG>(r.labels + a + f, (int64_t)L.g[f]);
    put<AG>(r.scores + a + f, (float)L.fs[f]);
  }
  out.start = start;
  out.end = start + rlast;
  out.objective = score;
  __syncthreads();
  return 1;
}


// Reads a descriptor every lane needs: 16-byte vector loads (one request per
// instruction for the whole wave), then readfirstlane into scalar registers.
template <class T>
struct Pending {  // a descriptor whose loads are issued but not yet waited for
  v4i_t raw[sizeof(T) / 16];
};

template <class T>
__device__ inline Pending<T> issue_uniform(const T* x) {
  static_assert(sizeof(T) % 16 == 0, "16-byte granules");
  Pending<T> out;
#pragma unroll
  for (size_t i = 0; i < sizeof(T) / 16; ++i) out.raw[i] = ((const GLB v4i_t*)x)[i];
  return out;
}

template <class T>
__device__ inline T finish_uniform(const Pending<T>& x) {
  int w[sizeof(T) / 4];
#pragma unroll
  for (size_t i = 0; i < sizeof(T) / 4; ++i) w[i] = __builtin_amdgcn_readfirstlane(x.raw[i / 4][i % 4]);
  T out;
  __builtin_memcpy(&out, w, sizeof(T));
  return out;
}

template <class T>
__device__ inline T load_uniform(const T* x) {
  return finish_uniform(issue_uniform(x));
}

// Substring placement of a chunk's greedy path by wave 0 (blank-free
// transcripts; cu:119-134). g0 / g1 are the greedy labels of frames lane and
// lane + 64 (-2 past the chunk). The relative walk r (0 same label, 1 when a
// blank is involved, 2 token to token) and the token change points form a
// pattern c_1..c_m; a start state s is a legal placement iff the pattern equals
// the contiguous target substring y[j .. j+m) (s = 2j+1-r1, r1 = r at the first
// token), plus the reference's start/end constraints, which for s = 2j+1-r1
// and terminal s + rlast reduce to an interval of j:
//   terminal < S        <=>  j <= E,  E = (S - 2 + r1 - rlast) >> 1
//   b == T: terminal >= S-2  <=>  j >= E
//   a == 0: s <= 1      <=>  j == 0
// Candidates come from the three-token keys (eight positions per lane per
// 16-byte LDS read) and are verified token by token, one per round, until two
// match. Returns min(number of legal placements, 2), *start and *rlast.
constexpr int VERIFY_CAP = 16;

__device__ __attribute__((always_inline)) int place_wave(const Lds& L, int g0, int g1, int n, int U, int S, int blank,
                                                        bool at_start, bool at_end, bool small_vocab, int* start_out,
                                                        int* rlast_out) {
  const int lane = threadIdx.x & 63;
  // keys of target positions 8*lane .. 8*lane+7, read before the pattern is
  // known (most chunks need only this first block of 512 positions)
  const v4i_t kv0 = *reinterpret_cast<const v4i_t*>(L.key3 + min(8 * lane, (U >> 3) << 3));
  const int gp0 = wave_shr1_int(g0, -1);
  const int gp1 = wave_shr1_int(g1, __builtin_amdgcn_readlane(g0, 63));
  auto step = [&](int f, int g, int gp, int& inc, int& tc) {
    inc = tc = 0;
    if (f >= n) return;
    if (f > 0) inc = g == gp ? 0 : (g == blank || gp == blank ? 1 : 2);  // cu:112-117
    tc = g != blank && (f == 0 || g != gp);
  };
  int inc0, tc0, inc1, tc1;
  step(lane, g0, gp0, inc0, tc0);
  step(lane + 64, g1, gp1, inc1, tc1);
  const int v0 = wave_scan_dpp(inc0 | (tc0 << 16));
  const int v1 = wave_scan_dpp(inc1 | (tc1 << 16)) + __builtin_amdgcn_readlane(v0, 63);
  const int m = __builtin_amdgcn_readlane(v1, 63) >> 16;
  const int rlast = (n <= 64 ? __builtin_amdgcn_readlane(v0, n - 1) : __builtin_amdgcn_readlane(v1, n - 65)) & 0xffff;
  *rlast_out = rlast;
  if (m == 0) {  // all-blank chunk: even states, closed form of the placement loop (cu:119-134)
    *start_out = at_start ? 0 : (at_end ? S - 1 : 0);
    if (at_start && at_end) return S == 1 ? 1 : 0;
    if (at_start || at_end) return 1;
    return min((S + 1) / 2, 2);
  }
  // pattern index of this lane's token change points (-1: none)
  const int i0 = tc0 ? (v0 >> 16) - 1 : -1;
  const int i1 = tc1 ? (v1 >> 16) - 1 : -1;
  // first three pattern tokens and r1 straight from the change-point masks
  uint64_t m0 = __ballot(tc0), m1 = __ballot(tc1);
  int c[3] = {0, 0, 0};
  int r1 = 0;
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    if (m0) {
      const int l = __builtin_ctzll(m0);
      m0 &= m0 - 1;
      c[q] = __builtin_amdgcn_readlane(g0, l);
      if (q == 0) r1 = __builtin_amdgcn_readlane(v0, l) & 0xffff;
    } else if (m1) {
      const int l = __builtin_ctzll(m1);
      m1 &= m1 - 1;
      c[q] = __builtin_amdgcn_readlane(g1, l);
      if (q == 0) r1 = __builtin_amdgcn_readlane(v1, l) & 0xffff;
    }
  }
  const int E = (S - 2 + r1 - rlast) >> 1;
  const int jlo = at_end ? max(E, 0) : 0;
  const int jhi = min(min(E, U - m), at_start ? 0 : INT_MAX);
  int matches = 0, start = -1;
  if (jlo > jhi) { *start_out = -1; return 0; }
  // y[j .. j+m) == pattern, checked in frame space: each change point compares
  // its own label with the target at its pattern index (all lanes take part)
  auto verify = [&](int j) {  // branch-free: both reads are in bounds (j + max(i, 0) < U)
    const int y0 = L.ytok[j + max(i0, 0)];
    const int y1 = L.ytok[j + max(i1, 0)];
    const bool bad = ((i0 >= 0) & (y0 != g0)) | ((i1 >= 0) & (y1 != g1));
    return __ballot(bad) == 0;
  };
  if (m >= 3 && jhi - jlo >= 8) {
    const uint32_t pkey = tri_key(c[0], c[1], c[2], small_vocab);
    // count the key hits first: 8 positions per lane per 16-byte read
    int total = 0;
    for (int base = jlo & ~7; base <= jhi; base += 512) {
      const int j0 = base + 8 * lane;
      const v4i_t kv = base == 0 ? kv0 : *reinterpret_cast<const v4i_t*>(L.key3 + min(j0, (jhi & ~7)));
      uint32_t hits = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t key = ((uint32_t)kv[e >> 1] >> (16 * (e & 1))) & 0xffffu;
        const int j = j0 + e;
        hits |= (uint32_t)((key == pkey) & (j >= jlo) & (j <= jhi)) << e;
      }
      const int cnt = __builtin_amdgcn_readlane(wave_scan_dpp(__popc(hits)), 63);
      if (cnt && total + cnt <= VERIFY_CAP) {
        // verify this block's candidates in order, lowest position first
        uint64_t lanes_hit = __ballot(hits != 0);
        while (lanes_hit && matches < 2) {
          const int l = __builtin_ctzll(lanes_hit);
          lanes_hit &= lanes_hit - 1;
          uint32_t h8 = (uint32_t)__builtin_amdgcn_readlane((int)hits, l);
          while (h8 && matches < 2) {
            const int j = base + 8 * l + __builtin_ctz(h8);
            h8 &= h8 - 1;
            if (verify(j)) {
              if (matches == 0) start = 2 * j + 1 - r1;
              ++matches;
            }
          }
        }
      }
      total += cnt;
      if (total > VERIFY_CAP || matches >= 2) break;
    }
    if (total <= VERIFY_CAP) {
      *start_out = start;
      return matches;
    }
    matches = 0;
    start = -1;
  } else if (jhi - jlo < 8) {
    // a few positions (start / end chunks, short transcripts): verify each
    for (int j = jlo; j <= jhi && matches < 2; ++j) {
      if (verify(j)) {
        if (matches == 0) start = 2 * j + 1 - r1;
        ++matches;
      }
    }
    *start_out = start;
    return matches;
  }
  // many candidates (repetitive transcripts) or m < 3: the pattern in LDS and
  // every position checked in full by its own lane
  if (tc0) L.pc[i0] = g0;
  if (tc1) L.pc[i1] = g1;
  for (int base = jlo; base <= jhi && matches < 2; base += 64) {  // uniform trip count for the ballots
    const int j = base + lane;
    bool hit = j <= jhi;
    for (int i = 0; i < m && hit; ++i) hit = L.ytok[j + i] == L.pc[i];
    const uint64_t mask = __ballot(hit);
    if (mask && start < 0) start = 2 * __builtin_amdgcn_readlane(j, __builtin_ctzll(mask)) + 1 - r1;
    matches += __popcll(mask);
  }
  *start_out = start;
  return min(matches, 2);
}

// Greedy shortcut of one chunk (greedy_shortcuts, cu:30-153) for n <= 128
// frames and V <= 32: lane f of waves 0 and 1 holds frame a+f's row in x.
// Per frame the unique maximum over the transcript alphabet (cu:65-91):
// columns outside the alphabet (and past V) read as -inf, so they cannot win
// and only tie a -inf maximum, which rejects the chunk anyway; IEEE max ignores
// NaN exactly as the reference's strict '>' scan does, and the maximum is
// unique iff exactly one column equals it. Wave 0 then places the chunk while
// wave 1 computes the serial fp32 chunk objective (cu:135-137). Writes the
// labels and scores of an accepted chunk; *g / *fs return the lane's frame.
// Per-row maximum of a lane's row over the columns in `cols` (others -inf):
// the value, the number of columns equal to it and the last such column.
struct RowMax {
  float mx;
  int count, idx;  // idx is meaningful only when count == 1
};

__device__ __attribute__((always_inline)) inline RowMax row_max(const float (&x)[32], uint32_t cols) {
  float v[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) v[c] = (cols >> c) & 1u ? x[c] : NEG_INF;
  float t[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) t[c] = fmaxf(v[2 * c], v[2 * c + 1]);
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
    for (int c = 0; c < w; ++c) t[c] = fmaxf(t[2 * c], t[2 * c + 1]);
  // columns equal to the maximum as a bit mask: the count is its population,
  // the column of a unique maximum its only bit
  uint32_t eq = 0;
#pragma unroll
  for (int c = 0; c < 32; ++c) eq |= (uint32_t)(v[c] == t[0]) << c;
  return RowMax{t[0], (int)__popc(eq), 31 - (int)__clz(eq)};
}

// `whole`: row_max over all 32 register columns (columns past V hold -inf),
// computed before the transcript alphabet is known. When its maximum is unique and its column is
// in the alphabet, it is also the unique maximum over the alphabet (cu:53-58
// scan); any other lane of the wave has the alphabet-restricted maximum
// computed here.
__device__ __attribute__((always_inline)) int greedy_fast(const Lds& L, const float (&x)[32], RowMax whole, int n, int U, int S, int V, int blank,
                           uint32_t alpha32, bool blank_in, bool at_start, bool at_end, Slot& out, int* ambiguous,
                           int* g_lane, float* fs_lane) {
  Header* h = L.h;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int g = -2;
  float fs = -0.0f;  // identity of the fp32 sum for padding frames
  if (tid < 128) {
    const bool live = tid < n;
    const bool redo = live && !(whole.count == 1 && ((alpha32 >> whole.idx) & 1u));
    if (__ballot(redo) != 0) whole = row_max(x, alpha32);
    const float mx = whole.mx;
    const int count = whole.count, idx = whole.idx;
    const bool bad = live && (!isfinite(mx) || count != 1);
    if (live) { g = idx; fs = mx; }
    L.g[tid] = g;
    L.fs[tid] = fs;
    const uint64_t anybad = __ballot(bad);
    if (lane == 0) h->gbad[wave] = anybad != 0;
  }
  *g_lane = g;
  *fs_lane = fs;
  __syncthreads();
  *ambiguous = 0;
  if (h->gbad[0] | h->gbad[1]) return 0;  // a tie or a non-finite maximum: no shortcut
  int matches, start, rlast;
  float score;
  if (blank_in) {
    matches = place_literal(L, L.ytok, n, S, blank, at_start, at_end, &start, &rlast);
    if (tid == 0) h->fbuf[1] = serial_sum128(L.fs);
    __syncthreads();
    score = h->fbuf[1];
  } else {
    if (wave == 0) {
      const int m = place_wave(L, g, L.g[lane + 64], n, U, S, blank, at_start, at_end, V <= 32, &start, &rlast);
      if (lane == 0) { h->ibuf[3] = m; h->ibuf[4] = start; h->ibuf[6] = rlast; }
    } else if (wave == 1 && lane == 0) {
      h->fbuf[1] = serial_sum128(L.fs);  // padding frames add -0.0, an exact identity
    }
    __syncthreads();
    matches = h->ibuf[3];
    start = h->ibuf[4];
    rlast = h->ibuf[6];
    score = h->fbuf[1];
  }
  *ambiguous = matches > 1;
  if (matches != 1 || !isfinite(score)) return 0;  // cu:129-139
  out.start = start;
  out.end = start + rlast;
  out.objective = score;
  return 1;
}

// ---------------------------------------------------------------------------
// Kernels.

// The per-record outputs of optimized mode besides the path (thread 0).
__device__ inline void tail_outputs(const Params& p, int rec, const TailStats& ts, int status, float objective,
                                    int stitched) {
  glb(p.status)[rec] = status;
  glb(p.objective)[rec] = objective;
  glb(p.stitched)[rec] = stitched;
  glb(p.repair_passes)[rec] = ts.passes;
  glb(p.repaired_frames)[rec] = ts.repaired;
  glb(p.shortcut_stats)[3 * rec + 0] = ts.sc_accepted;
  glb(p.shortcut_stats)[3 * rec + 1] = ts.sc_frames;
  glb(p.shortcut_stats)[3 * rec + 2] = ts.sc_ambiguous;
  glb(p.routing_stats)[3 * rec + 0] = ts.early;
  glb(p.routing_stats)[3 * rec + 1] = ts.rejected;
  glb(p.routing_stats)[3 * rec + 2] = ts.maxprop;
  if (p.reuse_stats) {
    GLB int64_t* u = glb(p.reuse_stats) + 4 * rec;
    u[0] = ts.reuse[0]; u[1] = ts.reuse[1]; u[2] = ts.reuse[2]; u[3] = ts.reuse[3];
  }
}

// The per-record outputs of conventional mode besides the path.
__device__ inline void conventional_outputs(const Params& p, int rec, int status, float objective) {
  glb(p.status)[rec] = status;
  glb(p.objective)[rec] = objective;
  glb(p.stitched)[rec] = 0;
  glb(p.repair_passes)[rec] = 0;
  glb(p.repaired_frames)[rec] = 0;
  for (int q = 0; q < 3; ++q) { glb(p.shortcut_stats)[3 * rec + q] = 0; glb(p.routing_stats)[3 * rec + q] = 0; }
}

template <int K, int D, bool LG, class TB>
__global__ void __launch_bounds__(K == 32 ? 640 : 256) conventional_kernel(Params p, TB tab) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const Lds L = carve(lds_raw, p);
  const int rec = blockIdx.x;
  RecordDesc d;
  if constexpr (kArgs<TB>) d = tab.rec[rec];
  else d = load_pod(glb(p.desc) + rec);
  Rec r = make_rec(d, p, L);
  if (LG) r.st = p.stats + d.frame_offset;
  const Staged st = stage_tokens<ALPHABET_NONE>(d, p, rec, L);
  if (st.status >= 2) {
    if (threadIdx.x == 0) conventional_outputs(p, rec, st.status, NEG_INF);
    write_failed(r, 0, r.T);
    return;
  }
  const DPOut o = dp_interval<K, D, LG, false>(r, L, 0, r.T, true, nullptr, 1, nullptr, TRACE_IF_FINITE);
  const bool ok = isfinite(o.score);
  if (threadIdx.x == 0) conventional_outputs(p, rec, ok ? 0 : 1, o.score);  // cu:507-510
  if (!ok) write_failed(r, 0, r.T);
}

// ---------------------------------------------------------------------------
// Banded DP: conventional mode for batches with transcripts of more than 1,024
// states. A record's states are cut into bands of BAND_STATES, one wave each
// (BAND_K contiguous states per lane), and every band is a workgroup of its
// own, so a record of 18,001 states runs on 71 CUs instead of one. State s at
// frame t reads states s, s-1 and s-2 at frame t-1 (cu:438-444); a band's first
// state is even (a blank state, which no skip enters, cu:407), so all a band
// needs from outside is the previous band's last state at frame t-1. Band j
// publishes that value for every frame as one 8-byte entry of its edge array
// (the float and a valid tag, an agent-scope store written through to
// memory); band j+1 loads the entries a group of BAND_D frames ahead with
// agent-scope loads and checks each tag at use, so it runs a few frames behind
// band j. The
// edge arrays and control words are zeroed before each call (zero_kernel).
// Workgroups take their band from a ticket counter in the order they start,
// so band j-1 is running whenever band j waits for it and every wait ends;
// a wait is bounded all the same (BAND_SPIN_LIMIT polls of one entry, then
// the band waits no more and uses NaN, so a broken hand-off gives wrong
// results instead of a hang, and sets control word 1 in the workspace).
// Each band writes its lanes' part of every backpointer row (the layout of
// the one-workgroup DP: thread index band*64+lane with BAND_K states), then
// counts itself on the record's arrival counter with a release; the last band
// to arrive acquires, selects the terminal state (cu:497-500), walks the path
// (finish, cu:642-667) and writes the record's outputs.
//
// FB (optimized mode, split tail, the same transcripts): the early full
// fallback of records whose repair budget was exceeded (repair_recurrence,
// cu:535-550), launched after the tail's first planning pass. Bands of other
// records return at once. The DP resumes from chunk 0's frontier where it is
// stored (rows before it are chunk 0's), and the last band leaves the status,
// objective and reuse counts in the record's tail state with the fallback
// marked done; repair_kernel's continuation then writes the outputs.
constexpr int BAND_K = 4;  // states per lane (C3 conventional: 9.5 ms with K = 4, 10.9 ms with K = 8, same loop)
constexpr int BAND_STATES = 64 * BAND_K;
constexpr int BAND_D = 8;                 // frames per group of gathers and edge loads in flight (two groups; 16 measured the same)
constexpr int BAND_SPIN_LIMIT = 1 << 21;  // polls of one entry (about a second) before a band stops waiting
constexpr int BAND_CTL_HEAD = 64;         // control words: [0] ticket, [1] a wait ran out, [2] ticket of the fallback after
                                          // failed seams, then an arrival count per record

__device__ inline uint64_t edge_load(const GLB uint64_t* at) {
  return __hip_atomic_load((const uint64_t*)at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The previous band's value in entry `ent` (loaded ahead from `at`), polling
// the entry while its tag is unset. `late`: a wait of this band ran out.
__device__ inline float edge_value(uint64_t ent, const GLB uint64_t* at, int& late, int32_t* ctl) {
  uint32_t tag = __builtin_amdgcn_readfirstlane((uint32_t)(ent >> 32));
  uint32_t val = __builtin_amdgcn_readfirstlane((uint32_t)ent);
  if (tag != 1u) {
    if (!late) {
      for (int spins = 0; spins < BAND_SPIN_LIMIT; ++spins) {
        __builtin_amdgcn_s_sleep(8);
        const uint64_t again = edge_load(at);
        tag = __builtin_amdgcn_readfirstlane((uint32_t)(again >> 32));
        val = __builtin_amdgcn_readfirstlane((uint32_t)again);
        if (tag == 1u) break;
      }
    }
    if (tag != 1u) {
      if (!late && threadIdx.x == 0) __hip_atomic_store(ctl + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      late = 1;
      return __builtin_nanf("");
    }
  }
  return __uint_as_float(val);
}

template <class TB, int FB>
__global__ void __launch_bounds__(64) band_kernel(Params p, TB tab) {
  constexpr bool kTab = kArgs<TB> && FB == 0;  // optimized mode reads the descriptors the chunk kernel left
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const Lds L = carve(lds_raw, p);
  const int lane = threadIdx.x;
  int ticket = 0;
  if (lane == 0)  // the fallback after failed seams counts on its own ticket word
    ticket = __hip_atomic_fetch_add(p.band_ctl + (FB == 2 ? 2 : 0), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  ticket = __builtin_amdgcn_readlane(ticket, 0);
  // ticket -> (record, band): bands are numbered record by record
  int rec = -1, band = 0, bands = 1;
  for (int g = 0, base = 0; g < p.count; g += 64) {
    const int i = g + lane;
    int nb = 0;
    if (i < p.count) {
      int U;
      if constexpr (kTab) U = tab.rec[i].tokens;
      else U = glb(p.desc)[i].tokens;
      nb = (2 * U + 1 + BAND_STATES - 1) / BAND_STATES;
    }
    const int incl = wave_incl_scan(nb);
    const uint64_t hit = __ballot(i < p.count && ticket < base + incl);
    if (hit) {
      const int l = (int)__builtin_ctzll(hit);
      rec = g + l;
      bands = __builtin_amdgcn_readlane(nb, l);
      band = ticket - (base + __builtin_amdgcn_readlane(incl, l) - bands);
      break;
    }
    base += __builtin_amdgcn_readlane(incl, 63);
  }
  if (rec < 0) return;  // (the grid has one workgroup per band)
  RecordDesc d;
  if constexpr (kTab) d = tab.rec[rec];
  else d = load_pod(glb(p.desc) + rec);
  Rec r = make_rec(d, p, L);
  const int S = r.S;
  const int64_t T = r.T;
  int64_t f0 = 0;  // the DP's first column: frame 0, or chunk 0's frontier
  bool resume = false;
  int frontier_end = 0;
  if constexpr (FB != 0) {
    GLB TailState* state = glb(p.tstate) + rec;
    const int done = __builtin_amdgcn_readfirstlane(state->done);
    if constexpr (FB == 1) {
      const int early = __builtin_amdgcn_readfirstlane(state->ts.early);
      if (done || !(p.overlap && early == 1)) return;  // not an early fallback: nothing to do
      const Slot c0 = load_pod(glb(p.slots) + d.chunk_offset);
      frontier_end = __builtin_amdgcn_readfirstlane(c0.frontier_end);
    } else {
      if (done || !__builtin_amdgcn_readfirstlane(state->fallback)) return;  // stitched, or finished before
      frontier_end = __builtin_amdgcn_readfirstlane(state->fallback_from);
    }
    load_tokens(r, L.ytok);
    resume = r.frontier != nullptr && frontier_end > 0 && frontier_end <= T;
    if (resume) f0 = frontier_end - 1;
  } else {
    const Staged st = stage_tokens<ALPHABET_NONE>(d, p, rec, L);
    if (st.status >= 2) {  // every band sees the same status; the first writes the outputs (cu:642-652)
      if (band == 0) {
        if (lane == 0) conventional_outputs(p, rec, st.status, NEG_INF);
        write_failed(r, 0, T);
      }
      return;
    }
  }
  constexpr int K = BAND_K;
  const int s0 = band * BAND_STATES + lane * K;
  const int gtid = band * 64 + lane;
  const bool active = s0 < S;
  uint32_t lab[K];
  float skb[K];  // 0 where the skip transition is legal, -inf elsewhere (cu:407)
  float al[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int s = s0 + k;
    const int ls = s < S ? label_of(r, s) : r.blank;
    lab[k] = 4u * (uint32_t)ls;
    const bool ok = s >= 2 && s < S && ls != r.blank && ls != label_of(r, s - 2);
    skb[k] = ok ? 0.0f : NEG_INF;
  }
  const GLB float* e = r.e;
  const int64_t V = r.V;
  GLB uint32_t* bp = r.bp;
  const int64_t stride = r.stride;
  const bool has_next = band + 1 < bands;
  GLB uint64_t* edges = glb(p.edges) + d.frame_offset * (int64_t)p.band_stride;
  const GLB uint64_t* ein = band > 0 ? edges + (int64_t)(band - 1) * T : nullptr;
  GLB uint64_t* eout = edges + (int64_t)band * T;  // written only when has_next
  int32_t* ctl = p.band_ctl;
  if (resume) {  // alpha at frame f0 from chunk 0's frontier (cu:451-454)
    const GLB float* fr = r.frontier;
#pragma unroll
    for (int k = 0; k < K; ++k) al[k] = (s0 + k < S) ? fr[s0 + k] : NEG_INF;
  } else {  // frame 0 (cu:409-410)
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const float v = ldg_at(e, lab[k]);
      al[k] = (s0 + k < S && s0 + k < 2) ? v : NEG_INF;
    }
    if (active) store_row<K>(bp, gtid, 0u);
  }
  if (has_next && lane == 63)
    __hip_atomic_store((uint64_t*)(eout + f0), (uint64_t)__float_as_uint(al[K - 1]) | (1ull << 32),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int late = 0;
  // Backpointer bytes of this lane (K = 4: one byte per lane and frame),
  // advanced by one row per frame; lanes past S write into the sink, so the
  // frame has no exec-masked memory operations and the compiler's waits for
  // the gathers count the stores exactly.
  static_assert(K == 4, "one backpointer byte per lane");
  GLB uint8_t* bpb = active ? (GLB uint8_t*)(bp + (f0 + 1) * stride) + gtid : (GLB uint8_t*)glb(g_bp_sink) + lane;
  const int64_t bstep = active ? 4 * stride : 0;
  // one frame of the recurrence (cu:438-444); strict '>' keeps stay > advance > skip on ties
  auto frame = [&](int64_t t, const float (&evk)[K], float fill) {
    const float up1 = wave_shr1(al[K - 1], fill);
    uint32_t bits = 0;
#pragma unroll
    for (int k = K - 1; k >= 0; --k) {
      const float stay = al[k];
      const float adv = k >= 1 ? al[k - 1] : up1;
      const float skp = k >= 2 ? al[k - 2] : up1;
      float best = stay;
      uint32_t j = 0;
      if (adv > best) { best = adv; j = 1; }
      bool take = false;
      if ((k & 1) != 0) take = skp + skb[k] > best;  // even states are blank states: no skip into them
      if (take) { best = skp; j = 2; }
      al[k] = best + evk[k];
      bits |= j << (2 * k);
    }
    *bpb = (uint8_t)bits;
    bpb += bstep;
    if (has_next) {  // every lane stores the last state's value to the same entry
      const uint32_t v = (uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(al[K - 1]), 63);
      __hip_atomic_store((uint64_t*)(eout + t), (uint64_t)v | (1ull << 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };
  if (T > f0 + 1) {
    const int64_t last = T - 1;
    // the first band loads a control word instead (values unused): the loads are unconditional
    const GLB uint64_t* esrc = ein ? ein : reinterpret_cast<const GLB uint64_t*>(glb(ctl));
    // Two groups of BAND_D frames in flight: while one group's frames are
    // computed, the next group's gathers and edge entries load into the other
    // buffer. The loop body holds both groups, so no loaded value is carried
    // into the next iteration (a carried ring is copied between registers
    // there, and the copy waits for the newest loads and write-through stores).
    float ea[BAND_D][K], eb[BAND_D][K];
    uint64_t ga[BAND_D], gb[BAND_D];
    auto load = [&](float (&ev)[BAND_D][K], uint64_t (&eg)[BAND_D], int64_t tg) {
#pragma unroll
      for (int dd = 0; dd < BAND_D; ++dd) {
        const int64_t t = min(tg + dd, last);
        const GLB float* row = e + t * V;
#pragma unroll
        for (int k = 0; k < K; ++k) ev[dd][k] = ldg_at(row, lab[k]);
        eg[dd] = edge_load(esrc + (ein ? t - 1 : 0));
      }
    };
    auto run = [&](const float (&ev)[BAND_D][K], const uint64_t (&eg)[BAND_D], int64_t tg, bool whole) {
#pragma unroll
      for (int dd = 0; dd < BAND_D; ++dd)
        if (whole || tg + dd < T)
          frame(tg + dd, ev[dd], ein ? edge_value(eg[dd], ein + tg + dd - 1, late, ctl) : NEG_INF);
    };
    int64_t tg = f0 + 1;
    load(ea, ga, tg);
    for (;;) {
      if (tg + BAND_D > T) { run(ea, ga, tg, false); break; }
      load(eb, gb, tg + BAND_D);
      run(ea, ga, tg, true);
      tg += BAND_D;
      if (tg + BAND_D > T) { run(eb, gb, tg, false); break; }
      load(ea, ga, tg + BAND_D);
      run(eb, gb, tg, true);
      tg += BAND_D;
    }
  }
  // the terminal candidates S-1 and S-2 (cu:497-500), from whichever band holds them
  GLB float* term = reinterpret_cast<GLB float*>(glb(ctl) + BAND_CTL_HEAD + p.count) + 2 * (int64_t)rec;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int s = s0 + k;
    if (s == S - 1) __hip_atomic_store((float*)term + 1, al[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (S > 1 && s == S - 2) __hip_atomic_store((float*)term, al[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  wait_stores();  // this band's rows and values are complete before its release
  int last_band = 0;
  if (lane == 0)
    last_band = __hip_atomic_fetch_add(ctl + BAND_CTL_HEAD + rec, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) ==
                bands - 1;
  if (!__builtin_amdgcn_readlane(last_band, 0)) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  const float v1 = __hip_atomic_load((float*)term + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const float v0 = S > 1 ? __hip_atomic_load((float*)term, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : NEG_INF;
  int terminal = S - 1;
  float score = v1;
  if (S > 1 && v0 >= v1) { terminal = S - 2; score = v0; }
  const bool ok = isfinite(score);
  if (ok) (void)trace_path(r, 0, T, terminal);
  if constexpr (FB == 2) {  // fallback_recurrence after failed seams (cu:552-559): the record's outputs
    if (!ok) write_failed(r, 0, T);
    if (lane == 0) {
      TailStats ts = load_pod(&glb(p.tstate)[rec].ts);
      if (resume && (d.flags & DESC_REUSE_COUNTED)) { ts.reuse[1] += frontier_end; ts.reuse[3] += S; }
      tail_outputs(p, rec, ts, ok ? 0 : 1, score, 0);
    }
  } else if constexpr (FB == 1) {  // the tail's continuation writes the outputs (TAIL_RESUME)
    if (lane == 0) {
      GLB TailState* state = glb(p.tstate) + rec;
      state->status = ok ? 0 : 1;
      state->objective = score;
      state->ts.early = 2;
      if (resume && (d.flags & DESC_REUSE_COUNTED)) {
        unsigned long long* reuse = reinterpret_cast<unsigned long long*>(p.tstate[rec].ts.reuse);
        atomicAdd(reuse + 1, (unsigned long long)frontier_end);
        atomicAdd(reuse + 3, (unsigned long long)S);
      }
    }
  } else {
    if (lane == 0) conventional_outputs(p, rec, ok ? 0 : 1, score);  // cu:507-510
    if (!ok) write_failed(r, 0, T);
  }
}

// Zeroes n 16-byte words (the banded DP's control words and edge arrays).
__global__ void __launch_bounds__(256) zero_kernel(v4i_t* dst, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    glb(dst)[i] = v4i_t{0, 0, 0, 0};
}

// XCD-aware placement: workgroup i runs on XCD i % 8, so consecutive slots of
// one record (which share its targets) are mapped to the same XCD's L2.
__device__ inline int xcd_slot(int bid, int total) {
  const int per = (total + 7) / 8;
  return (bid % 8) * per + bid / 8;
}

// A chunk slot, from LDS or from global memory (the tail's two slot arrays).
__device__ inline Slot load_slot(const Slot* x) { return *x; }
__device__ inline Slot load_slot(const GLB Slot* x) { return load_pod(x); }

// A value every lane of the wave holds alike, moved word by word into scalar
// registers (function arguments arrive in vector registers).
template <class T>
__device__ inline T uniform(const T& x) {
  static_assert(sizeof(T) % 4 == 0, "32-bit words");
  int w[sizeof(T) / 4];
  __builtin_memcpy(w, &x, sizeof(T));
#pragma unroll
  for (size_t i = 0; i < sizeof(T) / 4; ++i) w[i] = __builtin_amdgcn_readfirstlane(w[i]);
  T out;
  __builtin_memcpy(&out, w, sizeof(T));
  return out;
}

// The chunk, repair and fallback DPs of the optimized-mode kernels. For K = 32
// (transcripts of more than 8,192 states) they run in a function of their
// own: the chunk kernel's greedy code and the tail's repair bookkeeping then
// cost no registers inside the frame loop, which gets the conventional
// kernel's loop form and register budget (inlined into the tail, the K = 32
// frame loop spilled 12 to 30 registers per frame). The record view and the
// interval arrive as arguments, in vector registers; they are moved into
// scalar registers at entry, and the LDS view is rebuilt from the kernel's
// dynamic shared memory (not passed in), so that its pointers stay LDS
// pointers to the compiler.
template <int K, int D, bool LG>
__device__ __attribute__((noinline)) DPOut dp_k32(const Rec& rv, LdsShape shape, int64_t a, int64_t b,
                                                   bool record_end, const GLB float* resume_from, int64_t start_t,
                                                   GLB float* save_frontier, int trace) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const Lds L = carve(lds_raw, uniform(shape));
  Rec r = uniform(rv);
  r.ytok = L.ytok;  // the record's staged targets (the same LDS array, typed as LDS)
  return dp_interval<K, D, LG, false>(r, L, uniform(a), uniform(b), uniform((int)record_end) != 0,
                                      uniform(resume_from), uniform(start_t), uniform(save_frontier),
                                      uniform(trace));
}

template <int K, int D, bool LG>
__device__ __attribute__((always_inline)) DPOut run_dp(const Params& p, const Rec& r, const Lds& L, int64_t a,
                                                        int64_t b, bool record_end, const GLB float* resume_from,
                                                        int64_t start_t, GLB float* save_frontier, int trace) {
  if constexpr (K == 32)
    return dp_k32<K, D, LG>(r, lds_shape(p), a, b, record_end, resume_from, start_t, save_frontier, trace);
  else
    return dp_interval<K, D, LG>(r, L, a, b, record_end, resume_from, start_t, save_frontier, trace);
}

// The tail of one record; SP is the slot array, in LDS or in global memory.
// With phase TAIL_ALL it runs every repair round's DPs itself, one interval
// after another. In the split tail, TAIL_PLAN0 plans the first round and
// leaves its DPs to repair_kernel; TAIL_RESUME (in repair_kernel, once the
// record's first-round DPs are done) runs the later rounds and the seam check.
// The record's state lives in p.tstate between the two.
template <int K, int D, bool LG, class SP>
__device__ __attribute__((always_inline)) void tail_body(const Params& p, const RecordDesc& d, int rec, const Rec& r,
                                                      const Lds& L, SP sl, bool in_lds, int phase) {
  Header* h = L.h;
  const int tid = threadIdx.x;
  const int64_t T = r.T;
  const int n = (int)(1 + (T - 1) / p.H);
  const bool split = phase != TAIL_ALL;
  GLB TailState* state = p.tstate ? glb(p.tstate) + rec : nullptr;  // split tail, or banded fallbacks
  const int status0 = sl[0].status;
  if (status0 >= 2 && (!split || phase == TAIL_PLAN0)) {
    if (tid == 0) {
      glb(p.status)[rec] = status0;
      glb(p.objective)[rec] = NEG_INF;
      glb(p.stitched)[rec] = 0;
      glb(p.repair_passes)[rec] = 0;
      glb(p.repaired_frames)[rec] = 0;
      for (int q = 0; q < 3; ++q) { glb(p.shortcut_stats)[3 * rec + q] = 0; glb(p.routing_stats)[3 * rec + q] = 0; }
      if (p.reuse_stats)
        for (int q = 0; q < 4; ++q) glb(p.reuse_stats)[4 * rec + q] = 0;
      if (split) state->done = 1;
    }
    return;
  }
  load_tokens(r, L.ytok);
  const int S = r.S;
  const bool frontier_on = r.frontier != nullptr;  // frontiers are saved and resumed
  const bool counted = frontier_on && (d.flags & DESC_REUSE_COUNTED);  // and show in reuse_stats
  // Fast path (records of at most 64 chunks, slots in LDS): when every chunk
  // objective is finite and every seam is legal, the repair rounds merge
  // nothing (plan_repairs joins every neighbour and its budget preflight
  // proposes no region) and validate_seams stitches iff the fp32 total is
  // finite. Wave 0 checks all seams at once and writes the result.
  if (n <= 64 && in_lds && (!split || phase == TAIL_PLAN0)) {
    if (tid < 64) {
      const int k = tid;
      const bool valid = k < n;
      const Slot sk = load_slot(sl + (valid ? k : 0));
      const int end_prev = (valid && k > 0) ? sl[k - 1].end : 0;
      const bool ok = !valid || (isfinite(sk.objective) && (k == 0 || legal_seam(r, sk.start, end_prev)));
      int done = 0;
      if (__ballot(!ok) == 0) {
        float total = 0.0f;  // cu:578-584: chunk objectives summed in chunk order
        for (int i = 0; i < n; ++i) total += readlane_f(sk.objective, i);
        if (isfinite(total)) {
          done = 1;
          const uint64_t shortcut = __ballot(valid && sk.kind == 1);
          const uint64_t amb = __ballot(valid && sk.kind == 2);
          const uint64_t dp = __ballot(valid && sk.kind != 1);
          int frames = valid && sk.kind == 1 ? sk.b - sk.a : 0;
#pragma unroll
          for (int off = 32; off > 0; off >>= 1) frames += __shfl_xor(frames, off, 64);
          if (tid == 0) {
            glb(p.status)[rec] = 0;
            glb(p.objective)[rec] = total;
            glb(p.stitched)[rec] = 1;
            glb(p.repair_passes)[rec] = 0;
            glb(p.repaired_frames)[rec] = 0;
            glb(p.shortcut_stats)[3 * rec + 0] = __popcll(shortcut);
            glb(p.shortcut_stats)[3 * rec + 1] = frames;
            glb(p.shortcut_stats)[3 * rec + 2] = __popcll(amb);
            for (int q = 0; q < 3; ++q) glb(p.routing_stats)[3 * rec + q] = 0;
            if (p.reuse_stats) {
              GLB int64_t* u = glb(p.reuse_stats) + 4 * rec;
              u[0] = 0; u[1] = 0; u[2] = counted ? (int64_t)__popcll(dp) * S : 0; u[3] = 0;
            }
            if (split) state->done = 1;
          }
        }
      }
      if (tid == 0) h->ibuf[6] = done;
    }
    __syncthreads();
    if (h->ibuf[6]) return;
    __syncthreads();
  }
  TailStats& ts = h->ts;  // written by thread 0 only
  int early = 0;  // uniform copy of ts.early
  int status = 0;
  float objective = NEG_INF;
  if (!split || phase == TAIL_PLAN0) {
    if (tid == 0) {  // shortcut_stats (cu:129-133, 140-146) and frontier writes of the chunk DPs
      ts = TailStats{};
      for (int k = 0; k < n; ++k) {
        if (sl[k].kind == 1) { ++ts.sc_accepted; ts.sc_frames += sl[k].b - sl[k].a; }
        else {
          if (sl[k].kind == 2) ++ts.sc_ambiguous;
          if (counted) ts.reuse[2] += S;
        }
      }
    }
  } else {  // a later phase: the state the previous phases left
    if (tid == 0) {
      ts = load_pod(&state->ts);
      h->ibuf[5] = ts.early;
      h->ibuf[7] = state->status;
      h->fbuf[3] = state->objective;
    }
    __syncthreads();
    early = h->ibuf[5];
    status = h->ibuf[7];
    objective = h->fbuf[3];
    __syncthreads();
  }
  const bool repairs = p.repair_rounds > 0;
  const int first_round = phase == TAIL_RESUME ? 1 : 0;
  const int end_round = phase == TAIL_PLAN0 ? 1 : p.repair_rounds;
  for (int round = first_round; round < end_round; ++round) {
    if (tid == 0) {  // plan_repairs, cu:164-228
      early = ts.early;
      int run = !(p.overlap && early == 2);
      if (run && p.budget > 0 && T >= p.repair_min) {
        int before = -1;
        int64_t begin = 0, maximum = 0;
        bool reject = false;
        for (int k = 0; k < n; ++k) {
          sl[k].flag = 0;
          if (sl[k].a >= sl[k].b) continue;
          const bool join = before < 0 || (isfinite(sl[k].objective) && isfinite(sl[before].objective) &&
                                           legal_seam(r, sl[k].start, sl[before].end));
          if (join) begin = sl[k].a;
          else {
            maximum = max(maximum, (int64_t)sl[k].b - begin);
            if (maximum > p.budget) reject = true;
          }
          before = k;
        }
        if (reject) {
          ++ts.rejected;
          ts.maxprop = max(ts.maxprop, (int)maximum);
          if (p.overlap) early = 1;
          run = 0;
        }
      }
      if (run) {
        int previous = -1, group = -1;
        bool merged = false;
        for (int k = 0; k < n; ++k) {
          if (sl[k].a >= sl[k].b) continue;
          sl[k].flag = 0;
          const bool join = previous < 0 || (isfinite(sl[k].objective) && isfinite(sl[previous].objective) &&
                                             legal_seam(r, sl[k].start, sl[previous].end));
          if (join) group = k;
          else {
            sl[group].b = sl[k].b;
            sl[group].flag = 1;
            sl[k].b = sl[k].a;
            merged = true;
          }
          previous = k;
        }
        if (merged) {
          ++ts.passes;
          for (int k = 0; k < n; ++k)
            if (sl[k].flag) ts.repaired += sl[k].b - sl[k].a;
        }
      }
      ts.early = early;
      h->ibuf[5] = early;
    }
    __syncthreads();
    early = h->ibuf[5];
    __syncthreads();
    if (phase == TAIL_PLAN0) break;  // the first round's DPs run in repair_kernel
    if (p.overlap && early) {
      if (early == 1) {  // early full fallback (repair_recurrence, cu:535-550)
        const Slot s0 = load_slot(sl + (0));
        const bool resume = frontier_on && s0.frontier_end > 0 && s0.frontier_end <= T;
        if (resume && counted && tid == 0) { ts.reuse[1] += s0.frontier_end; ts.reuse[3] += S; }
        const DPOut o = run_dp<K, D, LG>(p, r, L, 0, T, true, resume ? r.frontier : nullptr,
                                          resume ? s0.frontier_end : 1, nullptr, TRACE_IF_FINITE);
        status = isfinite(o.score) ? 0 : 1;
        objective = o.score;
        early = 2;
        if (tid == 0) { ts.early = early; h->ibuf[5] = early; }
        __syncthreads();
      }
    } else {
      for (int k = 0; k < n; ++k) {  // repair DP over merged intervals (cu:727-760)
        const Slot s = load_slot(sl + (k));
        if (s.a >= s.b || (repairs && !s.flag)) continue;
        bool resume = false;
        int64_t start_t = s.a + 1;
        GLB float* fr = frontier_on ? r.frontier + (int64_t)k * S : nullptr;
        if (frontier_on) {
          if (s.frontier_end > s.a && s.frontier_end <= s.b) {
            resume = true;
            start_t = s.frontier_end;
            if (tid == 0 && counted) { ts.reuse[0] += s.frontier_end - s.a; ts.reuse[3] += S; }
          }
          if (tid == 0 && counted) ts.reuse[2] += S;
        }
        const DPOut o = run_dp<K, D, LG>(p, r, L, s.a, s.b, s.b == T, resume ? fr : nullptr, start_t, fr,
                                          TRACE_ALWAYS);
        if (tid == 0) {
          sl[k].objective = o.score;
          sl[k].end = o.terminal;
          sl[k].start = o.start;
          if (frontier_on) sl[k].frontier_end = s.b;
        }
        __syncthreads();
      }
    }
  }
  if (phase == TAIL_PLAN0) {  // hand the planned round to repair_kernel
    if (in_lds) {
      GLB Slot* gs = glb(p.slots) + d.chunk_offset;
      for (int k = tid; k < n; k += blockDim.x) store_pod(gs + k, load_slot(sl + k));
    }
    if (tid == 0) {
      int work = p.overlap && early == 1 ? 1 : 0;  // the early full fallback
      if (!(p.overlap && early))
        for (int k = 0; k < n; ++k) work += sl[k].a < sl[k].b && sl[k].flag;
      store_pod(&state->ts, ts);
      state->done = 0;
      state->fallback = 0;
      state->status = 0;
      state->objective = NEG_INF;
      state->work = work;
      state->pending = work;
    }
    return;
  }
  int stitched = 0;
  if (!(p.overlap && early == 2)) {  // validate_seams, cu:562-592
    if (tid == 0) {
      bool legal = true;
      float total = 0.0f;
      int previous = -1;
      if (!repairs) { ts.passes = 0; ts.repaired = 0; }
      for (int k = 0; k < n; ++k) {
        if (repairs && sl[k].a >= sl[k].b) continue;
        const float cost = sl[k].objective;
        legal = legal && isfinite(cost);
        total += cost;
        if (previous >= 0) legal = legal && legal_seam(r, sl[k].start, sl[previous].end);
        previous = k;
      }
      legal = legal && isfinite(total);
      h->ibuf[6] = legal ? 1 : 0;
      h->fbuf[2] = total;
    }
    __syncthreads();
    stitched = h->ibuf[6];
    status = 0;
    objective = h->fbuf[2];
    __syncthreads();
    if (!stitched && p.band_ctl && state) {  // banded: band_kernel<.., 2> runs it and writes the outputs
      if (tid == 0) {
        store_pod(&state->ts, ts);
        state->fallback_from = load_slot(sl + (0)).frontier_end;
        state->fallback = 1;
      }
      return;
    }
    if (!stitched) {  // fallback_recurrence, cu:552-559
      const Slot s0 = load_slot(sl + (0));
      const bool resume = frontier_on && s0.frontier_end > 0 && s0.frontier_end <= T;
      if (resume && counted && tid == 0) { ts.reuse[1] += s0.frontier_end; ts.reuse[3] += S; }
      const DPOut o = run_dp<K, D, LG>(p, r, L, 0, T, true, resume ? r.frontier : nullptr,
                                        resume ? s0.frontier_end : 1, nullptr, TRACE_IF_FINITE);
      status = isfinite(o.score) ? 0 : 1;
      objective = o.score;
    }
  }
  if (status != 0) write_failed(r, 0, T);
  if (tid == 0) tail_outputs(p, rec, ts, status, objective, stitched);
}

// Fast path of one record's tail in wave 0 (tid < 64, n <= 64 chunks): a
// rejected record, or every seam legal and a finite total, writes the record's
// outputs. Returns 1 when the record is finished. AG: the slots are read with
// agent-scope loads (fused tail: written by workgroups of the same kernel).
template <bool AG>
__device__ __attribute__((always_inline)) int tail_fast(const Params& p, const RecordDesc& d, int rec, const GLB Slot* gs,
                                                        int n) {
  const int k = threadIdx.x;
  const bool valid = k < n;
  const Slot sk = AG ? load_pod_agent(gs + (valid ? k : 0)) : load_pod(gs + (valid ? k : 0));
  const int status0 = __builtin_amdgcn_readfirstlane(sk.status);
  const int S = 2 * d.tokens + 1;
  const bool counted = d.frontier_offset >= 0 && (d.flags & DESC_REUSE_COUNTED);
  int done = 0;
  if (status0 >= 2) {  // rejected record: every chunk wrote -1 / -inf
    done = 1;
    if (k == 0) {
      glb(p.status)[rec] = status0;
      glb(p.objective)[rec] = NEG_INF;
      glb(p.stitched)[rec] = 0;
      glb(p.repair_passes)[rec] = 0;
      glb(p.repaired_frames)[rec] = 0;
      for (int q = 0; q < 3; ++q) { glb(p.shortcut_stats)[3 * rec + q] = 0; glb(p.routing_stats)[3 * rec + q] = 0; }
      if (p.reuse_stats)
        for (int q = 0; q < 4; ++q) glb(p.reuse_stats)[4 * rec + q] = 0;
    }
  } else {
    const int end_prev = wave_shr1_int(sk.end, 0);
    bool ok = !valid || isfinite(sk.objective);
    if (valid && k > 0) {  // legal_seam, cu:157-161
      const int jump = sk.start - end_prev;
      ok = ok && (jump == 0 || jump == 1 || (jump == 2 && sk.skip_ok));
    }
    if (__ballot(!ok) == 0) {
      float total = 0.0f;  // cu:578-584: chunk objectives summed in chunk order
      for (int i = 0; i < n; ++i) total += readlane_f(sk.objective, i);
      if (isfinite(total)) {
        done = 1;
        const uint64_t shortcut = __ballot(valid && sk.kind == 1);
        const uint64_t amb = __ballot(valid && sk.kind == 2);
        const uint64_t dp = __ballot(valid && sk.kind != 1);
        // shortcut frames: H per shortcut chunk, the last chunk's own length for it
        const uint64_t last_bit = 1ull << (n - 1);
        const int64_t frames = (int64_t)p.H * __popcll(shortcut & ~last_bit) +
                               ((shortcut & last_bit) ? (int64_t)d.frames - (int64_t)(n - 1) * p.H : 0);
        if (k == 0) {
          glb(p.status)[rec] = 0;
          glb(p.objective)[rec] = total;
          glb(p.stitched)[rec] = 1;
          glb(p.repair_passes)[rec] = 0;
          glb(p.repaired_frames)[rec] = 0;
          glb(p.shortcut_stats)[3 * rec + 0] = __popcll(shortcut);
          glb(p.shortcut_stats)[3 * rec + 1] = frames;
          glb(p.shortcut_stats)[3 * rec + 2] = __popcll(amb);
          for (int q = 0; q < 3; ++q) glb(p.routing_stats)[3 * rec + q] = 0;
          if (p.reuse_stats) {
            GLB int64_t* u = glb(p.reuse_stats) + 4 * rec;
            u[0] = 0; u[1] = 0; u[2] = counted ? (int64_t)__popcll(dp) * S : 0; u[3] = 0;
          }
        }
      }
    }
  }
  return done;
}

// The rest of one record's tail (every thread of the workgroup): its slots
// into LDS when they fit, then tail_body.
template <int K, int D, bool LG>
__device__ __attribute__((always_inline)) void tail_rest(const Params& p, const RecordDesc& d, int rec, const Lds& L,
                                                         int phase) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const int tid = threadIdx.x;
  const int n = (int)(1 + (d.frames - 1) / p.H);
  GLB Slot* gs = glb(p.slots) + d.chunk_offset;
  Rec r = make_rec(d, p, L);
  if (LG) r.st = p.stats + d.frame_offset;
  if (n <= p.lds_tail_slots) {
    Slot* ls = reinterpret_cast<Slot*>(lds_raw + ((uintptr_t)L.tslots - (uintptr_t)lds_raw));
    for (int k = tid; k < n; k += blockDim.x) ls[k] = load_pod(gs + k);
    __syncthreads();
    tail_body<K, D, LG>(p, d, rec, r, L, ls, true, phase);
  } else {
    tail_body<K, D, LG>(p, d, rec, r, L, gs, false, phase);
  }
}

// Optimized mode, one workgroup per chunk of H frames (XCD-aware order): it
// stages and validates the record's targets, takes the greedy shortcut
// (cu:30-153) or runs the relaxed chunk DP (cu:721-726), and writes the
// chunk's labels, scores and slot.
//
// FUSE (fused tail): the record's last chunk workgroup to finish, on whichever
// XCD it runs, then runs the record's tail (tail_kernel's work) itself, so a
// call needs one launch. Hand-off: a chunk that took the greedy shortcut (or
// was rejected) writes its labels, scores and slot with agent-scope stores
// and waits for their completion; a chunk that ran a DP wrote backpointers,
// frontiers and its path with ordinary stores and releases them at agent
// scope (thread 0's release-ordered count: one L2 write-back, which only the
// rarer DP chunks pay). Every wave first waits for its own stores. Then one
// arrival on the record's counter; the last one zeroes it for the next call.
// The tail's fast path reads the slots with agent-scope loads; the full tail
// first acquires at agent scope.
template <int K, int D, bool LG, class TB, bool FUSE>
__global__ void __launch_bounds__(K == 32 ? 640 : 256) chunk_kernel(Params p, TB tab) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const Lds L = carve(lds_raw, p);
  const int tid = threadIdx.x;
  const int slot_index = xcd_slot(blockIdx.x, p.total_slots);
  if (slot_index >= p.total_slots) return;
  int rec, n, U;
  int64_t chunk;
  bool fast;
  int quads;  // V / 4 (fast path)
  const GLB int64_t* y;
  RecordDesc d;
  TargetLoads tl;
  if constexpr (kArgs<TB>) {
    // Table in the kernel arguments: lane i of every wave reads the first 32
    // bytes of record i's descriptor (the batch has at most 64 records); the
    // record is the last one whose first chunk is at or before this one.
    const int lane = tid & 63;
    const bool mine = lane < p.count;
    const RecordDesc& lr = tab.rec[mine ? lane : 0];
    const v4i_t h0 = *reinterpret_cast<const v4i_t*>(&lr.emissions);
    const v4i_t h1 = *reinterpret_cast<const v4i_t*>(&lr.frames);
    const uint64_t below = __ballot(mine && h1[1] <= slot_index);
    rec = 63 - (int)__builtin_clzll(below);
    const int e_lo = __builtin_amdgcn_readlane(h0[0], rec), e_hi = __builtin_amdgcn_readlane(h0[1], rec);
    const int y_lo = __builtin_amdgcn_readlane(h0[2], rec), y_hi = __builtin_amdgcn_readlane(h0[3], rec);
    d.emissions = reinterpret_cast<const float*>((uint64_t)(uint32_t)e_lo | (uint64_t)(uint32_t)e_hi << 32);
    d.targets = reinterpret_cast<const int64_t*>((uint64_t)(uint32_t)y_lo | (uint64_t)(uint32_t)y_hi << 32);
    d.frames = __builtin_amdgcn_readlane(h1[0], rec);
    d.chunk_offset = __builtin_amdgcn_readlane(h1[1], rec);
    d.vocab = __builtin_amdgcn_readlane(h1[2], rec);
    d.tokens = __builtin_amdgcn_readlane(h1[3], rec);
    chunk = slot_index - d.chunk_offset;
    n = (int)min((int64_t)p.H, (int64_t)d.frames - chunk * p.H);
    U = d.tokens;
    y = glb(d.targets);
    fast = p.mode == 2 && p.H <= 128 && d.vocab <= 32 && (d.vocab & 3) == 0 &&
           (reinterpret_cast<uintptr_t>(d.emissions) & 15) == 0;
    quads = d.vocab >> 2;
    tl = issue_targets(y, U, p);
    const RecordDesc& rd = tab.rec[rec];  // the other half: uniform loads
    d.frame_offset = rd.frame_offset;
    d.bp_offset = rd.bp_offset;
    d.frontier_offset = rd.frontier_offset;
    d.blank = rd.blank;
    d.flags = rd.flags;
  } else {
    const ChunkEntry ce = load_uniform(p.chunks + slot_index);
    rec = (int)(ce.hi & 0xffffu);
    n = (int)((ce.hi >> 16) & 0x1ffu) + 1;
    chunk = (int64_t)(ce.hi >> 25);
    fast = ((ce.lo >> ENTRY_FAST_SHIFT) & 1u) != 0;
    quads = (int)((ce.lo >> ENTRY_QUADS_SHIFT) & 7u) + 1;
    U = (int)((ce.lo >> ENTRY_U_SHIFT) & 0x3fffu);
    y = (const GLB int64_t*)((ce.lo & ((1ull << ENTRY_U_SHIFT) - 1)) << 3);
    // The record descriptor and the first batch of targets are requested
    // together (the entry holds the targets' address and count).
    const Pending<RecordDesc> pd = issue_uniform(p.desc + rec);
    tl = issue_targets(y, U, p);
    d = finish_uniform(pd);
  }
  const int64_t a = chunk * p.H;
  const int64_t b = a + n;
  // The chunk's rows (fast path: lane f of waves 0-1 loads row a+f). Every
  // thread issues the same eight 16-byte loads: the row's quads (the chunk's
  // last row for lanes past it), then -inf for quads past V (chunks off the
  // fast path read the 64-byte -inf constant block instead; values unused).
  // With a fixed count the compiler's waits for the targets in the staging
  // below count these loads exactly instead of waiting for them. Lanes past
  // the chunk's rows hit lines already requested by lane n-1: no extra HBM
  // traffic.
  float x[32];
  {
    const GLB v4f_t* pad = (const GLB v4f_t*)glb(kNegInfQuad);
    const GLB v4f_t* src = fast ? (const GLB v4f_t*)glb(d.emissions + (a + min(tid, n - 1)) * (int64_t)d.vocab) : pad;
    const int qmax = fast ? quads - 1 : 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const v4f_t v = *(q <= qmax ? src + (fast ? q : 0) : pad);
      x[4 * q] = v.x; x[4 * q + 1] = v.y; x[4 * q + 2] = v.z; x[4 * q + 3] = v.w;
    }
  }
  // the tail kernel reads the record's descriptor from the workspace (stored
  // after the row loads are issued, so the waits for the targets do not count it)
  if constexpr (kArgs<TB> && !FUSE)
    if (chunk == 0 && tid == 0) store_pod(glb(const_cast<RecordDesc*>(p.desc)) + rec, d);
  const Staged st = fast ? finish_targets<ALPHABET_MASK32, true, true>(tl, d.vocab, d.blank, d.frames, rec, p, L)
                   : p.mode == 2 ? finish_targets<ALPHABET_BITMAP, false, true>(tl, d.vocab, d.blank, d.frames, rec, p, L)
                                 : finish_targets<ALPHABET_NONE, false, true>(tl, d.vocab, d.blank, d.frames, rec, p, L);
  float2 row_st = make_float2(0.0f, 0.0f);
  RowMax whole{NEG_INF, 0, -1};
  if (fast && tid < 128) {
    if (LG && tid < n) {  // logits: each lane normalizes its own row in registers
      row_st = lane_row_stats(x, 4 * quads);
#pragma unroll
      for (int c = 0; c < 32; ++c)
        if (c < 4 * quads) x[c] = lsm(x[c], row_st);
      L.st[tid] = row_st;
    }
    if (p.mode == 2) whole = row_max(x, 0xffffffffu);
  }
  // (L.st is complete before any DP of this chunk reads it: greedy_fast's
  // barrier comes first)
  if (LG) {  // the tail kernel's DP reads the statistics from global memory
    if (fast) {
      if (tid < n) store_stats(glb(p.stats) + d.frame_offset + a + tid, row_st);
    } else if (st.status < 2) {
      rows_stats(glb(d.emissions) + a * (int64_t)d.vocab, n, d.vocab, L.st, glb(p.stats) + d.frame_offset + a);
      __syncthreads();
    }
  }
  Slot out{};
  bool ran_dp = false;
  out.a = (int)a;
  out.b = (int)b;
  out.flag = 1;
  out.objective = NEG_INF;
  GLB int64_t* labels = glb(p.labels) + d.frame_offset + a;
  GLB float* scores = glb(p.scores) + d.frame_offset + a;
  if (st.status >= 2) {  // rejected before any label-indexed read (cu:36, cu:642-652)
    for (int f = tid; f < n; f += blockDim.x) { put<FUSE>(labels + f, (int64_t)-1); put<FUSE>(scores + f, NEG_INF); }
    out.flag = 0;
    out.status = (int16_t)st.status;
  } else {
    int accepted = 0, ambiguous = 0;
    if (p.mode == 2 && fast) {
      int g;
      float fs;
      accepted = greedy_fast(L, x, whole, n, d.tokens, 2 * d.tokens + 1, d.vocab, d.blank, st.alpha32, st.blank_in,
                             a == 0, b == d.frames, out, &ambiguous, &g, &fs);
      if (accepted && tid < n) {  // finish's label/score gather collapses to g and fs (cu:642-667)
        put<FUSE>(labels + tid, (int64_t)g);
        put<FUSE>(scores + tid, fs);
      }
    }
    if (!accepted) {
      Rec r = make_rec(d, p, L);
      if (LG) { r.st = L.st; r.st_first = a; }
      if (p.mode == 2 && !fast) accepted = greedy_chunk<FUSE>(r, L, a, b, st.blank_in, out, &ambiguous);
      if (!accepted) {  // initial chunk DP (cu:721-726), relaxed init for a > 0
        ran_dp = true;
        GLB float* fr = r.frontier ? r.frontier + chunk * r.S : nullptr;
        const DPOut o = run_dp<K, D, LG>(p, r, L, a, b, b == r.T, nullptr, a + 1, fr, TRACE_ALWAYS);
        out.objective = o.score;
        out.end = o.terminal;
        out.start = o.start;
        out.frontier_end = r.frontier ? (int)b : 0;
      }
    }
    out.kind = (int16_t)(accepted ? 1 : (ambiguous ? 2 : 0));
    const int s0 = out.start;  // skip rule at the chunk's start state (cu:157-161), for the tail's seam check
    if (s0 >= 2) {
      const int l0 = (s0 & 1) ? (int)L.ytok[s0 >> 1] : d.blank;
      const int l2 = (s0 & 1) ? (int)L.ytok[(s0 - 2) >> 1] : d.blank;
      out.skip_ok = (int16_t)(l0 != d.blank && l0 != l2);
    }
  }
  if constexpr (!FUSE) {
    if (tid == 0) store_pod(glb(p.slots) + slot_index, out);
  } else {
    Header* h = L.h;
    const int chunks = (int)(1 + (d.frames - 1) / p.H);
    if (tid == 0) store_pod_agent(glb(p.slots) + slot_index, out);
    wait_stores();  // every wave's stores are complete (in this XCD's L2, or written through) ...
    __syncthreads();  // ... before thread 0 counts; for a DP chunk its count is a release (one L2 write-back)
    if (tid == 0) {
      int32_t* counter = p.arrivals + rec * ARRIVAL_STRIDE;
      const int old = ran_dp ? __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT)
                             : __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = old == chunks - 1;
      if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      h->arrived = last;
    }
    __syncthreads();
    if (!h->arrived) return;
    if (chunks <= 64) {
      if (tid < 64) {
        const int done = tail_fast<true>(p, d, rec, glb(p.slots) + d.chunk_offset, chunks);
        if (tid == 0) h->last = done;
      }
      __syncthreads();
      if (h->last) return;
      __syncthreads();
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    tail_rest<K, D, LG>(p, d, rec, L, TAIL_ALL);
  }
}

// Optimized mode, one workgroup per record, after the chunk kernel: repair
// rounds, seam validation, full-DP fallback, final path and every per-record
// output (plan_repairs cu:164-228, repair DP cu:727-760, validate_seams
// cu:562-592, fallback_recurrence cu:552-559, finish cu:642-667).
//
// Fast path (at most 64 chunks): when every chunk objective is finite and
// every seam is legal, the repair rounds merge nothing (plan_repairs joins
// every neighbour and its budget preflight proposes no region) and
// validate_seams stitches iff the fp32 total is finite. Wave 0 checks all
// seams at once from registers and writes the record's outputs.
template <int K, int D, bool LG>
__global__ void __launch_bounds__(K == 32 ? 640 : 256) tail_kernel(Params p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const Lds L = carve(lds_raw, p);
  Header* h = L.h;
  const int tid = threadIdx.x;
  const int rec = blockIdx.x;
  const RecordDesc d = load_uniform(p.desc + rec);
  const int n = (int)(1 + (d.frames - 1) / p.H);
  const bool split = p.tail_phase != TAIL_ALL;
  if (!split && p.tstate && tid == 0) {  // one-pass tail with banded fallbacks: none handed over yet
    glb(p.tstate)[rec].done = 0;
    glb(p.tstate)[rec].fallback = 0;
  }
  if (n <= 64) {
    if (tid < 64) {
      const int done = tail_fast<false>(p, d, rec, glb(p.slots) + d.chunk_offset, n);
      if (split && done && tid == 0) glb(p.tstate)[rec].done = 1;
      if (tid == 0) h->last = done;
    }
    __syncthreads();
    if (h->last) return;
    __syncthreads();
  }
  tail_rest<K, D, LG>(p, d, rec, L, p.tail_phase);
}

// Split tail, after TAIL_PLAN0: one workgroup per (chunk k, record) runs the
// first round's repair DP of the merged interval that starts at chunk k
// (repair DP over merged intervals, cu:727-760), or, in chunk 0's workgroup,
// the record's early full fallback (repair_recurrence, cu:535-550). The
// record's reuse_stats counters are added atomically; each workgroup writes
// only its own slot. The record's last workgroup to finish (an arrival count
// behind an agent-scope release, so its slots and labels are visible to
// whichever workgroup continues, on any XCD) then runs the later rounds and
// the seam check for the record; a record with no first-round DP continues in
// chunk 0's workgroup. Records therefore progress independently: a long
// fallback in one record delays no other record's later rounds.
template <int K, int D, bool LG>
__global__ void __launch_bounds__(K == 32 ? 640 : 256) repair_kernel(Params p) {
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const Lds L = carve(lds_raw, p);
  Header* h = L.h;
  const int tid = threadIdx.x;
  const int k = blockIdx.x, rec = blockIdx.y;
  const RecordDesc d = load_uniform(p.desc + rec);
  const int n = (int)(1 + (d.frames - 1) / p.H);
  if (k >= n) return;
  GLB TailState* state = glb(p.tstate) + rec;
  if (__builtin_amdgcn_readfirstlane(state->done)) return;
  const int early = __builtin_amdgcn_readfirstlane(state->ts.early);  // 0 or 1 as planned; 2 after band_kernel's fallback
  const int work = __builtin_amdgcn_readfirstlane(state->work);
  GLB Slot* slot = glb(p.slots) + d.chunk_offset + k;
  const Slot s = load_uniform(p.slots + d.chunk_offset + k);
  const bool fallback = p.overlap && early == 1 && k == 0;
  const bool fell_back = p.overlap && early == 2 && k == 0;  // band_kernel ran the early fallback
  const bool repair = !(p.overlap && early) && s.a < s.b && s.flag;
  if (!fallback && !fell_back && !repair && !(work == 0 && k == 0)) return;
  Rec r = make_rec(d, p, L);
  if (LG) r.st = p.stats + d.frame_offset;
  load_tokens(r, L.ytok);
  const int64_t T = r.T;
  const int S = r.S;
  const bool frontier_on = r.frontier != nullptr;
  const bool counted = frontier_on && (d.flags & DESC_REUSE_COUNTED);
  unsigned long long* reuse = reinterpret_cast<unsigned long long*>(p.tstate[rec].ts.reuse);
  if (fallback) {
    const bool resume = frontier_on && s.frontier_end > 0 && s.frontier_end <= T;
    if (resume && counted && tid == 0) {
      atomicAdd(reuse + 1, (unsigned long long)s.frontier_end);
      atomicAdd(reuse + 3, (unsigned long long)S);
    }
    const DPOut o = run_dp<K, D, LG>(p, r, L, 0, T, true, resume ? r.frontier : nullptr,
                                     resume ? s.frontier_end : 1, nullptr, TRACE_IF_FINITE);
    if (tid == 0) {
      state->status = isfinite(o.score) ? 0 : 1;
      state->objective = o.score;
      state->ts.early = 2;
    }
  } else if (repair) {
    bool resume = false;
    int64_t start_t = s.a + 1;
    GLB float* fr = frontier_on ? r.frontier + (int64_t)k * S : nullptr;
    if (frontier_on) {
      if (s.frontier_end > s.a && s.frontier_end <= s.b) {
        resume = true;
        start_t = s.frontier_end;
        if (tid == 0 && counted) {
          atomicAdd(reuse + 0, (unsigned long long)(s.frontier_end - s.a));
          atomicAdd(reuse + 3, (unsigned long long)S);
        }
      }
      if (tid == 0 && counted) atomicAdd(reuse + 2, (unsigned long long)S);
    }
    const DPOut o = run_dp<K, D, LG>(p, r, L, s.a, s.b, s.b == T, resume ? fr : nullptr, start_t, fr, TRACE_ALWAYS);
    if (tid == 0) {
      Slot out = s;
      out.objective = o.score;
      out.end = o.terminal;
      out.start = o.start;
      if (frontier_on) out.frontier_end = s.b;
      store_pod(slot, out);
    }
  }
  if (work > 0) {
    // every thread's writes (slot, labels, scores, state) reach the device
    // before the arrival is counted; the last arrival continues the record
    __threadfence();
    __syncthreads();
    if (tid == 0) h->last = __hip_atomic_fetch_sub(&p.tstate[rec].pending, 1, __ATOMIC_ACQ_REL,
                                                   __HIP_MEMORY_SCOPE_AGENT) == 1;
    __syncthreads();
    if (!h->last) return;
    __threadfence();
  }
  GLB Slot* gs = glb(p.slots) + d.chunk_offset;
  if (n <= p.lds_tail_slots) {
    Slot* ls = reinterpret_cast<Slot*>(lds_raw + ((uintptr_t)L.tslots - (uintptr_t)lds_raw));
    for (int j = tid; j < n; j += blockDim.x) ls[j] = load_pod(gs + j);
    __syncthreads();
    tail_body<K, D, LG>(p, d, rec, r, L, ls, true, TAIL_RESUME);
  } else {
    tail_body<K, D, LG>(p, d, rec, r, L, gs, false, TAIL_RESUME);
  }
}

// Token spans of one record per workgroup (the reference README's
// "Converting frame labels to timestamps": split the path into equal-label
// runs, drop blank runs, keep each run's start and exclusive end frame;
// blank-separated repeats stay separate occurrences). A successful path has
// exactly `tokens` such runs; the k-th run is written to spans[span_offset + k]
// as {start, end}; rows past the last run (a transcript holding the blank id,
// reachable only unchecked) and every row of a record whose status is not 0
// are {-1, -1}. Frames are scanned in tiles of 8 per thread with one
// block-wide prefix count per tile.
__global__ void __launch_bounds__(256) spans_kernel(const ffa_span_record* recs, const int64_t* labels,
                                                    const int32_t* status, int64_t* spans) {
  __shared__ int wsum[4];
  const ffa_span_record d = recs[blockIdx.x];
  const GLB int64_t* lab = glb(labels) + d.frame_offset;
  GLB int64_t* out = glb(spans) + 2 * d.span_offset;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (glb(status)[blockIdx.x] != 0) {
    for (int64_t k = tid; k < 2 * (int64_t)d.tokens; k += blockDim.x) out[k] = -1;
    return;
  }
  const int64_t T = d.frames;
  const int64_t blank = d.blank;
  int carry = 0;  // runs started before this tile
  for (int64_t base = 0; base < T; base += 8 * (int64_t)blockDim.x) {
    const int64_t f0 = base + 8 * (int64_t)tid;
    int64_t x[10];  // frames f0-1 .. f0+8 (out-of-range frames read as blank)
#pragma unroll
    for (int q = 0; q < 10; ++q) {
      const int64_t f = f0 - 1 + q;
      x[q] = (f >= 0 && f < T) ? lab[f] : blank;
    }
    int starts = 0;
#pragma unroll
    for (int q = 1; q <= 8; ++q) starts += x[q] != blank && x[q] != x[q - 1];
    // block-wide exclusive prefix of the run starts
    int incl = wave_scan_dpp(starts);
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int before = carry;
    for (int w = 0; w < wave; ++w) before += wsum[w];
    int total = carry;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) total += wsum[w];
    int k = before + incl - starts;  // index of the first run starting in this thread's frames
#pragma unroll
    for (int q = 1; q <= 8; ++q) {
      const int64_t f = f0 - 1 + q;
      const bool run = x[q] != blank;
      if (run && x[q] != x[q - 1]) {  // run start
        if (k < d.tokens) out[2 * k] = f;
        ++k;
      }
      if (run && x[q + 1] != x[q] && k - 1 < d.tokens && k >= 1) out[2 * (k - 1) + 1] = f + 1;  // run end
    }
    __syncthreads();
    carry = total;
  }
  // fewer runs than tokens (a transcript holding the blank id, unchecked): rows past the runs are -1
  for (int64_t k = (int64_t)carry + tid; k < d.tokens; k += blockDim.x) { out[2 * k] = -1; out[2 * k + 1] = -1; }
}

// One workgroup per record: any NaN or +inf rejects it (cu:881-891).
// Conventional mode with logits input: the row statistics of every frame,
// one workgroup per 128 frames of a record (grid: frame groups x records),
// before the full-record DP reads them.
template <class TB>
__global__ void __launch_bounds__(256) stats_kernel(Params p, TB tab) {
  RecordDesc d;
  if constexpr (kArgs<TB>) d = tab.rec[blockIdx.y];
  else d = load_uniform(p.desc + blockIdx.y);
  const int64_t a = (int64_t)blockIdx.x * 128;
  if (a >= d.frames) return;
  const int n = (int)min((int64_t)128, d.frames - a);
  rows_stats(glb(d.emissions) + a * (int64_t)d.vocab, n, d.vocab, nullptr, glb(p.stats) + d.frame_offset + a);
}

// Materialized log-softmax with the same row statistics as the fused path:
// out = (x - m) - ls per element, 128 frames of one record per workgroup.
__global__ void __launch_bounds__(256) log_softmax_kernel(const ffa_logits_record* recs) {
  __shared__ float2 st[128];
  const ffa_logits_record d = load_uniform(recs + blockIdx.y);
  const int64_t a = (int64_t)blockIdx.x * 128;
  if (a >= d.frames) return;
  const int n = (int)min((int64_t)128, d.frames - a);
  const int V = (int)d.vocab;
  const GLB float* src = glb(d.logits) + a * V;
  GLB float* dst = glb(d.log_probs) + a * V;
  rows_stats(src, n, V, st, nullptr);
  __syncthreads();
  const int total = n * V;
  for (int i = threadIdx.x; i < total; i += blockDim.x) dst[i] = lsm(src[i], st[i / V]);
}

// Measurement: a kernel that does nothing, launched with a given shape, so
// that the fixed cost of one dispatch as seen by a timing method (HIP events,
// a profiler) can be set beside the kernels' durations.
__global__ void empty_kernel() {}

__global__ void __launch_bounds__(1024) validity_kernel(const int64_t* desc, uint8_t* valid) {
  const int rec = blockIdx.x;
  const GLB float* values = (const GLB float*)(glb(desc)[2 * rec]);
  const int64_t n = glb(desc)[2 * rec + 1];
  int bad = 0;
  const uintptr_t addr = reinterpret_cast<uintptr_t>(values);
  int64_t head = (int64_t)(((16 - (addr & 15)) & 15) / 4);
  if (head > n) head = n;
  for (int64_t i = threadIdx.x; i < head; i += blockDim.x) {
    const float v = values[i];
    bad |= isnan(v) || v == INFINITY;
  }
  const GLB v4f_t* v4 = (const GLB v4f_t*)(values + head);
  const int64_t n4 = (n - head) / 4;
  auto reject = [](const v4f_t v) {  // NaN or +inf (x != x, or x == +inf)
    return (v.x != v.x) | (v.x == INFINITY) | (v.y != v.y) | (v.y == INFINITY) | (v.z != v.z) | (v.z == INFINITY) |
           (v.w != v.w) | (v.w == INFINITY);
  };
  const int64_t stride = blockDim.x;
  int64_t i = threadIdx.x;
  for (; i + 3 * stride < n4; i += 4 * stride) {  // four 16-byte loads in flight per thread
    const v4f_t a = v4[i], b = v4[i + stride], c = v4[i + 2 * stride], d = v4[i + 3 * stride];
    bad |= reject(a) | reject(b) | reject(c) | reject(d);
  }
  for (; i < n4; i += stride) bad |= reject(v4[i]);
  for (int64_t i = head + 4 * n4 + threadIdx.x; i < n; i += blockDim.x) {
    const float v = values[i];
    bad |= isnan(v) || v == INFINITY;
  }
  bad = __syncthreads_or(bad);
  if (threadIdx.x == 0) glb(valid)[rec] = bad ? 0 : 1;
}

}  // namespace ffa

// ===========================================================================
// Host side: the C ABI of include/ffa.h.
namespace {

thread_local std::string g_error;
thread_local hipEvent_t g_profile_start = nullptr, g_profile_stop = nullptr;

int fail(int code, const std::string& message) {
  g_error = message;
  return code;
}

inline int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

// internal[] of ffa_align_plan
enum {
  I_K, I_NT, I_SLOTS, I_LDS, I_UCAP, I_DCAP, I_VWORDS, I_TAILSLOTS, I_FRONTIER, I_BUDGET,
  I_OVERLAP, I_WS_SLOTS, I_WS_FRONTIER, I_MODE, I_H, I_FMIN, I_REPAIR_MIN, I_EBLK, I_LOGITS, I_WS_STATS,
  I_MAX_FRAMES, I_WS_BP, I_SPLIT, I_WS_TSTATE, I_BANDS, I_BAND_STRIDE, I_WS_BAND, I_BAND_BYTES, I_BAND_LDS
};
static_assert(I_BAND_LDS < 32, "plan->internal holds 32 values");

// Banded DP launch (conventional mode, transcripts of more than 1,024 states):
// workgroups (one per band), LDS bytes, and the 16-byte words zeroed first.
struct BandLaunch {
  int64_t bands;
  size_t lds;
  int64_t zero_words;
};

template <int K, int D, bool LG, class TB>
int launch_geometry(const ffa::Params& p, const TB& tab, int NT, size_t lds, bool optimized, bool split, bool fused,
                    int64_t max_frames, const BandLaunch& band, hipStream_t stream) {
  hipEvent_t start = g_profile_start, stop = g_profile_stop;
  g_profile_start = g_profile_stop = nullptr;
  if (p.logits && !optimized)
    hipLaunchKernelGGL(ffa::stats_kernel<TB>, dim3((unsigned)((max_frames + 127) / 128), (unsigned)p.count), dim3(256),
                       0, stream, p, tab);
  if (band.bands > 0) {  // the banded DP's control words and edge arrays start at zero
    const int64_t blocks = std::min<int64_t>(2048, (band.zero_words + 255) / 256);
    hipLaunchKernelGGL(ffa::zero_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                       reinterpret_cast<ffa::v4i_t*>(p.band_ctl), band.zero_words);
  }
  if (start) (void)hipEventRecord(start, stream);
  if (!optimized && band.bands > 0) {
    hipLaunchKernelGGL((ffa::band_kernel<TB, 0>), dim3((unsigned)band.bands), dim3(64), band.lds, stream, p, tab);
  } else if (!optimized) {
    hipLaunchKernelGGL((ffa::conventional_kernel<K, D, LG, TB>), dim3(p.count), dim3(NT), lds, stream, p, tab);
  } else {
    const int grid = 8 * ((p.total_slots + 7) / 8);
    if constexpr (!LG && K <= 16) {
      if (fused) {  // one launch: the chunk kernel runs each record's tail in its last chunk workgroup
        hipLaunchKernelGGL((ffa::chunk_kernel<K, D, LG, TB, true>), dim3(grid), dim3(std::max(NT, 128)), lds, stream, p,
                           tab);
        if (stop) (void)hipEventRecord(stop, stream);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return fail(FFA_E_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
        return FFA_OK;
      }
    }
    hipLaunchKernelGGL((ffa::chunk_kernel<K, D, LG, TB, false>), dim3(grid), dim3(std::max(NT, 128)), lds, stream, p,
                       tab);
  }
  if (stop) (void)hipEventRecord(stop, stream);
  if (optimized && split) {  // first-round planning, then one workgroup per first-round interval
    ffa::Params q = p;
    const int64_t n_max = 1 + (max_frames - 1) / p.H;
    q.tail_phase = ffa::TAIL_PLAN0;
    hipLaunchKernelGGL((ffa::tail_kernel<K, D, LG>), dim3(p.count), dim3(NT), lds, stream, q);
    if (band.bands > 0)  // early full fallbacks as banded DPs
      hipLaunchKernelGGL((ffa::band_kernel<ffa::NoTable, 1>), dim3((unsigned)band.bands), dim3(64), band.lds, stream,
                         q, ffa::NoTable{0});
    hipLaunchKernelGGL((ffa::repair_kernel<K, D, LG>), dim3((unsigned)n_max, (unsigned)p.count), dim3(NT), lds, stream,
                       q);
    if (band.bands > 0)  // fallbacks after failed seams as banded DPs
      hipLaunchKernelGGL((ffa::band_kernel<ffa::NoTable, 2>), dim3((unsigned)band.bands), dim3(64), band.lds, stream,
                         q, ffa::NoTable{0});
  } else if (optimized) {
    hipLaunchKernelGGL((ffa::tail_kernel<K, D, LG>), dim3(p.count), dim3(NT), lds, stream, p);
    if (band.bands > 0)  // fallbacks after failed seams as banded DPs
      hipLaunchKernelGGL((ffa::band_kernel<ffa::NoTable, 2>), dim3((unsigned)band.bands), dim3(64), band.lds, stream,
                         p, ffa::NoTable{0});
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(FFA_E_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
  return FFA_OK;
}

// Arrival counters of the fused tail: 128 KiB per (device, stream) (one counter
// per 128-byte line for each of up to FUSED_MAX_CHUNKS records),
// zeroed once on the stream when first needed and held until the process
// ends; every record's last chunk workgroup leaves its counter at zero again.
// Calls on one stream run in order, so they never use the counters at the same
// time; calls on different streams have their own. Returns nullptr (the call
// then takes the two-launch path) while the stream is being captured into a
// graph and has no counters yet, or when the allocation fails.
int32_t* arrival_counters(hipStream_t stream) {
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess) return nullptr;
  thread_local int last_device = -1;
  thread_local hipStream_t last_stream = nullptr;
  thread_local int32_t* last_counters = nullptr;
  if (last_counters && device == last_device && stream == last_stream) return last_counters;
  static std::mutex lock;
  static std::map<std::pair<int, hipStream_t>, int32_t*> pool;
  std::lock_guard<std::mutex> guard(lock);
  auto it = pool.find({device, stream});
  if (it == pool.end()) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone) return nullptr;
    void* ptr = nullptr;
    const size_t bytes = sizeof(int32_t) * ffa::FUSED_MAX_CHUNKS * ffa::ARRIVAL_STRIDE;
    if (hipMalloc(&ptr, bytes) != hipSuccess) return nullptr;
    if (hipMemsetAsync(ptr, 0, bytes, stream) != hipSuccess) {
      (void)hipFree(ptr);
      return nullptr;
    }
    it = pool.emplace(std::make_pair(device, stream), static_cast<int32_t*>(ptr)).first;
  }
  last_device = device;
  last_stream = stream;
  last_counters = it->second;
  return last_counters;
}

int states_of(const ffa_record& r) { return (int)(2 * r.tokens + 1); }
int64_t stride_of(int S) { return 2 * (((int64_t)S + 31) / 32); }

// Frontier storage beyond the reference's gating (alignment.cu:374, T >=
// frontier_min_frames): in optimized mode with chunks of at least 32 frames
// every record keeps one frontier per chunk (S floats, at most an eighth of its
// backpointer bytes), so a repair that starts where a chunk DP started, and a
// fallback after a repair from frame 0, resume instead of recomputing those
// frames. A resumed DP gives the same values as a fresh one, so only
// reuse_stats follows the reference's gating.
bool frontier_for_every_record(bool optimized, int64_t H) { return optimized && H >= 32; }

// The 2-bit backpointer row of a record is 2*ceil(S/32) words; K contiguous
// states per thread. K = 4, 8 or 16 keep a record in at most 4 waves (one per
// SIMD); wider transcripts take K = 32 and up to 10 waves.
void geometry(int s_max, int* K, int* NT) {
  int k = 4;
  while (k < 32 && (s_max + k - 1) / k > 256) k *= 2;
  const int threads = (s_max + k - 1) / k;
  *K = k;
  *NT = (int)std::max<int64_t>(64, align_up(threads, 64));
}

}  // namespace

extern "C" {

const char* ffa_last_error(void) { return g_error.c_str(); }

int ffa_profile_next_launch(hipEvent_t start, hipEvent_t stop) {
  g_profile_start = start;
  g_profile_stop = stop;
  return FFA_OK;
}

int ffa_launch_floor(int32_t workgroups, int32_t threads, hipStream_t stream) {
  if (workgroups <= 0 || threads <= 0 || threads > 1024) return fail(FFA_E_INVALID, "workgroups > 0, threads 1..1024");
  hipLaunchKernelGGL(ffa::empty_kernel, dim3((unsigned)workgroups), dim3((unsigned)threads), 0, stream);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(FFA_E_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
  return FFA_OK;
}

void ffa_default_options(int optimized, ffa_align_options* o) {  // alignment.py:496-501
  std::memset(o, 0, sizeof(*o));
  o->chunk_frames = 128;
  o->mode = optimized ? 2 : 0;
  o->threads = 512;
  o->repair_rounds = 2;
  o->optimization_pass = 2;
  o->variant = 2;
  o->repair_budget_frames = optimized ? 512 : 0;
  o->repair_threads = 0;
  o->compact_alphabet = 0;
  o->parallel_traceback = 1;
  o->overlap_fallback = optimized ? 1 : 0;
  o->trace_min_frames = 2048;
  o->repair_min_frames = 2048;
  o->frontier_reuse = optimized ? 1 : 0;
  o->frontier_min_frames = 2048;
  o->check_inputs = 1;
}

int ffa_align_plan_batch(const ffa_record* records, int64_t count, const ffa_align_options* o,
                         ffa_align_plan* plan) {
  using ffa::MAX_H;
  // option checks, alignment.cu:924-941
  if (o->frontier_min_frames < 0 || o->frontier_min_frames > INT_MAX)
    return fail(FFA_E_INVALID, "frontier_min_frames must be a nonnegative int32");
  if (o->repair_min_frames < 0 || o->repair_min_frames > INT_MAX)
    return fail(FFA_E_INVALID, "repair_min_frames must be a nonnegative int32");
  if (o->trace_min_frames <= 0 || o->trace_min_frames > INT_MAX)
    return fail(FFA_E_INVALID, "trace_min_frames must be a positive int32");
  if (o->overlap_fallback && o->repair_threads != 0 && o->repair_threads != o->threads)
    return fail(FFA_E_INVALID, "overlap preserves fallback geometry");
  if (o->repair_budget_frames < 0 || o->repair_budget_frames > INT_MAX)
    return fail(FFA_E_INVALID, "repair budget must fit nonnegative int32");
  if (!(o->repair_threads == 0 || o->repair_threads == 128 || o->repair_threads == 256 || o->repair_threads == 512))
    return fail(FFA_E_INVALID, "repair threads must be 0/128/256/512");
  if (o->variant < 0 || o->variant > 2) return fail(FFA_E_INVALID, "variant must be 0, 1, or 2");
  if (!(o->threads == 128 || o->threads == 256 || o->threads == 512)) return fail(FFA_E_INVALID, "invalid block size");
  if (!(o->optimization_pass == 2 || o->optimization_pass == 3))
    return fail(FFA_E_INVALID, "optimization pass must be 2 or 3");
  if (o->repair_rounds < 0 || o->repair_rounds > 2) return fail(FFA_E_INVALID, "invalid repair rounds");
  if (count <= 0 || count > FFA_MAX_BATCH)
    return fail(FFA_E_INVALID, "batch must contain 1..65535 matching emissions, targets and blanks");
  if (o->chunk_frames <= 0 || o->chunk_frames > MAX_H || o->mode < 0 || o->mode > 2)
    return fail(FFA_E_INVALID, "invalid chunk size or mode (chunk_frames must be 1..512)");
  if (o->logits != 0 && o->logits != 1) return fail(FFA_E_INVALID, "logits must be 0 or 1");
  const bool logits = o->logits != 0;
  const bool optimized = o->mode != 0;
  const int64_t H = o->chunk_frames;
  int64_t total_frames = 0, bp_words = 0, slots = 0, frontier_floats = 0;
  int64_t max_frames = 0, u_max = 0, v_max = 0, d_cap = 1, n_max = 0;
  int s_max = 1;
  int64_t v_min = INT64_MAX;
  for (int64_t i = 0; i < count; ++i) {
    const ffa_record& r = records[i];
    if (r.frames <= 0 || r.frames > INT_MAX || r.vocab <= 0 || r.vocab > FFA_MAX_VOCAB || r.tokens < 0 ||
        2 * r.tokens + 1 > FFA_MAX_STATES || r.blank < 0 || r.blank >= r.vocab)
      return fail(FFA_E_INVALID, "resident input shape or blank outside supported range");
    if (!r.emissions || (r.tokens > 0 && !r.targets))
      return fail(FFA_E_INVALID, "null emission or target pointer");
    if ((reinterpret_cast<uintptr_t>(r.targets) & 7) != 0 || (reinterpret_cast<uintptr_t>(r.targets) >> 48) != 0)
      return fail(FFA_E_INVALID, "target pointer not 8-byte aligned inside the 48-bit GPU address space");
    const int S = states_of(r);
    total_frames += r.frames;
    bp_words += r.frames * stride_of(S);
    max_frames = std::max(max_frames, r.frames);
    u_max = std::max(u_max, r.tokens);
    v_max = std::max(v_max, r.vocab);
    d_cap = std::max(d_cap, std::min(r.vocab, r.tokens + 1));
    s_max = std::max(s_max, S);
    v_min = std::min(v_min, r.vocab);
    if (optimized) {
      const int64_t n = 1 + (r.frames - 1) / H;
      slots += n;
      n_max = std::max(n_max, n);
    }
  }
  if (slots > INT_MAX || bp_words < 0) return fail(FFA_E_INVALID, "chunk endpoints or interval indices exceed int32 range");
  const bool budget_on = max_frames >= o->repair_min_frames;  // alignment.cu:993-996
  const bool frontier = optimized && o->frontier_reuse && max_frames >= o->frontier_min_frames;  // :935, :1002
  const bool store_all = frontier_for_every_record(optimized, H);
  for (int64_t i = 0; i < count; ++i)
    if (store_all || (frontier && records[i].frames >= o->frontier_min_frames))
      frontier_floats += (1 + (records[i].frames - 1) / H) * (int64_t)states_of(records[i]);
  int K, NT;
  geometry(s_max, &K, &NT);
  const int64_t v_words = (v_max + 31) / 32;
  const int64_t tail_slots = optimized ? std::min<int64_t>(n_max, ffa::TAIL_SLOT_CAP) : 0;
  const int64_t greedy_bytes = 20 * ffa::greedy_frames(H) + 2048 + align_up(2 * d_cap, 16) + 8 * v_words +
                               (logits ? 16 + 8 * ffa::greedy_frames(H) : 0);
  const int64_t region = std::max(greedy_bytes, 32 * tail_slots);
  const int64_t targets = align_up(2 * (std::max<int64_t>(u_max, 1) + ffa::YTOK_PAD), 16);
  int64_t lds = align_up((int64_t)sizeof(ffa::Header), 16) + 2 * targets + region;
  if (lds > 64 * 1024) return fail(FFA_E_INVALID, "batch needs more than 64 KiB of LDS per workgroup");
  // DP emission blocks (two halves of F rows of up to 64 values) for records
  // with V <= 64: 32 frames per block when the space fits, else 16, else none
  int64_t eblk_frames = 0;
  if (v_min <= ffa::EBLK_COLS)
    for (int64_t f = 32; f >= 16 && !eblk_frames; f /= 2)
      if (lds + 8 * f * ffa::EBLK_COLS <= 64 * 1024) eblk_frames = f;
  lds += 8 * eblk_frames * ffa::EBLK_COLS;
  // workspace: the record table (uploaded batches: the whole table; batches
  // passed in the kernel arguments: the descriptors the chunk kernel copies
  // for the tail kernel), backpointers, chunk slots, frontiers, statistics
  const bool uploaded = count > ffa::ARG_RECORDS;
  const int64_t table_bytes =
      count * (int64_t)sizeof(ffa::RecordDesc) + (uploaded ? (int64_t)sizeof(ffa::ChunkEntry) * slots : 0);
  int64_t ws = align_up(table_bytes, 256);
  const int64_t ws_bp = ws;
  ws += align_up(4 * bp_words, 256);
  const int64_t ws_slots = ws;
  ws += align_up(32 * slots, 256);
  const int64_t ws_frontier = ws;
  ws += align_up(4 * frontier_floats, 256);
  // split tail: batches with a record of at least 2,048 frames run each repair
  // round's intervals in parallel workgroups (a few more launches, against
  // repair DPs of milliseconds)
  const bool split = optimized && o->repair_rounds > 0 && max_frames >= 2048 && count * n_max <= (1 << 20);
  // optimized batches of transcripts with more than 4,096 states that take no
  // split tail (no repair rounds) hand their fallbacks to the banded DP too,
  // through the same per-record state
  const bool band_tail = optimized && !split && !logits && K == 32;
  const int64_t ws_tstate = ws;
  if (split || band_tail) ws += align_up((int64_t)sizeof(ffa::TailState) * count, 256);
  const int64_t ws_stats = ws;
  if (logits) ws += align_up(8 * total_frames, 256);
  // banded DP (log-probabilities, more than 1,024 states; conventional mode,
  // or optimized mode's early full fallbacks under the split tail):
  // control words (ticket, late flag, arrival counts, terminal values) and
  // the edge arrays (8 bytes per frame and band boundary of the widest record)
  int64_t bands = 0, band_stride = 0, band_bytes = 0, band_lds = 0;
  const int64_t ws_band = ws;
  if ((!logits && K >= 8 && (!optimized || split)) || band_tail) {
    int64_t nb_max = 1;
    for (int64_t i = 0; i < count; ++i) {
      const int64_t nb = (states_of(records[i]) + ffa::BAND_STATES - 1) / ffa::BAND_STATES;
      bands += nb;
      nb_max = std::max(nb_max, nb);
    }
    band_stride = nb_max - 1;
    band_bytes = align_up(4 * (ffa::BAND_CTL_HEAD + count) + 8 * count, 256) + 8 * total_frames * band_stride;
    band_bytes = align_up(band_bytes, 256);
    ws += band_bytes;
    band_lds = align_up((int64_t)sizeof(ffa::Header), 16) + targets;
  }
  std::memset(plan, 0, sizeof(*plan));
  plan->count = count;
  plan->total_frames = total_frames;
  plan->table_bytes = table_bytes;
  plan->table_uploaded = uploaded ? 1 : 0;
  plan->workspace_bytes = std::max<int64_t>(ws, 256);
  plan->reuse_rows = frontier ? count : 0;
  int64_t* in = plan->internal;
  in[I_K] = K;
  in[I_NT] = NT;
  in[I_SLOTS] = slots;
  in[I_LDS] = lds;
  in[I_UCAP] = std::max<int64_t>(u_max, 1);
  in[I_DCAP] = d_cap;
  in[I_VWORDS] = v_words;
  in[I_TAILSLOTS] = tail_slots;
  in[I_EBLK] = eblk_frames;
  in[I_FRONTIER] = frontier ? 1 : 0;
  in[I_BUDGET] = budget_on ? o->repair_budget_frames : 0;
  in[I_OVERLAP] = (budget_on && o->overlap_fallback) ? 1 : 0;
  in[I_WS_SLOTS] = ws_slots;
  in[I_WS_FRONTIER] = ws_frontier;
  in[I_MODE] = o->mode;
  in[I_H] = H;
  in[I_FMIN] = o->frontier_min_frames;
  in[I_REPAIR_MIN] = o->repair_min_frames;
  in[I_LOGITS] = logits ? 1 : 0;
  in[I_WS_STATS] = ws_stats;
  in[I_MAX_FRAMES] = max_frames;
  in[I_WS_BP] = ws_bp;
  in[I_SPLIT] = split ? 1 : 0;
  in[I_WS_TSTATE] = ws_tstate;
  in[I_BANDS] = bands;
  in[I_BAND_STRIDE] = band_stride;
  in[I_WS_BAND] = ws_band;
  in[I_BAND_BYTES] = band_bytes;
  in[I_BAND_LDS] = band_lds;
  return FFA_OK;
}

int ffa_align_describe(const ffa_align_plan* plan, const ffa_record* records, void* host_table,
                       int64_t host_table_bytes) {
  if (host_table_bytes < plan->table_bytes) return fail(FFA_E_SIZE, "descriptor table buffer too small");
  const int64_t count = plan->count;
  const int64_t* in = plan->internal;
  const bool optimized = in[I_MODE] != 0;
  const bool frontier = in[I_FRONTIER] != 0;
  const int64_t H = in[I_H];
  auto* desc = static_cast<ffa::RecordDesc*>(host_table);
  auto* chunks = reinterpret_cast<ffa::ChunkEntry*>(desc + count);
  const bool store_all = frontier_for_every_record(optimized, H);
  int64_t frame = 0, bp = 0, fr = 0;
  int32_t slot = 0;
  for (int64_t i = 0; i < count; ++i) {
    const ffa_record& r = records[i];
    const int S = states_of(r);
    ffa::RecordDesc& d = desc[i];
    d.emissions = r.emissions;
    d.targets = r.targets;
    d.frames = (int32_t)r.frames;
    d.chunk_offset = slot;
    d.vocab = (int32_t)r.vocab;
    d.tokens = (int32_t)r.tokens;
    d.frame_offset = frame;
    d.bp_offset = bp;
    d.frontier_offset = -1;
    d.blank = (int32_t)r.blank;
    const bool counted = frontier && r.frames >= in[I_FMIN];  // alignment.cu:374
    d.flags = counted ? ffa::DESC_REUSE_COUNTED : 0;
    const int64_t n = 1 + (r.frames - 1) / H;
    if (counted || store_all) {  // per-record frontier storage, one block of S floats per chunk
      d.frontier_offset = fr;
      fr += n * S;
    }
    if (optimized && plan->table_uploaded) {
      // greedy fast path: whole rows in registers (V <= 32, 16-byte rows) and
      // one frame per lane of two waves
      const bool fast = in[I_MODE] == 2 && H <= 128 && r.vocab <= 32 && r.vocab % 4 == 0 &&
                        (reinterpret_cast<uintptr_t>(r.emissions) & 15) == 0;
      const uint64_t lo = (uint64_t)reinterpret_cast<uintptr_t>(r.targets) >> 3 |
                          (uint64_t)r.tokens << ffa::ENTRY_U_SHIFT |
                          (fast ? (1ull << ffa::ENTRY_FAST_SHIFT | (uint64_t)(r.vocab / 4 - 1) << ffa::ENTRY_QUADS_SHIFT)
                                : 0ull);
      for (int64_t c = 0; c < n; ++c) {
        ffa::ChunkEntry& e = chunks[slot + c];
        e.lo = lo;
        e.hi = (uint64_t)i | (uint64_t)(std::min<int64_t>(H, r.frames - c * H) - 1) << 16 | (uint64_t)c << 25;
      }
    }
    if (optimized) slot += (int32_t)n;
    frame += r.frames;
    bp += r.frames * stride_of(S);
  }
  return FFA_OK;
}

}  // extern "C"

namespace {

// ffa_align_launch with the fused tail's arrival counters chosen by the caller:
// `counters` (FFA_MAX_BATCH zeroed ints) or, when it is null, the stream's own
// (arrival_counters).
int align_launch(const ffa_align_plan* plan, const ffa_align_options* o, const void* host_table,
                 const uint8_t* emission_validity, const ffa_align_outputs* out, void* workspace, int32_t* counters,
                 hipStream_t stream) {
  const int64_t* in = plan->internal;
  const bool optimized = in[I_MODE] != 0;
  if (!host_table || !workspace || !out->labels || !out->scores || !out->status || !out->objective ||
      !out->stitched || !out->repair_passes || !out->repaired_frames || !out->shortcut_stats || !out->routing_stats)
    return fail(FFA_E_INVALID, "null table, workspace or output pointer");
  if (plan->reuse_rows > 0 && !out->reuse_stats) return fail(FFA_E_INVALID, "reuse_stats required for this plan");
  if (o->mode != in[I_MODE] || o->chunk_frames != in[I_H] || (o->logits != 0) != (in[I_LOGITS] != 0))
    return fail(FFA_E_INVALID, "options differ from the plan");
  auto* ws = static_cast<unsigned char*>(workspace);
  ffa::Params p{};
  // the record table: in the workspace's head (uploaded batches), or the
  // descriptor copies the chunk kernel leaves there for the tail kernel
  p.desc = reinterpret_cast<const ffa::RecordDesc*>(ws);
  p.chunks = reinterpret_cast<const ffa::ChunkEntry*>(p.desc + plan->count);
  p.validity = emission_validity;
  p.labels = out->labels;
  p.scores = out->scores;
  p.status = out->status;
  p.objective = out->objective;
  p.stitched = out->stitched;
  p.repair_passes = out->repair_passes;
  p.repaired_frames = out->repaired_frames;
  p.shortcut_stats = out->shortcut_stats;
  p.routing_stats = out->routing_stats;
  p.reuse_stats = plan->reuse_rows > 0 ? out->reuse_stats : nullptr;
  p.bp = reinterpret_cast<uint32_t*>(ws + in[I_WS_BP]);
  p.slots = reinterpret_cast<ffa::Slot*>(ws + in[I_WS_SLOTS]);
  p.frontiers = reinterpret_cast<float*>(ws + in[I_WS_FRONTIER]);
  p.budget = in[I_BUDGET];
  p.repair_min = in[I_REPAIR_MIN];
  p.frontier_min = in[I_FMIN];
  p.count = (int32_t)plan->count;
  p.total_slots = (int32_t)in[I_SLOTS];
  p.H = (int32_t)in[I_H];
  p.mode = (int32_t)in[I_MODE];
  p.repair_rounds = (int32_t)o->repair_rounds;
  p.check_inputs = o->check_inputs ? 1 : 0;
  p.overlap = (int32_t)in[I_OVERLAP];
  p.u_cap = (int32_t)in[I_UCAP];
  p.d_cap = (int32_t)in[I_DCAP];
  p.v_words = (int32_t)in[I_VWORDS];
  p.lds_tail_slots = (int32_t)in[I_TAILSLOTS];
  p.eblk_frames = (int32_t)in[I_EBLK];
  p.logits = (int32_t)in[I_LOGITS];
  p.stats = p.logits ? reinterpret_cast<float2*>(ws + in[I_WS_STATS]) : nullptr;
  const int NT = (int)in[I_NT];
  const size_t lds = (size_t)in[I_LDS];
  const int64_t max_frames = in[I_MAX_FRAMES];
  const bool split = in[I_SPLIT] != 0;
  p.tstate = (split || (optimized && in[I_BANDS] > 0)) ? reinterpret_cast<ffa::TailState*>(ws + in[I_WS_TSTATE])
                                                       : nullptr;
  // the fused tail: optimized mode with greedy shortcuts, log-probabilities,
  // no split tail, at most 16 states per thread, and at most four chunks per
  // CU (larger grids run in several rounds of workgroups, and the hand-off's
  // wait at each chunk's end would hold back the later rounds: C5's 2,300
  // chunks measured 1.3% slower fused)
  const bool fusable = optimized && p.mode == 2 && !p.logits && !split && in[I_K] <= 16 &&
                       p.total_slots <= ffa::FUSED_MAX_CHUNKS;
  p.arrivals = !fusable ? nullptr : counters ? counters : arrival_counters(stream);
  const bool fused = p.arrivals != nullptr;
  BandLaunch band{in[I_BANDS], (size_t)in[I_BAND_LDS], in[I_BAND_BYTES] / 16};
  if (band.bands > 0) {
    p.band_ctl = reinterpret_cast<int32_t*>(ws + in[I_WS_BAND]);
    p.edges = reinterpret_cast<uint64_t*>(
        ws + in[I_WS_BAND] + align_up(4 * (ffa::BAND_CTL_HEAD + plan->count) + 8 * plan->count, 256));
    p.band_stride = (int32_t)in[I_BAND_STRIDE];
  }
  auto run = [&](const auto& tab) -> int {
    using TB = std::decay_t<decltype(tab)>;
    switch (in[I_K]) {
      case 4: return p.logits ? launch_geometry<4, 8, true, TB>(p, tab, NT, lds, optimized, split, fused, max_frames, band, stream)
                              : launch_geometry<4, 8, false, TB>(p, tab, NT, lds, optimized, split, fused, max_frames, band, stream);
      case 8: return p.logits ? launch_geometry<8, 6, true, TB>(p, tab, NT, lds, optimized, split, fused, max_frames, band, stream)
                              : launch_geometry<8, 6, false, TB>(p, tab, NT, lds, optimized, split, fused, max_frames, band, stream);
      case 16: return p.logits ? launch_geometry<16, 4, true, TB>(p, tab, NT, lds, optimized, split, fused, max_frames, band, stream)
                               : launch_geometry<16, 4, false, TB>(p, tab, NT, lds, optimized, split, fused, max_frames, band, stream);
      case 32: return p.logits ? launch_geometry<32, 1, true, TB>(p, tab, NT, lds, optimized, split, fused, max_frames, band, stream)
                               : launch_geometry<32, 1, false, TB>(p, tab, NT, lds, optimized, split, fused, max_frames, band, stream);
      default: return fail(FFA_E_INVALID, "corrupt plan");
    }
  };
  if (plan->table_uploaded) {
    const hipError_t err = hipMemcpyAsync(ws, host_table, plan->table_bytes, hipMemcpyHostToDevice, stream);
    if (err != hipSuccess) return fail(FFA_E_HIP, std::string("descriptor upload failed: ") + hipGetErrorString(err));
    return run(ffa::NoTable{0});
  }
  if (plan->count > ffa::ARG_RECORDS || plan->table_bytes != plan->count * (int64_t)sizeof(ffa::RecordDesc))
    return fail(FFA_E_INVALID, "corrupt plan");
  ffa::ArgTable tab;
  std::memcpy(tab.rec, host_table, plan->table_bytes);
  std::memset(tab.rec + plan->count, 0, sizeof(tab) - plan->table_bytes);
  return run(tab);
}

}  // namespace

extern "C" int ffa_align_launch(const ffa_align_plan* plan, const ffa_align_options* o, const void* host_table,
                                const uint8_t* emission_validity, const ffa_align_outputs* out, void* workspace,
                                hipStream_t stream) {
  return align_launch(plan, o, host_table, emission_validity, out, workspace, nullptr, stream);
}

// Allocation-free alignment (ffa_align_launch_noalloc). The descriptor table
// and the workspace of a call live in this array, one copy per GPU, held until
// the process ends. In host code `scratch` names a host-side stand-in, not the
// device memory: the host only ever uses the per-device address that
// hipGetSymbolAddress returns for it.
static __device__ __align__(256) unsigned char scratch[FFA_NOALLOC_MAX_BYTES];
// The fused tail's arrival counters of that entry (one per record, each on its
// own 128-byte line): zero when
// the library is loaded, and every call leaves them at zero again.
static __device__ __align__(256) int32_t arrival_scratch[ffa::FUSED_MAX_CHUNKS * ffa::ARRIVAL_STRIDE];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch_ptr[kMaxDevices] = {};
void* g_arrival_ptr[kMaxDevices] = {};

// The device addresses of `scratch` and `arrival_scratch` on the current
// device `device`, looked up once per device (with that device current) and kept.
int scratch_address(int device, unsigned char** out, int32_t** arrivals) {
  std::lock_guard<std::mutex> lock(g_scratch_lock);
  if (!g_scratch_ptr[device]) {
    void* ptr = nullptr;
    hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr)
      return fail(FFA_E_HIP, std::string("scratch address lookup failed: ") + hipGetErrorString(err));
    void* counters = nullptr;
    err = hipGetSymbolAddress(&counters, HIP_SYMBOL(arrival_scratch));
    if (err != hipSuccess || !counters)
      return fail(FFA_E_HIP, std::string("scratch address lookup failed: ") + hipGetErrorString(err));
    g_arrival_ptr[device] = counters;
    g_scratch_ptr[device] = ptr;
  }
  *out = static_cast<unsigned char*>(g_scratch_ptr[device]);
  *arrivals = static_cast<int32_t*>(g_arrival_ptr[device]);
  return FFA_OK;
}

}  // namespace

extern "C" int ffa_align_launch_noalloc(const ffa_align_plan* plan, const ffa_align_options* o,
                                        const void* host_table, const uint8_t* emission_validity,
                                        const ffa_align_outputs* out, hipStream_t stream) {
  if (!plan || !o || !host_table || !out) return fail(FFA_E_INVALID, "null plan, options, table or outputs");
  if (plan->workspace_bytes <= 0 || plan->workspace_bytes > (int64_t)FFA_NOALLOC_MAX_BYTES)
    return fail(FFA_E_SIZE, "batch needs " + std::to_string(plan->workspace_bytes) +
                                " bytes of device scratch; the allocation-free entry holds at most " +
                                std::to_string((int64_t)FFA_NOALLOC_MAX_BYTES) + " (use ffa_align_launch)");
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess || device < 0 || device >= kMaxDevices)
    return fail(FFA_E_HIP, std::string("no usable current device: ") + hipGetErrorString(err));
  if (stream) {
    int stream_device = -1;
    err = hipStreamGetDevice(stream, &stream_device);
    if (err != hipSuccess) return fail(FFA_E_HIP, std::string("stream query failed: ") + hipGetErrorString(err));
    if (stream_device != device) return fail(FFA_E_INVALID, "the stream belongs to another device than the current one");
  }
  unsigned char* base = nullptr;
  int32_t* arrivals = nullptr;
  const int rc = scratch_address(device, &base, &arrivals);
  if (rc != FFA_OK) return rc;
  // nothing in the workspace has to start at zero: every kernel writes what it
  // reads; the fused tail's counters start at zero and every call leaves them so
  return align_launch(plan, o, host_table, emission_validity, out, base, arrivals, stream);
}

extern "C" int ffa_token_spans_launch(const ffa_span_record* device_records, int64_t count, const int64_t* labels,
                                      const int32_t* status, int64_t* spans, hipStream_t stream) {
  if (count <= 0 || count > FFA_MAX_BATCH) return fail(FFA_E_INVALID, "provide 1..65535 records");
  if (!device_records || !labels || !status || !spans) return fail(FFA_E_INVALID, "null record, label, status or span pointer");
  hipLaunchKernelGGL(ffa::spans_kernel, dim3((unsigned)count), dim3(256), 0, stream, device_records, labels, status, spans);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(FFA_E_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
  return FFA_OK;
}

extern "C" int ffa_log_softmax_launch(const ffa_logits_record* device_records, int64_t count, int64_t max_frames,
                                      hipStream_t stream) {
  if (count <= 0 || count > FFA_MAX_BATCH) return fail(FFA_E_INVALID, "provide 1..65535 records");
  if (max_frames <= 0 || max_frames > INT_MAX) return fail(FFA_E_INVALID, "max_frames must be 1..2^31-1");
  if (!device_records) return fail(FFA_E_INVALID, "null record pointer");
  hipLaunchKernelGGL(ffa::log_softmax_kernel, dim3((unsigned)((max_frames + 127) / 128), (unsigned)count), dim3(256),
                     0, stream, device_records);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(FFA_E_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
  return FFA_OK;
}

extern "C" int ffa_emission_validity_launch(const int64_t* device_descriptors, int64_t count, uint8_t* valid,
                                            hipStream_t stream) {
  if (count <= 0 || count > FFA_MAX_BATCH) return fail(FFA_E_INVALID, "provide 1..65535 emission tensors");
  if (!device_descriptors || !valid) return fail(FFA_E_INVALID, "null descriptor or output pointer");
  hipLaunchKernelGGL(ffa::validity_kernel, dim3((unsigned)count), dim3(1024), 0, stream, device_descriptors, valid);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(FFA_E_HIP, std::string("kernel launch failed: ") + hipGetErrorString(err));
  return FFA_OK;
}
