/*
 * CPU oracle for the CTC forced-alignment hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is a plain-C restatement of the
 * reference's alignment algorithm, used by tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg as the checker. Nothing in the product
 * path links or calls it; the GPU path fails loudly without its HIP library.
 *
 * Every function cites the reference code it restates
 * (src/fast_forced_aligner/csrc/alignment.cu, "cu:<line>"; alignment.py, "py:<line>").
 *
 * Parity pins (see tests/test_oracle.py):
 *   - orc_record_status: the exact status vectors of the reference tests.
 *   - conventional DP + traceback: the compiled reference CPU comparator
 *     (benchmarks/patches/cpu_corrected.cpp, same recurrence and tie rule),
 *     golden vectors, exhaustive path enumeration, float64 optima on
 *     integer-valued emissions, and the reference's known-answer cases.
 *   - optimized mode: equality with conventional on non-adversarial inputs,
 *     hand-constructed shortcut / ambiguity / repair / fallback cases whose
 *     diagnostics follow from the rules below. Diagnostics on arbitrary
 *     adversarial inputs have no independent pin ("parity unpinned").
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_EXPORT __attribute__((visibility("default")))

/* Planted-mistake hooks for tests/test_oracle.py: built only into
 * libffa_oracle_mutants.so (-DORC_MUTANTS), never into libffa_oracle.so.
 * MUT(n) is true when mistake n is selected; the pins must reject each one. */
#ifdef ORC_MUTANTS
static int g_mutant = 0;
ORC_EXPORT void orc_set_mutant(int n) { g_mutant = n; }
#define MUT(n) (g_mutant == (n))
#else
#define MUT(n) 0
#endif

typedef struct {
  int64_t chunk_frames;         /* H, py:498 passes 128 */
  int32_t mode;                 /* 0 conventional, 1 chunks without greedy, 2 full (cu:3) */
  int32_t repair_rounds;        /* 0..2 */
  int64_t repair_budget_frames; /* py:499: 512 optimized, 0 conventional */
  int32_t overlap_fallback;
  int64_t repair_min_frames;
  int32_t frontier_reuse;
  int64_t frontier_min_frames;
  int32_t check_inputs;
} orc_options;

typedef struct {
  int32_t stitched, repair_passes;
  int64_t repaired_frames;
  int64_t shortcut[3];
  int32_t routing[3];
  int64_t reuse[4];
  int32_t status;
  float objective;
} orc_diag;

/* ------------------------------------------------------------------------ */
/* Target validation: cu:852-875 (pack_inputs) and py:304-305.               */
/* Returns 0 ok, 2 masked, 3 invalid id, 4 insufficient frames; 3/4 override 2. */
/* Unchecked out-of-vocabulary ids are undefined behaviour in the reference    */
/* (an out-of-bounds read, py:400-402); this build rejects them with 3.        */
ORC_EXPORT int32_t orc_record_status(const int64_t* y, int64_t U, int64_t T, int64_t V,
                                     int64_t blank, int32_t check_inputs, int32_t masked) {
  int32_t status = masked ? 2 : 0; /* cu:836 */
  for (int64_t i = 0; i < U; ++i)
    if (y[i] < 0 || y[i] >= V) return 3;
  if (!check_inputs) return status;
  int64_t invalid = 0, repeats = 0;
  for (int64_t i = 0; i < U; ++i) {
    /* cu:860: range-checked as int64 before any narrowing */
    if (y[i] < 0 || y[i] >= V || y[i] == blank) ++invalid;
    if (i > 0 && y[i] == y[i - 1]) ++repeats; /* cu:861 */
  }
  if (invalid) return 3;           /* cu:872 */
  if (U + repeats > T) return 4;   /* cu:873: S/2 + repeats > T */
  return status;
}

/* ------------------------------------------------------------------------ */
/* Per-record DP context. l is the blank-interleaved label sequence (cu:855-857). */
typedef struct {
  const float* e;
  int64_t T, V;
  const int32_t* l;
  int32_t S, blank;
  uint8_t* bp;    /* [T][S] jumps 0/1/2 */
  int32_t* path;  /* [T] state per frame */
  float* alpha;   /* S */
  float* next;    /* S */
} rec_ctx;

static inline int can_skip(const rec_ctx* c, int32_t s) { /* cu:407, cu:441 */
  return s >= 2 && c->l[s] != c->blank && c->l[s] != c->l[s - 2];
}

/* Viterbi over frames [a, b) of one record: recurrence_impl, cu:355-523.
 * init: relaxed (every state) when a > 0, only s < 2 when a == 0 (cu:409).
 * resume: alpha already holds the frontier at frame start_t - 1 (cu:374-385).
 * record_end selects the S-2/S-1 terminal (cu:497-500); otherwise the lowest-
 * index argmax with the NaN-at-state-0 rule (cu:462-492).
 * Returns the terminal; writes *score, path[a..b) and *start_state when trace. */
static int32_t dp_interval(rec_ctx* c, int64_t a, int64_t b, int resume, int64_t start_t,
                           float* score, int trace, int32_t* start_state) {
  const int32_t S = c->S;
  float* prev = c->alpha;
  float* next = c->next;
  if (!resume) {
    for (int32_t s = 0; s < S; ++s) {
      prev[s] = ((a > 0 && !MUT(1)) || s < 2) ? c->e[a * c->V + c->l[s]] : -INFINITY;
      c->bp[a * S + s] = 0;
    }
    start_t = a + 1;
  }
  for (int64_t t = start_t; t < b; ++t) {
    const float* row = c->e + t * c->V;
    uint8_t* bpr = c->bp + t * S;
    for (int32_t s = 0; s < S; ++s) { /* cu:438-443, strict '>' so ties prefer stay, then advance */
      float best = prev[s];
      uint8_t jump = 0;
      if (s >= 1 && prev[s - 1] > best) { best = prev[s - 1]; jump = 1; }
      if (can_skip(c, s) && prev[s - 2] > best) { best = prev[s - 2]; jump = 2; }
      next[s] = best + row[c->l[s]]; /* one fp32 add, cu:444 */
      bpr[s] = jump;
    }
    float* swap = prev; prev = next; next = swap;
  }
  /* keep alpha pointing at the final row */
  if (prev != c->alpha) { memcpy(c->alpha, prev, sizeof(float) * (size_t)S); }
  prev = c->alpha;
  int32_t terminal;
  if (b == c->T) {
    terminal = S - 1;
    if (S > 1 && prev[S - 2] >= prev[S - 1]) terminal = S - 2;
  } else {
    float best = -INFINITY;
    int32_t state = INT32_MAX;
    for (int32_t s = 0; s < S; ++s)
      if (prev[s] > best || (prev[s] == best && (MUT(2) ? s > state : s < state))) { best = prev[s]; state = s; }
    terminal = isnan(prev[0]) ? 0 : state;
  }
  *score = prev[terminal];
  if (trace) { /* cu:512-520 */
    int32_t s = terminal;
    for (int64_t t = b - 1; t >= a; --t) {
      c->path[t] = s;
      s -= c->bp[t * S + s];
    }
    *start_state = s;
  }
  return terminal;
}

/* Greedy shortcut for one chunk: greedy_shortcuts, cu:30-153.
 * Returns 1 when accepted (writes path states, *start, *end, *objective);
 * sets *ambiguous when more than one legal placement exists (cu:129-133). */
static int greedy_chunk(rec_ctx* c, int64_t a, int64_t b, const uint8_t* alphabet,
                        int32_t* g, float* fs, int32_t* r, int32_t* start, int32_t* end,
                        float* objective, int* ambiguous) {
  *ambiguous = 0;
  int bad = 0;
  for (int64_t t = a; t < b; ++t) { /* cu:65-91: argmax over the transcript alphabet */
    float best = -INFINITY;
    int32_t chosen = -1, count = 0;
    const float* row = c->e + t * c->V;
    for (int64_t v = 0; v < c->V; ++v) {
      if (!alphabet[v]) continue;
      const float score = row[v];
      if (score > best) { best = score; chosen = (int32_t)v; count = 1; }
      else if (score == best) { count = count + 1 > 2 ? 2 : count + 1; }
    }
    g[t - a] = chosen;
    fs[t - a] = best;
    if (!isfinite(best) || count != 1) bad = 1;
  }
  if (bad) return 0;
  r[0] = 0; /* cu:112-117 relative state walk */
  for (int64_t t = a + 1; t < b; ++t) {
    const int32_t x = g[t - a], w = g[t - a - 1];
    r[t - a] = r[t - a - 1] + (x == w ? 0 : (x == c->blank || w == c->blank ? 1 : 2));
  }
  int32_t matches = 0, found = -1;
  for (int32_t s = 0; s < c->S; ++s) { /* cu:119-134 unique legal placement */
    if (c->l[s] != g[0] || (a == 0 && s > 1)) continue;
    const int32_t terminal = s + r[b - 1 - a];
    if (terminal >= c->S || (b == c->T && terminal < c->S - 2)) continue;
    int legal = 1;
    for (int64_t t = a + 1; t < b; ++t) {
      if (g[t - a] != g[t - a - 1] && c->l[s + r[t - a]] != g[t - a]) { legal = 0; break; }
    }
    if (legal) { ++matches; found = s; }
  }
  if (matches != 1) { *ambiguous = matches > 1; return 0; }
  float score = fs[0]; /* cu:135-137: serial fp32 chunk objective */
  for (int64_t t = a + 1; t < b; ++t) score += fs[t - a];
  if (!isfinite(score)) return 0; /* cu:139 */
  *start = found;
  *end = found + r[b - 1 - a];
  *objective = score;
  for (int64_t t = a; t < b; ++t) c->path[t] = found + r[t - a]; /* cu:151-152 */
  return 1;
}

static int legal_seam(const rec_ctx* c, int32_t start, int32_t before) { /* cu:157-161 */
  const int32_t jump = start - before;
  return jump == 0 || jump == 1 ||
         (jump == 2 && (MUT(9) || (c->l[start] != c->blank && c->l[start] != c->l[start - 2])));
}

/* One record through the whole pipeline (launch_alignment, cu:669-815, and
 * finish, cu:642-667). The effective batch-level gates are passed in:
 * budget/overlap are zeroed by the caller when the batch's longest record is
 * shorter than repair_min_frames (cu:993-996), frontier reuse when it is shorter
 * than frontier_min_frames (cu:1002). Returns 0, or -1 on allocation failure. */
static int orc_record(const float* e, int64_t T, int64_t V, const int64_t* y, int64_t U,
                      int64_t blank, int32_t masked, const orc_options* o, int64_t budget,
                      int overlap, int frontier_batch, int64_t* labels, float* scores,
                      orc_diag* d) {
  memset(d, 0, sizeof(*d));
  d->objective = -INFINITY; /* cu:837 */
  d->status = orc_record_status(y, U, T, V, blank, o->check_inputs, masked);
  if (d->status >= 2) { /* rejected before any label-indexed read */
    for (int64_t t = 0; t < T; ++t) { labels[t] = -1; scores[t] = -INFINITY; }
    return 0;
  }
  const int32_t S = (int32_t)(2 * U + 1);
  int rc = -1;
  int32_t* l = malloc(sizeof(int32_t) * (size_t)S);
  float* alpha = malloc(sizeof(float) * (size_t)S);
  float* next = malloc(sizeof(float) * (size_t)S);
  uint8_t* bp = malloc((size_t)T * (size_t)S);
  int32_t* path = malloc(sizeof(int32_t) * (size_t)T);
  const int64_t H = o->chunk_frames;
  const int64_t n = 1 + (T - 1) / H;
  int32_t *ia = NULL, *ib = NULL, *iflag = NULL, *es = NULL, *ee = NULL, *shortcut = NULL;
  int64_t* fend = NULL;
  float *co = NULL, *frontier = NULL;
  int32_t *g = NULL, *r = NULL;
  float* fs = NULL;
  uint8_t* alphabet = NULL;
  if (!l || !alpha || !next || !bp || !path) goto done;
  for (int32_t s = 0; s < S; ++s) l[s] = (s & 1) ? (int32_t)y[s / 2] : (int32_t)blank; /* cu:855-857 */
  rec_ctx c = {e, T, V, l, S, (int32_t)blank, bp, path, alpha, next};
  const int frontier_on = frontier_batch && T >= o->frontier_min_frames; /* cu:374 */
  int32_t terminal = 0;
  int stitched = 0;
  int early = 0; /* routing[0]: 0 ordinary, 1 queued, 2 completed early fallback */

  if (o->mode != 0) {
    ia = malloc(sizeof(int32_t) * (size_t)n); ib = malloc(sizeof(int32_t) * (size_t)n);
    iflag = malloc(sizeof(int32_t) * (size_t)n); es = malloc(sizeof(int32_t) * (size_t)n);
    ee = malloc(sizeof(int32_t) * (size_t)n); shortcut = malloc(sizeof(int32_t) * (size_t)n);
    co = malloc(sizeof(float) * (size_t)n); fend = calloc((size_t)n, sizeof(int64_t));
    g = malloc(sizeof(int32_t) * (size_t)H); r = malloc(sizeof(int32_t) * (size_t)H);
    fs = malloc(sizeof(float) * (size_t)H); alphabet = calloc((size_t)V, 1);
    if (frontier_on) frontier = malloc(sizeof(float) * (size_t)S * (size_t)n);
    if (!ia || !ib || !iflag || !es || !ee || !shortcut || !co || !fend || !g || !r || !fs ||
        !alphabet || (frontier_on && !frontier)) goto done;
    for (int64_t k = 0; k < n; ++k) { /* cu:844-851 */
      ia[k] = (int32_t)(k * H < T ? k * H : T);
      ib[k] = (int32_t)((k + 1) * H < T ? (k + 1) * H : T);
      iflag[k] = 1;
      shortcut[k] = 0;
    }
    for (int32_t s = 0; s < S; ++s) alphabet[l[s]] = 1; /* cu:53-58 */
    if (o->mode == 2) {
      for (int64_t k = 0; k < n; ++k) {
        int amb = 0;
        if (greedy_chunk(&c, ia[k], ib[k], alphabet, g, fs, r, &es[k], &ee[k], &co[k], &amb)) {
          shortcut[k] = 1;
          d->shortcut[0] += 1;
          d->shortcut[1] += ib[k] - ia[k];
        } else if (amb) {
          d->shortcut[2] += 1;
        }
      }
    }
    /* initial chunk DP over non-shortcut chunks (cu:721-726; relaxed init for a > 0) */
    for (int64_t k = 0; k < n; ++k) {
      if (shortcut[k]) continue;
      const int64_t a = ia[k], b = ib[k];
      if (a >= b) continue;
      float score;
      int32_t st;
      ee[k] = dp_interval(&c, a, b, 0, a + 1, &score, 1, &st);
      co[k] = score;
      es[k] = st;
      if (frontier_on) { /* cu:377-383 written-values count, cu:451-454 save */
        d->reuse[2] += S;
        memcpy(frontier + (size_t)k * S, alpha, sizeof(float) * (size_t)S);
        fend[k] = b;
      }
    }
    const int repairs = o->repair_rounds > 0;
    for (int round = 0; round < o->repair_rounds; ++round) {
      /* plan_repairs, cu:164-228 */
      int run_repairs = 1;
      if (overlap && early == 2) run_repairs = 0;
      if (run_repairs && budget > 0 && T >= o->repair_min_frames) {
        int64_t before = -1, begin = 0, maximum_proposed = 0;
        int reject = 0;
        for (int64_t k = 0; k < n; ++k) {
          iflag[k] = 0;
          if (ia[k] >= ib[k]) continue;
          const int join = before < 0 || (isfinite(co[k]) && isfinite(co[before]) &&
                                          legal_seam(&c, es[k], ee[before]));
          if (join) begin = ia[k];
          else {
            if (ib[k] - begin > maximum_proposed) maximum_proposed = ib[k] - begin;
            if (MUT(3) ? maximum_proposed > 2 * budget : maximum_proposed > budget) reject = 1;
          }
          before = k;
        }
        if (reject) {
          d->routing[1] = MUT(4) ? 1 : d->routing[1] + 1;
          if (maximum_proposed > d->routing[2]) d->routing[2] = (int32_t)maximum_proposed;
          if (overlap) early = 1;
          run_repairs = 0;
        }
      }
      if (run_repairs) {
        int64_t previous = -1, group = -1;
        int merged = 0;
        for (int64_t k = 0; k < n; ++k) {
          if (ia[k] >= ib[k]) continue;
          iflag[k] = 0;
          const int join = previous < 0 || (isfinite(co[k]) && isfinite(co[previous]) &&
                                            legal_seam(&c, es[k], ee[MUT(5) ? group : previous]));
          if (join) group = k;
          else {
            ib[group] = ib[k];
            iflag[group] = 1;
            ib[k] = ia[k];
            merged = 1;
          }
          previous = k;
        }
        if (merged) {
          d->repair_passes += 1;
          for (int64_t k = 0; k < n; ++k) if (iflag[k] || MUT(6)) d->repaired_frames += ib[k] - ia[k];
        }
      }
      /* repair DP (cu:727-760); with overlap, a queued record runs the full
       * fallback instead on chunk 0 (repair_recurrence, cu:535-550). */
      if (overlap && early) {
        if (early == 1) {
          int resume = 0;
          int64_t start_t = 1;
          if (frontier_on && fend[0] > 0 && fend[0] <= T) {
            resume = 1; start_t = fend[0];
            memcpy(alpha, frontier, sizeof(float) * (size_t)S);
            d->reuse[1] += fend[0]; d->reuse[3] += S;
            if (MUT(8)) d->reuse[2] += S;
          }
          float score;
          terminal = dp_interval(&c, 0, T, resume, start_t, &score, 0, NULL);
          d->objective = score;
          d->status = isfinite(score) ? 0 : 1;
          early = 2;
        }
      } else {
        for (int64_t k = 0; k < n; ++k) {
          const int64_t a = ia[k], b = ib[k];
          if (a >= b || (repairs && !iflag[k])) continue;
          int resume = 0;
          int64_t start_t = a + 1;
          if (frontier_on) {
            const int64_t saved = fend[k];
            if (saved > a && saved <= b) {
              resume = 1; start_t = saved;
              memcpy(alpha, frontier + (size_t)k * S, sizeof(float) * (size_t)S);
              d->reuse[0] += MUT(7) ? saved : saved - a; d->reuse[3] += S;
            }
            d->reuse[2] += S;
          }
          float score;
          int32_t st;
          ee[k] = dp_interval(&c, a, b, resume, start_t, &score, 1, &st);
          co[k] = score;
          es[k] = st;
          if (frontier_on) {
            memcpy(frontier + (size_t)k * S, alpha, sizeof(float) * (size_t)S);
            fend[k] = b;
          }
        }
      }
    }
    /* validate_seams, cu:562-592 */
    if (!(overlap && early == 2)) {
      int legal = 1;
      float total = 0.0f;
      int64_t previous = -1;
      if (!repairs) { d->repair_passes = 0; d->repaired_frames = 0; }
      for (int64_t k = 0; k < n; ++k) {
        if (repairs && ia[k] >= ib[k]) continue;
        const float cost = co[k];
        legal = legal && isfinite(cost);
        total += cost;
        if (previous >= 0) legal = legal && legal_seam(&c, es[k], ee[previous]);
        previous = k;
      }
      legal = legal && isfinite(total);
      stitched = legal;
      d->status = 0;
      d->objective = total;
    }
  }
  /* full-record DP: conventional mode, or fallback for unstitched records
   * (cu:767-780, fallback_recurrence cu:552-559) */
  if (!stitched && !(overlap && early == 2)) {
    int resume = 0;
    int64_t start_t = 1;
    if (o->mode != 0 && frontier_on && fend[0] > 0 && fend[0] <= T) {
      resume = 1; start_t = fend[0];
      memcpy(alpha, frontier, sizeof(float) * (size_t)S);
      d->reuse[1] += fend[0]; d->reuse[3] += S;
      if (MUT(8)) d->reuse[2] += S;
    }
    float score;
    terminal = dp_interval(&c, 0, T, resume, start_t, &score, 0, NULL);
    d->objective = score;
    d->status = isfinite(score) ? 0 : 1;
  }
  d->stitched = stitched;
  d->routing[0] = early;
  /* finish, cu:642-667 */
  if (d->status != 0) {
    for (int64_t t = 0; t < T; ++t) { labels[t] = -1; scores[t] = -INFINITY; }
  } else {
    if (!stitched) {
      int32_t s = terminal;
      for (int64_t t = T - 1; t >= 0; --t) { path[t] = s; s -= bp[t * S + s]; }
    }
    for (int64_t t = 0; t < T; ++t) {
      const int32_t label = l[path[t]];
      labels[t] = label;
      scores[t] = e[t * V + label];
    }
  }
  rc = 0;
done:
  free(l); free(alpha); free(next); free(bp); free(path);
  free(ia); free(ib); free(iflag); free(es); free(ee); free(shortcut); free(co); free(fend);
  free(frontier); free(g); free(r); free(fs); free(alphabet);
  return rc;
}

/* ------------------------------------------------------------------------ */
/* Batch driver with a thread pool (one record per task, like the reference's
 * CPU comparator lane, benchmarks/adapters/cpp.py:99-117).                  */
typedef struct {
  int64_t count;
  const float* const* e; const int64_t* T; const int64_t* V;
  const int64_t* const* y; const int64_t* U; const int64_t* blank;
  const uint8_t* validity;
  const orc_options* o;
  int64_t budget; int overlap; int frontier;
  const int64_t* offsets;
  int64_t* labels; float* scores;
  int32_t* status; float* objective; int32_t* stitched; int32_t* repair_passes;
  int64_t* repaired_frames; int64_t* shortcut_stats; int32_t* routing_stats; int64_t* reuse_stats;
  int64_t next_index;
  pthread_mutex_t lock;
  int failed;
} batch_job;

static void* batch_worker(void* arg) {
  batch_job* j = arg;
  for (;;) {
    pthread_mutex_lock(&j->lock);
    const int64_t i = j->next_index++;
    pthread_mutex_unlock(&j->lock);
    if (i >= j->count) break;
    orc_diag d;
    const int32_t masked = j->validity ? !j->validity[i] : 0;
    if (orc_record(j->e[i], j->T[i], j->V[i], j->y[i], j->U[i], j->blank[i], masked, j->o,
                   j->budget, j->overlap, j->frontier, j->labels + j->offsets[i],
                   j->scores + j->offsets[i], &d) != 0) {
      pthread_mutex_lock(&j->lock); j->failed = 1; pthread_mutex_unlock(&j->lock);
      continue;
    }
    j->status[i] = d.status; j->objective[i] = d.objective; j->stitched[i] = d.stitched;
    j->repair_passes[i] = d.repair_passes; j->repaired_frames[i] = d.repaired_frames;
    for (int q = 0; q < 3; ++q) { j->shortcut_stats[3 * i + q] = d.shortcut[q]; j->routing_stats[3 * i + q] = d.routing[q]; }
    if (j->reuse_stats) for (int q = 0; q < 4; ++q) j->reuse_stats[4 * i + q] = d.reuse[q];
  }
  return NULL;
}

/* align(), cu:919-1061 for the result-relevant knobs. reuse_stats may be NULL;
 * *reuse_rows receives B when frontier reuse is active for the batch, else 0
 * (cu:1036). Returns 0, -1 on allocation failure. */
ORC_EXPORT int orc_align(int64_t count, const float* const* e, const int64_t* T, const int64_t* V,
                         const int64_t* const* y, const int64_t* U, const int64_t* blank,
                         const uint8_t* validity, const orc_options* o, int32_t threads,
                         int64_t* labels, float* scores, int32_t* status, float* objective,
                         int32_t* stitched, int32_t* repair_passes, int64_t* repaired_frames,
                         int64_t* shortcut_stats, int32_t* routing_stats, int64_t* reuse_stats,
                         int64_t* reuse_rows) {
  int64_t max_frames = 0;
  int64_t* offsets = malloc(sizeof(int64_t) * (size_t)(count + 1));
  if (!offsets) return -1;
  offsets[0] = 0;
  for (int64_t i = 0; i < count; ++i) {
    offsets[i + 1] = offsets[i] + T[i];
    if (T[i] > max_frames) max_frames = T[i];
  }
  batch_job j;
  memset(&j, 0, sizeof(j));
  j.count = count; j.e = e; j.T = T; j.V = V; j.y = y; j.U = U; j.blank = blank;
  j.validity = validity; j.o = o;
  j.budget = o->repair_budget_frames;
  j.overlap = o->overlap_fallback;
  if (max_frames < o->repair_min_frames) { j.budget = 0; j.overlap = 0; } /* cu:993-996 */
  j.frontier = o->frontier_reuse && o->mode != 0 && max_frames >= o->frontier_min_frames; /* cu:935, 1002 */
  if (reuse_rows) *reuse_rows = j.frontier ? count : 0;
  j.offsets = offsets; j.labels = labels; j.scores = scores; j.status = status;
  j.objective = objective; j.stitched = stitched; j.repair_passes = repair_passes;
  j.repaired_frames = repaired_frames; j.shortcut_stats = shortcut_stats;
  j.routing_stats = routing_stats; j.reuse_stats = j.frontier ? reuse_stats : NULL;
  pthread_mutex_init(&j.lock, NULL);
  if (threads < 1) threads = 1;
  if (threads > 256) threads = 256;
  if (threads == 1) batch_worker(&j);
  else {
    pthread_t pool[256];
    int started = 0;
    for (int q = 0; q < threads; ++q)
      if (pthread_create(&pool[q], NULL, batch_worker, &j) == 0) ++started;
    if (!started) batch_worker(&j);
    for (int q = 0; q < started; ++q) pthread_join(pool[q], NULL);
  }
  pthread_mutex_destroy(&j.lock);
  free(offsets);
  return j.failed ? -1 : 0;
}

/* emission_validity_kernel, cu:881-891: false if any NaN or +inf. */
ORC_EXPORT int32_t orc_emission_valid(const float* values, int64_t numel) {
  for (int64_t i = 0; i < numel; ++i) {
    const float v = values[i];
    if (isnan(v) || v == INFINITY) return 0;
  }
  return 1;
}
