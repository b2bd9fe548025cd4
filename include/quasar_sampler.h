/* quasar_sampler.h - MI355X (gfx950) token sampler, C ABI.
 *
 * Part 1 is the reference's sample.h surface, unchanged: the same five symbols with the
 * same argument meaning, so the reference's server.o / quasar.o link against this
 * library instead of sample.o (reference Makefile:17-18 object list).  The work runs on
 * the GPU; `logits` stays a host pointer, copied in per call.
 *
 * Part 2 is the extension the reference does not have: a batch of rows whose logits,
 * generator states and histories live in device memory, picked in one enqueue.
 *
 * Part 3 is plumbing for callers without their own GPU runtime (tests, the benchmark):
 * device buffers, copies, the synthetic-input generator and event timing.
 *
 * Part 4 is the mixture-of-experts router's expert choice, the same selection at 128
 * experts per token (the reference's forward_cpu.c:296-304).
 *
 * Part 5 is the output layer (forward_cpu.c:319-323) on the matrix cores with the
 * sampler's first pass in its epilogue, and the pick of every row from it.
 *
 * Return codes of the extension functions: 0 on success, QS_EINVAL for bad arguments,
 * QS_ENOMEM when device memory cannot be allocated, QS_EAGAIN (qs_batch_synchronize only)
 * when rows must be picked again, QS_EDEVICE for any other HIP failure; qs_last_error()
 * describes the last failure on the calling thread.
 */
#ifndef QUASAR_SAMPLER_H
#define QUASAR_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------------------
 * Part 1: sample.h (reference sample.h:12-29)
 * ------------------------------------------------------------------------------------ */

typedef struct quasar_sampler quasar_sampler;

/* Replaces sample.h:14 (sample.c:31-39).  Defaults: greedy (temperature 0), top_p 1,
 * top_k 0, min_p 0, repeat_penalty 1, repeat_last_n 0, generator state
 * 0x9E3779B97F4A7C15.  NULL when host memory is exhausted. */
quasar_sampler *quasar_sampler_new(void);

/* Replaces sample.h:15 (sample.c:41-45).  NULL-safe. */
void quasar_sampler_free(quasar_sampler *s);

/* Replaces sample.h:19-22 (sample.c:47-68).  Disable values: top_p outside (0,1) -> 1,
 * top_k <= 0 -> 0, min_p <= 0 -> 0, repeat_penalty <= 1 -> 1, repeat_last_n <= 0 -> 0.
 * temperature <= 0 forces greedy.  seed 0 -> time-seeded.  Empties the history. */
void quasar_sampler_config(quasar_sampler *s, float temperature, float top_p, int top_k,
                           float min_p, float repeat_penalty, int repeat_last_n,
                           uint64_t seed);

/* Replaces sample.h:25 (sample.c:70).  Forgets the history; keeps the generator state. */
void quasar_sampler_reset(quasar_sampler *s);

/* Replaces sample.h:29 (sample.c:111-179).  Picks the next token from the host array
 * logits[n_vocab] (not modified) and records it in the history.  Returns 0 when
 * n_vocab <= 0 (no record).  Never fails, as in the reference: where sample.c:113-115
 * answers an allocation failure with the argmax of the raw logits (first index of the
 * largest, no penalty, generator untouched) and records it, this pick does the same when
 * the device cannot take it (no device memory, no GPU, a device error), printing one line
 * to stderr for the sampler's first such pick. */
int quasar_sampler_pick(quasar_sampler *s, const float *logits, int n_vocab);

/* Extension (no counterpart in sample.h): the sampler's generator state and the last
 * min(hist_cap, history length) ids of its history, oldest first, into hist.  For tests
 * and for callers that checkpoint a sequence. */
int qs_sampler_get_state(const quasar_sampler *s, uint64_t *rng, int32_t *hist, int hist_cap,
                         int *hist_len);

/* Extension for tests (no counterpart in sample.h): the next n calls of
 * quasar_sampler_pick (process-wide) find the device unavailable, as on an allocation
 * failure.  0, or QS_EINVAL for n < 0. */
int qs_debug_fail_picks(int n);

/* ------------------------------------------------------------------------------------
 * Part 2: device-resident batch (extension)
 * ------------------------------------------------------------------------------------ */

#define QS_EINVAL  (-22)
#define QS_ENOMEM  (-12)
#define QS_EDEVICE (-5)
#define QS_EAGAIN  (-11)   /* qs_batch_synchronize: some rows could not take a whole-window
                              scratch slot in time; they returned -3 and kept their state */

typedef struct qs_batch qs_batch;

/* Per-row report of one pick (optional output of qs_batch_pick). */
typedef struct {
    int32_t id;          /* chosen token */
    int32_t path;        /* QS_PATH_*: how the row was decided */
    int32_t n_window;    /* ids inside the 30-nat window of the max scaled logit (-1: not
                            counted, QS_PATH_CERT rows whose window is partly preselected) */
    int32_t n_cand;      /* candidates whose exact numerator was computed */
    int32_t keep_topk;   /* prefix length after top-k */
    int32_t keep_topp;   /* ... after top-p */
    int32_t keep;        /* sampled prefix (after min-p, at least 1) */
    int32_t rank;        /* position of the chosen id in the (p desc, id asc) order */
    float   maxl;        /* max penalised logit */
    float   msc;         /* maxl / temperature */
    float   inv;         /* (float)(1 / sum), the softmax normaliser; QS_PATH_CERT: the
                            smallest value the proof allows */
    float   inv_hi;      /* the largest value it allows (== inv on the exact paths) */
    float   p0;          /* top probability (at inv) */
    int32_t fallback;    /* why a row of the streaming kernel left the certified decision
                            for the exact path (0: it did not; see qs_cert.h CF_*) */
    double  sum;         /* softmax denominator (double); QS_PATH_CERT: its lower bound */
    double  sum_hi;      /* its upper bound (== sum on the exact paths) */
    double  rsum;        /* mass of the sampled prefix (double, at inv) */
    double  u;           /* uniform draw */
} qs_pick_diag;

enum {
    QS_PATH_GREEDY = 0,  /* temperature <= 0: argmax, no draw */
    QS_PATH_FAST = 1,    /* exact softmax denominator, top candidates preselected by logit,
                            exact order proven */
    QS_PATH_FULL = 2,    /* whole window sorted on the device (large nucleus, ties across
                            the preselection boundary, non-finite maxima) */
    QS_PATH_EMPTY = 3,   /* empty window (temperature NaN or 1/T overflowing on a zero
                            max): id 0, as documented in quasar_sampler_pick */
    QS_PATH_CERT = 4     /* the streaming kernel's path: the denominator bounded to an
                            interval, the cuts and the draw proved identical for every
                            normaliser the interval allows */
};

/* A batch of up to max_rows rows of width up to max_vocab, each with a history ring of
 * up to max_last_n ids.  Every row starts as quasar_sampler_new() would. */
qs_batch *qs_batch_new(int max_rows, int max_vocab, int max_last_n);
void      qs_batch_free(qs_batch *b);

/* quasar_sampler_config applied to rows [row0, row0 + n_rows), row r seeded with
 * seeds[r - row0] (seeds may be NULL: all rows seeded with 0, i.e. time-seeded).
 * repeat_last_n above max_last_n is QS_EINVAL. */
int qs_batch_config(qs_batch *b, int row0, int n_rows, float temperature, float top_p,
                    int top_k, float min_p, float repeat_penalty, int repeat_last_n,
                    const uint64_t *seeds);

/* quasar_sampler_reset for rows [row0, row0 + n_rows). */
int qs_batch_reset(qs_batch *b, int row0, int n_rows);

/* Preload histories: row r receives ids[(r - row0) * n_per_row ...] in order, oldest
 * first, as if each had been picked (the ring keeps the newest repeat_last_n).  The
 * workloads start from such histories; sample.h cannot express them. */
int qs_batch_set_history(qs_batch *b, int row0, int n_rows, const int32_t *ids,
                         int n_per_row);

/* Pick one token for each of rows [0, n_rows) from device logits d_logits[r*row_stride
 * + i], i < n_vocab (row_stride >= n_vocab; a 16-byte-aligned base and a stride that is
 * a multiple of 4 take the vector path).  Writes d_out[r] (device) and, when d_diag is
 * not NULL, d_diag[r] (device).  Updates each row's generator state and history on the
 * device.  Asynchronous on the batch's stream. */
int qs_batch_pick(qs_batch *b, const float *d_logits, int64_t row_stride, int n_rows,
                  int n_vocab, int32_t *d_out, qs_pick_diag *d_diag);

/* qs_batch_pick for the batch's rows [row0, row0 + n_rows) from logits rows 0 .. n_rows - 1
 * of d_logits, ids and diagnostics at d_out[0 ..], d_diag[0 ..]: only those rows' states
 * change.  The retry of rows a pick left at -3 (QS_EAGAIN): pick each again alone, e.g.
 * row r with row0 = r, n_rows = 1 and its own logits row. */
int qs_batch_pick_rows(qs_batch *b, int row0, const float *d_logits, int64_t row_stride,
                       int n_rows, int n_vocab, int32_t *d_out, qs_pick_diag *d_diag);

/* Which kernels qs_batch_pick uses.  AUTO (the default) takes the row kernel for batches
 * of at least one row per CU whose sampling rows have a top-k of at most 256 (or top-k
 * off), the streaming kernels for smaller batches and larger top-k, and the split-row
 * kernels for rows neither supports.  ROW: one kernel, one workgroup per row,
 * every logit read once and the row decided from LDS (16-byte aligned rows, a vocabulary
 * and a row stride that are multiples of 4, vocabulary up to 262,144).  STREAM: two
 * kernels, every logit read once by workgroups that each take a part of a row, then one
 * decision workgroup per row (the same alignment, vocabulary up to 655,360).  SPLIT:
 * three kernels per pick, the logits streamed twice (any layout).  A mode that does not
 * support a pick returns QS_EINVAL.  The results are identical. */
enum { QS_MODE_AUTO = 0, QS_MODE_SPLIT = 1, QS_MODE_STREAM = 2, QS_MODE_ROW = 3 };
int qs_batch_set_mode(qs_batch *b, int mode);
/* The QS_MODE_* (SPLIT, STREAM or ROW) a qs_batch_pick with these arguments would use;
 * QS_EINVAL for arguments it would reject. */
int qs_batch_resolve_mode(qs_batch *b, const float *d_logits, int64_t row_stride, int n_rows,
                          int n_vocab);

/* Set one row's generator state and history exactly (oldest first), e.g. to carry a
 * sampler's state into a larger batch. */
int qs_batch_set_state(qs_batch *b, int row, uint64_t rng, const int32_t *hist, int n);

/* Wait for everything enqueued on the batch's stream.  Device-side failures of the picks
 * enqueued since the last call surface here: QS_EAGAIN when a row that needed a
 * whole-window scratch slot (a rare fallback; the batch has a few, shared by its rows)
 * could not take one within the wait limit.  Such a row's id is -3 and its generator state
 * and history are unchanged, so picking it again (qs_batch_pick_rows, that row alone: the
 * other rows' states have advanced) gives the reference's result. */
int qs_batch_synchronize(qs_batch *b);

/* Read one row's generator state and history (oldest first; up to cap ids). */
int qs_batch_get_state(qs_batch *b, int row, uint64_t *rng, int32_t *hist, int cap,
                       int *hist_len);

/* The batch's HIP stream (hipStream_t), for callers that order their own work on it. */
void *qs_batch_stream(qs_batch *b);

/* Message of the last failure on the calling thread ("" if none). */
const char *qs_last_error(void);

/* ------------------------------------------------------------------------------------
 * Part 2b: a pick that allocates nothing (extension)
 * ------------------------------------------------------------------------------------ */

/* One row's sampling parameters as the device reads them (qs_row_config_set fills it). */
typedef struct {
    float   temperature, top_p, min_p, repeat_penalty;
    int32_t top_k;
    int32_t ring_cap;      /* history ring capacity (repeat_last_n after the clamp) */
    float   inv_t;         /* 1.0f / temperature, or 0 for greedy rows */
    int32_t pad;
} qs_row_config;

/* quasar_sampler_config's clamps into a qs_row_config (host memory; no generator state:
 * the caller owns the rows' states).  A fresh ring has capacity repeat_last_n clamped. */
void qs_row_config_set(qs_row_config *c, float temperature, float top_p, int top_k,
                       float min_p, float repeat_penalty, int repeat_last_n);

/* Largest work qs_pick_noalloc takes: rows x parts (a part is 10,240 logits), vocabulary,
 * and the rows that can be on the whole-window fallback at once; QS_NOALLOC_SCRATCH_BYTES
 * is the static device array each GPU the library runs on holds until the process ends. */
#define QS_NOALLOC_MAX_PARTS 4096
#define QS_NOALLOC_MAX_VOCAB 262144
#define QS_NOALLOC_SLOTS 4
#define QS_NOALLOC_SCRATCH_BYTES 26345984

/* No counterpart in the reference (its sampler allocates its scratch, sample.c:94-104):
 * qs_batch_pick for callers that cannot allocate (HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  Picks rows [0, n_rows) of d_logits (device memory,
 * 16-byte aligned, n_vocab and row_stride multiples of 4) with every row's state in the
 * caller's device buffers: d_config[n_rows], d_rng[n_rows] (xorshift64 states, nonzero),
 * the history ring d_ring[row * ring_stride + slot] with d_hist_len[row] valid slots from
 * d_hist_head[row] (capacity d_config[row].ring_cap <= ring_stride), all updated as the
 * reference updates them; ids to d_out[n_rows].  Enqueued on `stream` (a hipStream_t;
 * NULL: the null stream).  Its scratch is the library's static device array: no
 * allocation, and calls that overlap on one GPU race (order them).  QS_EINVAL beyond the
 * limits above or for an unaligned pick.  A row whose whole-window fallback found no free
 * slot in time gets id -3 with its state unchanged: pick it again. */
int qs_pick_noalloc(const float *d_logits, int64_t row_stride, int n_rows, int n_vocab,
                    const qs_row_config *d_config, uint64_t *d_rng, int32_t *d_ring,
                    int ring_stride, int32_t *d_hist_len, int32_t *d_hist_head,
                    int32_t *d_out, void *stream);

/* ------------------------------------------------------------------------------------
 * Part 3: plumbing for tests and the benchmark
 * ------------------------------------------------------------------------------------ */

void *qs_device_alloc(size_t bytes);          /* NULL on failure */
void  qs_device_free(void *p);
int   qs_memcpy_h2d(void *d_dst, const void *src, size_t bytes);
int   qs_memcpy_d2h(void *dst, const void *d_src, size_t bytes);
int   qs_device_synchronize(void);
/* Name and global memory size of the current device; QS_EDEVICE when there is none. */
int   qs_device_info(char *name, int name_cap, size_t *total_mem, int *n_cu);

/* The synthetic workloads' per-row sampler seeds (never 0) and history ids (row-major,
 * hist_n per row; uniform over [0, n_vocab), or drawn from a per-row pool of `pool` ids
 * when pool > 0), from the generator qs_gen_logits_device uses.  Host only. */
int qs_gen_row_seeds(uint64_t seed, int64_t row0, int n_rows, uint64_t *out);
int qs_gen_history(uint64_t seed, int64_t row0, int n_rows, int hist_n, int n_vocab, int pool,
                   int32_t *out);

/* Fill rows [row0, row0 + n_rows) of the synthetic workload distribution `dist`
 * (0 normal, 1 normal plus a boosted column, 2 Student-t with 3 degrees of freedom) into
 * d_out[(r - row0) * row_stride + i] on the device.  Bit-identical to the host build of
 * the same generator. */
int qs_gen_logits_device(float *d_out, int64_t row_stride, int64_t row0, int n_rows,
                         int n_vocab, int dist, float sigma, float boost, uint64_t seed);

/* Attempts a row makes at a whole-window scratch slot before giving up (default about
 * a million, half a second): a test hook that forces the QS_EAGAIN path with 0. */
int qs_batch_set_spin_limit(qs_batch *b, int attempts);

/* Rows that leave the certified decision recount their softmax denominator with the
 * reference's numerators in a fixed order, and again in id order as sample.c adds them
 * wherever the two orders' rounding could reach a different float normaliser.  With
 * always = 1 every such row is summed in id order (a test hook: the recount's sum then
 * equals the reference's bit for bit); 0, the default, only where needed. */
int qs_batch_set_sum_in_order(qs_batch *b, int always);

/* `iters` plain streaming copies of `bytes` (a multiple of 16, 16-byte aligned) from
 * d_src to d_dst, then a device synchronization: a kernel of known memory traffic for
 * calibrating hardware memory counters. */
int qs_copy_device(void *d_dst, const void *d_src, size_t bytes, int iters);
/* The same copies with another load instruction: kind 0 plain global loads (as
 * qs_copy_device), 1 raw buffer loads of 16 bytes, nontemporal (the row kernel's), 2 those
 * loads written straight into LDS (the streaming part kernel's), 3 plain loads of 4 bytes.
 * Counters that count a load kind differently are calibrated against the copy of that
 * kind. */
int qs_copy_device_kind(void *d_dst, const void *d_src, size_t bytes, int iters, int kind);

/* The row pick's loads alone: `iters` back-to-back launches on the null stream, launch i
 * reading d_logits[i % n_buffers] (n_rows rows of n_vocab floats, row_stride apart, as
 * qs_batch_pick takes them) with the row kernel's launch shape at one row per CU (one
 * workgroup of 16 wavefronts per row), its chunks and its load instruction (raw 16-byte
 * nontemporal buffer loads, two chunks in flight a wavefront), adding up each row's floats
 * and nothing else.  *ms: the elapsed milliseconds of all launches (HIP events).  The
 * same bytes read at the same shape without the sampling: the ceiling a row pick's time is
 * compared with.  d_sink: n_rows floats, written only for a sum no finite row reaches.
 * Needs 16-byte aligned rows, n_vocab and row_stride multiples of 4 (QS_EINVAL otherwise).
 * No counterpart in the reference: a measurement aid. */
int qs_time_row_reads(const float *const *d_logits, int n_buffers, int64_t row_stride,
                      int n_rows, int n_vocab, float *d_sink, int iters, float *ms);

/* y[i] = the library's expf(x[i]) on the device, i < n (the softmax numerator routine,
 * exposed so tests can compare it with the host C library's expf). */
int qs_expf_device(const float *d_x, float *d_y, int64_t n);

/* Enqueue `iters` back-to-back qs_batch_pick calls between two HIP events recorded on the
 * batch's stream, wait, and return the elapsed milliseconds in *ms.  Pick i reads
 * d_logits[i % n_buffers]: rotating over buffers whose total exceeds the GPU's
 * last-level cache keeps every pick's input in HBM only. */
int qs_batch_time_picks(qs_batch *b, const float *const *d_logits, int n_buffers,
                        int64_t row_stride, int n_rows, int n_vocab, int32_t *d_out, int iters,
                        float *ms);

/* The same picks with an event before each and one after its dominant kernel: *ms_stream
 * is the summed time from each pick's start to the end of its streaming kernel (k_part)
 * when the pick takes the streaming kernels, or to the end of the pick (its one kernel,
 * k_row) when it takes the row kernel.  QS_EINVAL when it takes neither. */
int qs_batch_time_kernels(qs_batch *b, const float *const *d_logits, int n_buffers,
                          int64_t row_stride, int n_rows, int n_vocab, int32_t *d_out,
                          int iters, float *ms_stream);

/* Workgroups of the row kernel with `waves` wavefronts (16 or 8) one CU of the current
 * device holds at once: 1 and 2 by design (registers and LDS), so that a row per CU takes
 * the chip in one wave of workgroups and, beyond 1.5 rows per CU, one row decides while
 * the other streams.  0 when the runtime cannot tell. */
int qs_row_workgroups_per_cu(int waves);

/* The timeline build's clocks (make -C quasar_amd/csrc timeline; quasar_amd/timeline.py):
 * which 0 = the streaming kernel's per-wavefront phase stamps, 1 = the decision kernel's
 * per-row stamps, 2 = the row kernel's per-wavefront stamps, n entries.  QS_EINVAL in the
 * ordinary build. */
int qs_timeline_read(int which, uint64_t *dst, int n);

/* ------------------------------------------------------------------------------------
 * Part 4: the mixture-of-experts router's expert choice (extension)
 *
 * Replaces forward_cpu.c:296-304 (softmax of the router logits, forward_cpu.c:165-172,
 * then n_used strict-`>` arg-max scans, then the optional renormalisation), for a batch
 * of tokens whose router logits are on the device.  No counterpart in sample.h: the
 * reference runs it inline in its CPU forward pass.
 * ------------------------------------------------------------------------------------ */

/* For each token t < n_tokens, from d_logits[t*row_stride + e], e < n_expert: the
 * softmax p (libm-equal expf, the reference's sequential float sum), then the n_used
 * experts of largest p (lowest index among equal p; never a NaN) into
 * d_idx[t*n_used + s] and their p into d_wt[t*n_used + s], slot s in choice order; with
 * norm_topk != 0 the weights are divided by their sequential sum when it is positive.
 * Bit-identical to the reference.  A slot left with nothing to take (every remaining p
 * NaN, where the reference reads index -1) gets expert -1 and weight 0.
 * 1 <= n_expert <= 256, 1 <= n_used <= min(64, n_expert), row_stride >= n_expert (the
 * reference's array bounds).  Asynchronous on `stream` (a hipStream_t; NULL for the
 * default stream). */
int qs_router_topk(const float *d_logits, int64_t row_stride, int n_tokens, int n_expert,
                   int n_used, int norm_topk, int32_t *d_idx, float *d_wt, void *stream);

/* Enqueue `iters` back-to-back qs_router_topk calls between two HIP events on a stream of
 * its own, wait, and return the elapsed milliseconds in *ms (plumbing for the
 * benchmark). */
int qs_router_time(const float *d_logits, int64_t row_stride, int n_tokens, int n_expert,
                   int n_used, int norm_topk, int32_t *d_idx, float *d_wt, int iters,
                   float *ms);

/* ------------------------------------------------------------------------------------
 * Part 5: the output layer with the sampler's first pass (extension)
 *
 * The logits' producer is the output layer: logits = W . xn, W the n_vocab x n_embd
 * output matrix and xn the final normed hidden state (forward_cpu.c:319-323,
 * metal.m:848-851).  For a batch of rows decoded together these compute the layer on the
 * matrix cores (bf16 operands: d_hidden[n_rows][n_embd] and d_weight[n_vocab][n_embd],
 * row-major, as bf16 bit patterns; fp32 accumulation) and take the sampler's first pass
 * over each tile of logits while it is in registers, so that a pick reads back only the
 * tiles that hold its candidates instead of the whole row.
 * ------------------------------------------------------------------------------------ */

/* The output matrix is read in a tile order of its own, made once (at model load) from the
 * row-major d_weight[n_vocab][n_embd]: qs_head_packed_bytes(n_embd, n_vocab) bytes (the
 * vocabulary rounded up to a multiple of 128; 0 for sizes the output layer does not take)
 * at d_packed, written asynchronously on the batch's stream by qs_batch_head_pack.  Each
 * weight row is then read as contiguous 1 KB pieces instead of 64 bytes per row per step. */
size_t qs_head_packed_bytes(int n_embd, int n_vocab);
int qs_batch_head_pack(qs_batch *b, const void *d_weight, int n_embd, int n_vocab,
                       void *d_packed);

/* The output layer alone: d_logits[r * n_vocab + v] = sum_k hidden[r][k] * weight[v][k],
 * d_packed the packed weight matrix.  1 <= n_rows <= min(max_rows, 256), n_vocab a multiple
 * of 4 up to min(max_vocab, 262,144), n_embd a multiple of 64, 16-byte aligned buffers.
 * Asynchronous on the batch's stream. */
int qs_batch_head_logits(qs_batch *b, const void *d_hidden, const void *d_packed, int n_embd,
                         int n_rows, int n_vocab, float *d_logits);

/* The output layer and the pick of rows [0, n_rows) from its logits in one enqueue: the
 * same ids, generator states and histories as qs_batch_head_logits followed by
 * qs_batch_pick on d_logits (which it also writes: the rows the certified decision does
 * not cover are recounted from them).  Limits as qs_batch_head_logits. */
int qs_batch_pick_head(qs_batch *b, const void *d_hidden, const void *d_packed, int n_embd,
                       int n_rows, int n_vocab, float *d_logits, int32_t *d_out,
                       qs_pick_diag *d_diag);

/* `iters` back-to-back output-layer calls between two HIP events on the batch's stream:
 * fused = 1, picks by qs_batch_pick_head; 0, qs_batch_head_logits then qs_batch_pick; 2,
 * qs_batch_head_logits alone.  Waits and returns the elapsed milliseconds in *ms
 * (plumbing for the benchmark). */
int qs_batch_time_head(qs_batch *b, const void *d_hidden, const void *d_packed, int n_embd,
                       int n_rows, int n_vocab, float *d_logits, int32_t *d_out, int iters,
                       int fused, float *ms);

/* ------------------------------------------------------------------------------------
 * Part 5b: the output layer at the reference's own arithmetic (extension)
 *
 * Replaces forward_cpu.c:140-147 (gemv) for the output matrix, forward_cpu.c:321-322:
 * logits[r][v] = the float sum over k ascending of w[v][k] * xn[r][k], a product then a
 * sum, with w[v] the GGUF row dequantized exactly as quasar_dequant_row does (quant.c:
 * F32, F16, Q8_0 and Q6_K rows; Q6_K is the output matrix of the reference's model).  Every
 * logit equals the reference's bit for bit (NaN payloads aside).  For the few rows a
 * decoding step produces (the reference decodes one): one thread per vocabulary row keeps
 * the reference's order, so the cost grows with the rows; larger batches take part 5.
 * ------------------------------------------------------------------------------------ */

/* GGUF tensor types taken (ggml's type numbers, as gguf.h numbers them). */
#define QS_WTYPE_F32  0
#define QS_WTYPE_F16  1
#define QS_WTYPE_Q8_0 8
#define QS_WTYPE_Q6_K 14
#define QS_HEAD_EXACT_MAX_ROWS 8
#define QS_HEAD_EXACT_MAX_EMBD 16384   /* n_rows * n_embd at most this (64 KB of LDS) */

/* The output matrix is read in an interleaved layout of its own, made once (at model load)
 * from the n_vocab GGUF rows at d_weight (device memory, the file's bytes: row v at
 * v * row_bytes): qs_head_exact_packed_bytes bytes at d_packed (16-byte aligned; 0 for a
 * type or n_embd not taken: F32 and F16 need n_embd a multiple of 16, Q8_0 of 32, Q6_K of
 * 256), written asynchronously on the batch's stream by qs_batch_head_exact_pack. */
size_t qs_head_exact_packed_bytes(int wtype, int n_embd, int n_vocab);
int qs_batch_head_exact_pack(qs_batch *b, int wtype, const void *d_weight, int n_embd,
                             int n_vocab, void *d_packed);

/* The output layer alone: d_logits[r * n_vocab + v] from d_xn[r * n_embd + k] (fp32),
 * 1 <= n_rows <= min(max_rows, QS_HEAD_EXACT_MAX_ROWS), n_rows * n_embd at most
 * QS_HEAD_EXACT_MAX_EMBD, n_vocab a multiple of 4 up to min(max_vocab, 262,144), d_xn and
 * d_logits 16-byte aligned.  Asynchronous on the batch's stream. */
int qs_batch_head_exact_logits(qs_batch *b, int wtype, const void *d_packed,
                               const float *d_xn, int n_embd, int n_rows, int n_vocab,
                               float *d_logits);

/* The output layer and the pick of rows [0, n_rows) from its logits in one enqueue (the
 * sampler's first pass taken per tile of 128 logits as they are computed; the decision
 * reads back only the tiles that hold its candidates): the same ids, generator states and
 * histories as qs_batch_head_exact_logits followed by qs_batch_pick on d_logits, which it
 * also writes.  Limits as qs_batch_head_exact_logits. */
int qs_batch_pick_head_exact(qs_batch *b, int wtype, const void *d_packed, const float *d_xn,
                             int n_embd, int n_rows, int n_vocab, float *d_logits,
                             int32_t *d_out, qs_pick_diag *d_diag);

/* `iters` back-to-back calls between two HIP events on the batch's stream: fused = 1,
 * qs_batch_pick_head_exact; 0, qs_batch_head_exact_logits then qs_batch_pick; 2,
 * qs_batch_head_exact_logits alone.  Waits; the elapsed milliseconds in *ms (plumbing for
 * the benchmark). */
int qs_batch_time_head_exact(qs_batch *b, int wtype, const void *d_packed, const float *d_xn,
                             int n_embd, int n_rows, int n_vocab, float *d_logits,
                             int32_t *d_out, int iters, int fused, float *ms);

#ifdef __cplusplus
}
#endif

#endif /* QUASAR_SAMPLER_H */
