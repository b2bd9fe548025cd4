/* orc_sampler.h - CPU restatement of the reference token sampler.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker that tests/, the smoke check and the
 * benchmark's CPU-baseline leg compare the GPU sampler against.  The product library
 * (quasar_amd) never includes, links or calls anything under oracle/.
 *
 * It restates sample.c (franzvill/quasar) from its semantics, function by function:
 *   orc_sampler_new / free / config / reset   sample.c:31-39, 41-45, 47-68, 70
 *   orc_xorshift64, orc_rng_unit              sample.c:72-77, 79-81
 *   orc_record                                sample.c:83-92
 *   orc_pick_row                              sample.c:111-179
 *   orc_router_topk (orc_router.c)            forward_cpu.c:165-172, 296-304
 * using the host C library's expf (sample.c:148) and an explicit (p desc, id asc) order
 * for the sort (sample.c:106-109,151: glibc's qsort is a stable merge sort on an
 * ascending-id array, so equal p keep ascending ids).
 */
#ifndef ORC_SAMPLER_H
#define ORC_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    float   temperature, top_p, min_p, repeat_penalty;
    int32_t top_k, repeat_last_n;
} orc_params;

/* Intermediate values of one pick, for parity reports. */
typedef struct {
    int32_t  id;            /* chosen token */
    int32_t  greedy;        /* 1 when temperature <= 0 */
    int32_t  n_window;      /* candidates inside the 30-nat window */
    int32_t  keep_topk;     /* prefix length after top-k */
    int32_t  keep_topp;     /* ... after top-p */
    int32_t  keep;          /* ... after min-p and the max(.,1) clamp: the sampled prefix */
    int32_t  rank;          /* position of the chosen id in the sorted prefix */
    int32_t  pad;
    float    maxl, msc, inv, p0;
    double   sum;           /* double softmax denominator */
    double   rsum;          /* mass of the kept prefix */
    double   u;             /* uniform draw in [0,1) */
    double   bdist;         /* min over kept j of |u - acc_j / rsum| (CDF boundary distance) */
    uint64_t rng_after;
} orc_diag;

typedef struct orc_sampler orc_sampler;

orc_sampler *orc_sampler_new(void);
void         orc_sampler_free(orc_sampler *s);
void         orc_sampler_config(orc_sampler *s, float temperature, float top_p, int top_k,
                                float min_p, float repeat_penalty, int repeat_last_n,
                                uint64_t seed);
void         orc_sampler_reset(orc_sampler *s);
int          orc_sampler_pick(orc_sampler *s, const float *logits, int n_vocab);

/* Test hooks: the workloads start with a preloaded history (ids in ring order, oldest
 * first; the ring keeps the newest repeat_last_n of them), which the five-function API
 * cannot express.  Also read back the state. */
void     orc_sampler_set_history(orc_sampler *s, const int32_t *ids, int n);
int      orc_sampler_get_history(const orc_sampler *s, int32_t *out, int cap);
uint64_t orc_sampler_get_rng(const orc_sampler *s);
/* Stored parameters: f = {temperature, top_p, min_p, repeat_penalty},
 * i = {top_k, repeat_last_n, ring capacity}. */
void     orc_sampler_get_params(const orc_sampler *s, float *f, int32_t *i);
void     orc_sampler_set_rng(orc_sampler *s, uint64_t rng);
/* Test hook: while on, every pick finds its scratch unavailable and takes the
 * out-of-memory branch (sample.c:113-116); the reference reaches it only when the scratch
 * must grow, which the checks against it arrange. */
void     orc_sampler_fail_scratch(orc_sampler *s, int on);
int      orc_sampler_pick_diag(orc_sampler *s, const float *logits, int n_vocab, orc_diag *d);

/* xorshift64* step and the uniform built from it (sample.c:72-81). */
uint64_t orc_xorshift64(uint64_t *state);
double   orc_rng_unit(uint64_t *state);

/* Batch driver for the CPU baseline: rows [0, n_rows) of a row-major batch, one sampler
 * per row configured from `p` with seeds[r] and history hist[r * hist_n .. + hist_n),
 * picked once each, on `n_threads` POSIX threads.  Returns wall seconds spent inside
 * the pick calls (configuration excluded), ids in out[r]. */
double orc_pick_rows(const orc_params *p, const float *logits, long row_stride, int n_rows,
                     int n_vocab, const int32_t *hist, int hist_n, const uint64_t *seeds,
                     int32_t *out, int n_threads);
/* The same with each row's intermediate values (diag[n_rows]). */
double orc_pick_rows_diag(const orc_params *p, const float *logits, long row_stride,
                          int n_rows, int n_vocab, const int32_t *hist, int hist_n,
                          const uint64_t *seeds, int32_t *out, orc_diag *diag, int n_threads);

/* Portable generator (same code as the GPU's), for tests. */
void orc_gen_logits(int32_t dist, float sigma, float boost, uint64_t seed, long row0,
                    int n_rows, int n_vocab, float *out, long row_stride);
void orc_gen_hist(uint64_t seed, long row0, int n_rows, int hist_n, int n_vocab, int pool,
                  int32_t *out);
uint64_t orc_gen_row_seed(uint64_t seed, long row);

/* The product's libm-compatible expf, compiled for the host (checked against expf). */
float orc_product_expf(float x);
/* y[i] = host C library expf(x[i]). */
void  orc_libm_expf_array(const float *x, float *y, long n);
/* Count x in [lo, hi] (by float ordering, both finite) where the product expf differs
 * from the host expf; n_threads POSIX threads. */
long  orc_check_expf_range(float lo, float hi, int n_threads);

/* forward_cpu.c:165-172, 296-304: the mixture-of-experts router's choice per token
 * (orc_router.c): idx/wt hold n_used slots per token. */
void orc_router_topk(const float *logits, long row_stride, int n_tokens, int n_expert,
                     int n_used, int norm_topk, int32_t *idx, float *wt);
/* One row's softmax (forward_cpu.c:165-172) and the float sum of its numerators. */
void orc_router_probs(const float *x, int n, float *p, float *sum_out);

/* The output layer (orc_head.c): forward_cpu.c:140-147 over weights of the reference's
 * GGUF types (ggml numbering) as quant.c dequantizes them. */
enum { ORC_W_F32 = 0, ORC_W_F16 = 1, ORC_W_Q8_0 = 8, ORC_W_Q6_K = 14 };
long orc_head_row_bytes(int type, int n);
void orc_dequant_row(int type, const uint8_t *src, float *dst, int n);
void orc_head_gemv(int type, const uint8_t *w, const float *x, int nx, int E, int V,
                   float *y, int n_threads);

#ifdef __cplusplus
}
#endif

#endif /* ORC_SAMPLER_H */
