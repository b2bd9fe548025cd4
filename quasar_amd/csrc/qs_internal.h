/* qs_internal.h - declarations shared by the C host layer and the HIP layer. */
#ifndef QS_INTERNAL_H
#define QS_INTERNAL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One row's stored sampling parameters, as laid out on the device.  The first six
 * fields are the values sample.c keeps after its clamps (sample.c:47-56); inv_t is
 * 1.0f / temperature, computed once on the host in IEEE single precision exactly as
 * sample.c:137 does per pick. */
typedef struct {
    float   temperature;
    float   top_p;
    float   min_p;
    float   repeat_penalty;
    int32_t top_k;
    int32_t ring_cap;        /* repeat_last_n after the clamp: history ring capacity */
    float   inv_t;
    int32_t pad;
} qs_row_param;

/* sample.c:47-66: clamp the arguments to their disable values and derive the generator
 * state (seed 0 means time-seeded; a zero state becomes the default constant).  The
 * history ring is re-sized only for repeat_last_n > 0 (sample.c:61-66): with 0 the row
 * keeps prev_cap, its current ring capacity, and goes on recording into it. */
void qs_clamp_config(float temperature, float top_p, int top_k, float min_p,
                     float repeat_penalty, int repeat_last_n, uint64_t seed, int prev_cap,
                     qs_row_param *out, uint64_t *rng_out);

/* The state quasar_sampler_new starts from (sample.c:31-39). */
void qs_default_param(qs_row_param *out, uint64_t *rng_out);

/* Fault injection for tests: nonzero while injected device failures remain (each call
 * consumes one); see qs_debug_fail_picks. */
int qs_debug_take_failure(void);

/* sample.h's pick of one row in one round trip: the host row copied to d_logits on the
 * batch's stream, the pick of row 0, its id and the batch's error flag copied back into
 * pinned host memory, one wait.  QS_EAGAIN (the flag cleared) as qs_batch_synchronize. */
struct qs_batch;
int qs_batch_pick1_host(struct qs_batch *b, float *d_logits, const float *logits, int n_vocab,
                        int32_t *d_out, int32_t *id);

/* Thread-local error message used by qs_last_error(). */
void qs_set_error(const char *fmt, ...);

#ifdef __cplusplus
}
#endif

#endif /* QS_INTERNAL_H */
