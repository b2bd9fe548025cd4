/* stub_device.c - the device layer as a machine without a GPU sees it, for the sanitizer
 * build of the host code (tests/c/sanitize_host.c): every device call fails the way the
 * HIP layer reports an unavailable device. */
#include <stddef.h>
#include <stdint.h>

#include "quasar_sampler.h"

void qs_set_error(const char *fmt, ...);

#define NODEV(name) do { qs_set_error("%s: no device (stub)", name); } while (0)

qs_batch *qs_batch_new(int max_rows, int max_vocab, int max_last_n) {
    (void)max_rows; (void)max_vocab; (void)max_last_n;
    NODEV("qs_batch_new");
    return NULL;
}
void qs_batch_free(qs_batch *b) { (void)b; }
int qs_batch_config(qs_batch *b, int row0, int n_rows, float temperature, float top_p,
                    int top_k, float min_p, float repeat_penalty, int repeat_last_n,
                    const uint64_t *seeds) {
    (void)b; (void)row0; (void)n_rows; (void)temperature; (void)top_p; (void)top_k;
    (void)min_p; (void)repeat_penalty; (void)repeat_last_n; (void)seeds;
    NODEV("qs_batch_config");
    return QS_EDEVICE;
}
int qs_batch_reset(qs_batch *b, int row0, int n_rows) {
    (void)b; (void)row0; (void)n_rows;
    return QS_EDEVICE;
}
int qs_batch_pick(qs_batch *b, const float *d_logits, int64_t row_stride, int n_rows,
                  int n_vocab, int32_t *d_out, qs_pick_diag *d_diag) {
    (void)b; (void)d_logits; (void)row_stride; (void)n_rows; (void)n_vocab; (void)d_out;
    (void)d_diag;
    return QS_EDEVICE;
}
int qs_batch_synchronize(qs_batch *b) { (void)b; return QS_EDEVICE; }
int qs_batch_pick1_host(struct qs_batch *b, float *d_logits, const float *logits, int n_vocab,
                        int32_t *d_out, int32_t *id) {
    (void)b; (void)d_logits; (void)logits; (void)n_vocab; (void)d_out; (void)id;
    return QS_EDEVICE;
}
int qs_batch_set_state(qs_batch *b, int row, uint64_t rng, const int32_t *hist, int n) {
    (void)b; (void)row; (void)rng; (void)hist; (void)n;
    return QS_EDEVICE;
}
int qs_batch_get_state(qs_batch *b, int row, uint64_t *rng, int32_t *hist, int cap, int *len) {
    (void)b; (void)row; (void)rng; (void)hist; (void)cap; (void)len;
    return QS_EDEVICE;
}
void *qs_device_alloc(size_t bytes) { (void)bytes; NODEV("qs_device_alloc"); return NULL; }
void qs_device_free(void *p) { (void)p; }
int qs_memcpy_h2d(void *d, const void *s, size_t n) { (void)d; (void)s; (void)n; return QS_EDEVICE; }
int qs_memcpy_d2h(void *d, const void *s, size_t n) { (void)d; (void)s; (void)n; return QS_EDEVICE; }
