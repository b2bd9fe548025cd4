/* orc_router.c - CPU restatement of the reference's mixture-of-experts router choice.
 *
 * TEST INFRASTRUCTURE: only the tests use this (as the checker); the product is the HIP
 * kernel behind qs_router_topk.
 *
 * Follows forward_cpu.c:165-172 (softmax: max by a strict `>` scan from element 0, expf
 * of the differences summed in float in index order, one float reciprocal, products)
 * and forward_cpu.c:296-304 (n_used scans for the largest untaken probability with a
 * strict `>` from -1e30, so the lowest index wins ties and a NaN never does; then, with
 * norm_topk_prob, the weights divided by their float sum in slot order when it is
 * positive).  Where the reference's scan finds nothing (every remaining probability
 * NaN) it reads index -1 out of bounds; this restatement records expert -1 with weight 0
 * there and takes nothing.  expf is the host C library's, as in the reference.
 */
#include <math.h>
#include <stdint.h>

#include "orc_sampler.h"

/* forward_cpu.c:165-172 */
static void orc_softmax(float *a, int n) {
    float mx = a[0];
    for (int i = 1; i < n; i++)
        if (a[i] > mx) mx = a[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        a[i] = expf(a[i] - mx);
        sum += a[i];
    }
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) a[i] *= inv;
}

/* The softmax of one row as orc_softmax leaves it (p[n]) and the float sum of its
 * numerators (for the tests' bounds on it). */
void orc_router_probs(const float *x, int n, float *p, float *sum_out) {
    float mx = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += expf(x[i] - mx);
    for (int i = 0; i < n; i++) p[i] = x[i];
    orc_softmax(p, n);
    *sum_out = sum;
}

/* forward_cpu.c:296-304, token by token.  n_expert <= 256, n_used <= 64. */
void orc_router_topk(const float *logits, long row_stride, int n_tokens, int n_expert,
                     int n_used, int norm_topk, int32_t *idx, float *wt) {
    for (int t = 0; t < n_tokens; t++) {
        float p[256] = {0.0f};
        unsigned char taken[256] = {0};
        for (int e = 0; e < n_expert; e++) p[e] = logits[(long)t * row_stride + e];
        orc_softmax(p, n_expert);
        int32_t *ti = idx + (long)t * n_used;
        float *tw = wt + (long)t * n_used;
        for (int s = 0; s < n_used; s++) {
            int bi = -1;
            float best = -1e30f;
            for (int e = 0; e < n_expert; e++)
                if (!taken[e] && p[e] > best) {
                    best = p[e];
                    bi = e;
                }
            ti[s] = bi;
            tw[s] = bi >= 0 ? p[bi] : 0.0f;
            if (bi >= 0) taken[bi] = 1;
        }
        if (norm_topk) {
            float sm = 0.0f;
            for (int s = 0; s < n_used; s++) sm += tw[s];
            if (sm > 0.0f)
                for (int s = 0; s < n_used; s++) tw[s] /= sm;
        }
    }
}
