/* orc_head.c - CPU restatement of the reference's output layer, logits = W . xn.
 *
 * TEST INFRASTRUCTURE: only the tests and the benchmark's checks use this (as the checker);
 * the product is the HIP kernel behind qs_batch_head_exact_logits / qs_batch_pick_head_exact.
 *
 * Follows forward_cpu.c:140-147 (gemv: per output row, the weight row dequantized to
 * float, then acc += w[k] * x[k] in float for k ascending, a product then a sum) and
 * quant.c:8-27, 62-70, 106-130, 205-217 (quasar_dequant_row for F32, F16, Q8_0 and Q6_K:
 * the fp16 scale widened exactly, Q8_0's d * q, Q6_K's (d * sc) * q with q the 6-bit value
 * less 32).  Built with -ffp-contract=off, as the reference's -std=c11 build contracts
 * nothing.
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "orc_sampler.h"

/* quant.c:8-27: binary16 bits to float, exactly (subnormals normalised, inf/NaN kept). */
static float orc_half(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16, e = (h >> 10) & 0x1F, m = h & 0x3FF, f;
    if (e == 0) {
        if (m == 0) {
            f = sign;
        } else {
            e = 127 - 15 + 1;
            while ((m & 0x400) == 0) {
                m <<= 1;
                e--;
            }
            f = sign | (e << 23) | ((m & 0x3FF) << 13);
        }
    } else if (e == 0x1F) {
        f = sign | 0x7F800000u | (m << 13);
    } else {
        f = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &f, 4);
    return out;
}

static uint16_t rd16(const uint8_t *p) {
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
}

/* Bytes of one row of n elements of a type (0: a type this restatement does not take). */
long orc_head_row_bytes(int type, int n) {
    switch (type) {
        case ORC_W_F32: return 4L * n;
        case ORC_W_F16: return 2L * n;
        case ORC_W_Q8_0: return n % 32 ? 0 : (long)n / 32 * 34;
        case ORC_W_Q6_K: return n % 256 ? 0 : (long)n / 256 * 210;
        default: return 0;
    }
}

/* quant.c:205-217 for the four types. */
void orc_dequant_row(int type, const uint8_t *src, float *dst, int n) {
    if (type == ORC_W_F32) {
        memcpy(dst, src, (size_t)n * 4);
    } else if (type == ORC_W_F16) {
        for (int i = 0; i < n; i++) dst[i] = orc_half(rd16(src + 2 * (size_t)i));
    } else if (type == ORC_W_Q8_0) {                        /* quant.c:62-70 */
        for (int i = 0; i < n / 32; i++) {
            const uint8_t *b = src + (size_t)i * 34;
            const float d = orc_half(rd16(b));
            const int8_t *q = (const int8_t *)(b + 2);
            for (int j = 0; j < 32; j++) dst[i * 32 + j] = d * q[j];
        }
    } else if (type == ORC_W_Q6_K) {                        /* quant.c:106-130 */
        for (int i = 0; i < n / 256; i++) {
            const uint8_t *b = src + (size_t)i * 210, *ql = b, *qh = b + 128;
            const int8_t *sc = (const int8_t *)(b + 192);
            const float d = orc_half(rd16(b + 208));
            float *y = dst + (size_t)i * 256;
            for (int half = 0; half < 2; half++) {
                for (int l = 0; l < 32; l++) {
                    const int is = l / 16;
                    const int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    const int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    y[l] = d * sc[is + 0] * q1;
                    y[l + 32] = d * sc[is + 2] * q2;
                    y[l + 64] = d * sc[is + 4] * q3;
                    y[l + 96] = d * sc[is + 6] * q4;
                }
                y += 128;
                ql += 64;
                qh += 32;
                sc += 8;
            }
        }
    } else {
        for (int i = 0; i < n; i++) dst[i] = 0.0f;
    }
}

/* forward_cpu.c:140-147 over rows [r0, r1) for each of the nx hidden rows. */
typedef struct {
    int type, E, V, nx, r0, r1;
    const uint8_t *w;
    const float *x;
    float *y;
} GemvJob;

static void *gemv_job(void *p) {
    const GemvJob *j = (const GemvJob *)p;
    const long rb = orc_head_row_bytes(j->type, j->E);
    float *row = (float *)malloc(sizeof(float) * (size_t)j->E);
    if (!row) return NULL;
    for (int r = j->r0; r < j->r1; r++) {
        orc_dequant_row(j->type, j->w + (size_t)r * rb, row, j->E);
        for (int b = 0; b < j->nx; b++) {
            const float *x = j->x + (size_t)b * j->E;
            float acc = 0.0f;
            for (int k = 0; k < j->E; k++) acc += row[k] * x[k];
            j->y[(size_t)b * j->V + r] = acc;
        }
    }
    free(row);
    return NULL;
}

/* y[b][r] = W[r] . x[b] for every row r < V and hidden row b < nx (W: V rows of `type`,
 * E elements each, as the GGUF file lays them out), on n_threads POSIX threads. */
void orc_head_gemv(int type, const uint8_t *w, const float *x, int nx, int E, int V,
                   float *y, int n_threads) {
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 64) n_threads = 64;
    pthread_t th[64];
    GemvJob jobs[64];
    for (int t = 0; t < n_threads; t++) {
        jobs[t] = (GemvJob){type, E, V, nx, (int)((long)V * t / n_threads),
                            (int)((long)V * (t + 1) / n_threads), w, x, y};
        if (pthread_create(&th[t], NULL, gemv_job, &jobs[t]) != 0) {
            gemv_job(&jobs[t]);
            th[t] = 0;
        }
    }
    for (int t = 0; t < n_threads; t++)
        if (th[t]) pthread_join(th[t], NULL);
}
