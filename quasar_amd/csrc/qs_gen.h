/* qs_gen.h - portable synthetic-logit generator, shared by host C11 and HIP device code.
 *
 * Every value is a pure function of (seed, row, column): a counter-based hash feeds
 * IEEE binary64 arithmetic that uses only +, -, * and integer bit manipulation (no
 * division, no libm, no sqrt).  Compiled with -ffp-contract=off on both sides, the host
 * (gcc, SSE2) and gfx950 (hipcc) produce bit-identical logits, so a batch generated on
 * the GPU can be checked against the CPU sampler on the same bits without a copy.
 *
 * Distributions used by the workloads:
 *   QS_DIST_NORMAL      sigma * N(0,1)
 *   QS_DIST_NORMAL_PEAK sigma * N(0,1), plus `boost` added (in float) at one column per
 *                       row chosen by the hash
 *   QS_DIST_STUDENT_T3  sigma * Z0 / sqrt((Z1^2 + Z2^2 + Z3^2) / 3)
 * Normals come from Marsaglia's polar method.  The helpers below (reciprocal, reciprocal
 * square root, log) are Newton iterations / a short atanh series, written out so the
 * operation sequence is fixed. */
#ifndef QS_GEN_H
#define QS_GEN_H

#include <stdint.h>

#ifdef __HIPCC__
#define QS_GEN_FN __host__ __device__ static inline
#else
#define QS_GEN_FN static inline
#endif

enum { QS_DIST_NORMAL = 0, QS_DIST_NORMAL_PEAK = 1, QS_DIST_STUDENT_T3 = 2 };

typedef struct {
    int32_t  dist;      /* QS_DIST_* */
    float    sigma;     /* scale of the base distribution */
    float    boost;     /* NORMAL_PEAK: value added at the boosted column */
    int32_t  pad;
    uint64_t seed;      /* workload seed */
} qs_gen_spec;

QS_GEN_FN uint64_t qs_mix64(uint64_t z) {           /* splitmix64 finaliser */
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Hash of (seed, a, b): independent streams for rows, columns and draw indices. */
QS_GEN_FN uint64_t qs_hash3(uint64_t seed, uint64_t a, uint64_t b) {
    return qs_mix64(qs_mix64(seed ^ qs_mix64(a * 0xD1B54A32D192ED03ull + 0x632BE59BD9B4E019ull))
                    + b * 0x8CB92BA72F3D8DD7ull);
}

QS_GEN_FN double qs_bits_to_double(uint64_t u) {
    union { uint64_t u; double d; } c; c.u = u; return c.d;
}
QS_GEN_FN uint64_t qs_double_to_bits(double d) {
    union { uint64_t u; double d; } c; c.d = d; return c.u;
}

/* Uniform in the open interval (0, 1), exact in binary64. */
QS_GEN_FN double qs_u01(uint64_t h) { return ((double)(h >> 11) + 0.5) * 0x1p-53; }

/* 2^e for |e| < 1000, built from the exponent field (exact). */
QS_GEN_FN double qs_pow2(int e) { return qs_bits_to_double((uint64_t)(1023 + e) << 52); }

/* 1/a for finite a > 0: scale to m in [1,2), Newton from the 24/17 - 8/17 m guess
 * (relative error <= 1/17, squared by each step). */
QS_GEN_FN double qs_recip(double a) {
    uint64_t b = qs_double_to_bits(a);
    int e = (int)((b >> 52) & 0x7ff) - 1023;
    double m = qs_bits_to_double((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull);
    double x = 1.411764705882353 - 0.47058823529411764 * m;
    for (int i = 0; i < 5; i++) {
        double t = m * x;
        double u = 1.0 - t;
        double v = x * u;
        x = x + v;
    }
    return x * qs_pow2(-e);
}

/* 1/sqrt(a) for finite a > 0: scale to m in [1,4), Newton from a linear guess. */
QS_GEN_FN double qs_rsqrt(double a) {
    uint64_t b = qs_double_to_bits(a);
    int e = (int)((b >> 52) & 0x7ff) - 1023;
    int k = e >> 1;                              /* floor(e/2) */
    double m = qs_bits_to_double((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull);
    if (e - 2 * k) m = m * 2.0;                  /* m in [1,4) and a = m * 4^k */
    double y = 1.0 - 0.16 * (m - 1.0);
    for (int i = 0; i < 7; i++) {
        double y2 = y * y;
        double t = m * y2;
        double h = 1.5 - 0.5 * t;
        y = y * h;
    }
    return y * qs_pow2(-k);
}

/* Natural log for finite x > 0: x = m 2^e with m in [sqrt(1/2), sqrt(2)),
 * log m = 2 atanh(t), t = (m-1)/(m+1), 14-term odd series (|t| < 0.172). */
QS_GEN_FN double qs_log(double x) {
    uint64_t b = qs_double_to_bits(x);
    int e = (int)((b >> 52) & 0x7ff) - 1023;
    double m = qs_bits_to_double((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull);
    if (m > 1.4142135623730951) { m = m * 0.5; e = e + 1; }
    double t = (m - 1.0) * qs_recip(m + 1.0);
    double t2 = t * t;
    const double c[14] = {
        0x1.0000000000000p+0, 0x1.5555555555555p-2, 0x1.999999999999ap-3, 0x1.2492492492492p-3,
        0x1.c71c71c71c71cp-4, 0x1.745d1745d1746p-4, 0x1.3b13b13b13b14p-4, 0x1.1111111111111p-4,
        0x1.e1e1e1e1e1e1ep-5, 0x1.af286bca1af28p-5, 0x1.8618618618618p-5, 0x1.642c8590b2164p-5,
        0x1.47ae147ae147bp-5, 0x1.2f684bda12f68p-5 };
    double p = c[13];
    for (int i = 12; i >= 0; i--) { p = p * t2; p = p + c[i]; }
    double lm = 2.0 * t;
    lm = lm * p;
    double le = (double)e * 0x1.62e42fefa39efp-1;
    return le + lm;
}

/* Standard normal for (seed, row, col, stream) by the polar method. */
QS_GEN_FN double qs_normal(uint64_t seed, uint64_t row, uint64_t col, uint32_t stream) {
    uint64_t base = qs_hash3(seed, row, col);
    for (uint32_t k = 0; k < 64; k++) {
        uint64_t h1 = qs_hash3(base, (uint64_t)stream * 131u + 2u * k, 0x51u);
        uint64_t h2 = qs_hash3(base, (uint64_t)stream * 131u + 2u * k + 1u, 0xA7u);
        double x = 2.0 * qs_u01(h1) - 1.0;
        double y = 2.0 * qs_u01(h2) - 1.0;
        double s = x * x;
        double y2 = y * y;
        s = s + y2;
        if (s < 1.0 && s > 0.0) {
            double q = -2.0 * qs_log(s);
            q = q * qs_recip(s);
            double f = q * qs_rsqrt(q);         /* sqrt(q) */
            return x * f;
        }
    }
    return 0.0;                                   /* probability < 1e-40 */
}

/* Column that receives the boost in a NORMAL_PEAK row. */
QS_GEN_FN int32_t qs_peak_col(uint64_t seed, uint64_t row, int32_t n_vocab) {
    return (int32_t)(qs_hash3(seed ^ 0x5EEDB0057ull, row, 0xB0057ull) % (uint64_t)n_vocab);
}

/* One logit. */
QS_GEN_FN float qs_gen_logit(const qs_gen_spec *g, uint64_t row, int32_t col, int32_t n_vocab) {
    double z;
    if (g->dist == QS_DIST_STUDENT_T3) {
        double z0 = qs_normal(g->seed, row, (uint64_t)col, 0);
        double z1 = qs_normal(g->seed, row, (uint64_t)col, 1);
        double z2 = qs_normal(g->seed, row, (uint64_t)col, 2);
        double z3 = qs_normal(g->seed, row, (uint64_t)col, 3);
        double c = z1 * z1;
        double t2 = z2 * z2;
        double t3 = z3 * z3;
        c = c + t2;
        c = c + t3;
        c = c * 0x1.5555555555555p-2;
        z = z0 * qs_rsqrt(c);
    } else {
        z = qs_normal(g->seed, row, (uint64_t)col, 0);
    }
    double v = (double)g->sigma * z;
    float f = (float)v;
    if (g->dist == QS_DIST_NORMAL_PEAK && col == qs_peak_col(g->seed, row, n_vocab))
        f = f + g->boost;
    return f;
}

/* History id j of `row`: uniform over [0, n_vocab), or drawn from a per-row pool of
 * `pool` ids when pool > 0 (which makes duplicates likely). */
QS_GEN_FN int32_t qs_gen_hist_id(uint64_t seed, uint64_t row, int32_t j, int32_t n_vocab,
                                 int32_t pool) {
    if (pool > 0) {
        uint64_t k = qs_hash3(seed ^ 0x9001ull, row, (uint64_t)j) % (uint64_t)pool;
        return (int32_t)(qs_hash3(seed ^ 0x9002ull, row, k) % (uint64_t)n_vocab);
    }
    return (int32_t)(qs_hash3(seed ^ 0x9003ull, row, (uint64_t)j) % (uint64_t)n_vocab);
}

/* Per-row sampler seed, never 0 (0 would mean "time-seeded" to the sampler). */
QS_GEN_FN uint64_t qs_gen_row_seed(uint64_t seed, uint64_t row) {
    uint64_t s = qs_hash3(seed ^ 0x5EEDull, row, 0x1234ull);
    return s ? s : 1ull;
}

#endif /* QS_GEN_H */
