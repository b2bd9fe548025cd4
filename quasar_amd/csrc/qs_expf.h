/* qs_expf.h - single-precision exp that reproduces the host C library's expf bit for bit.
 *
 * The reference sampler computes its softmax numerators with libm expf (sample.c:148).
 * On the x86-64 glibc used here (2.35) that routine is the table-driven binary64 method
 * published by Szabolcs Nagy (ARM optimized-routines, adopted by glibc 2.28):
 *     x * 32/ln2 = k + r,  |r| <= 1/2,   2^(k/32) = 2^(k>>5) * T[k & 31],
 *     exp(x) ~= 2^(k/32) * (1 + C2 r + C1 r^2 + C0 r^3),  rounded once to float,
 * in the build of that routine that uses fused multiply-adds for the argument reduction
 * and the polynomial.  T[i] holds the binary64 bits of 2^(i/32) (correctly rounded) minus
 * i << 47, so adding k << 47 rescales by 2^(k>>5).  The same operation sequence written
 * with fma() runs on the host (gcc) and on gfx950 (v_fma_f64), so GPU softmax numerators
 * equal the reference's exactly.  Checked against the host expf on all 2^32 inputs.
 *
 * Device code passes a pointer to a copy of the table held in LDS (qs_expf_tab); host
 * code calls qs_expf. */
#ifndef QS_EXPF_H
#define QS_EXPF_H

#include <stdint.h>

#ifdef __HIPCC__
#define QS_EXPF_FN __host__ __device__ static inline
#else
#include <math.h>
#define QS_EXPF_FN static inline
#endif

#define QS_EXPF_TAB_N 32

#define QS_EXPF_TABLE_INIT {                                                             \
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull }

/* 32/ln2, the 1.5*2^52 rounding shifter, and the cubic's coefficients scaled by 1/32^k. */
#define QS_EXPF_INVLN2N (0x1.71547652b82fep+0 * 32.0)
#define QS_EXPF_SHIFT   0x1.8p+52
#define QS_EXPF_C0      (0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0)
#define QS_EXPF_C1      (0x1.ebfce50fac4f3p-3 / 32.0 / 32.0)
#define QS_EXPF_C2      (0x1.62e42ff0c52d6p-1 / 32.0)

QS_EXPF_FN uint32_t qs_f2u(float f) { union { float f; uint32_t u; } c; c.f = f; return c.u; }
QS_EXPF_FN float qs_u2f(uint32_t u) { union { float f; uint32_t u; } c; c.u = u; return c.f; }
QS_EXPF_FN uint64_t qs_d2u(double d) { union { double d; uint64_t u; } c; c.d = d; return c.u; }
QS_EXPF_FN double qs_u2d(uint64_t u) { union { double d; uint64_t u; } c; c.u = u; return c.d; }

/* Core for |x| < 88 (and the sub-range [-103.97, -88] that still rounds to a subnormal):
 * no special-case tests.  Adding ki << 47 to a table entry leaves its low word unchanged
 * and adds (ki << 15) mod 2^32 to its high word; the device code does exactly that with
 * one 32-bit shift-add (written as such, since the compiler would otherwise widen it back
 * to a 64-bit add). */
QS_EXPF_FN float qs_expf_core(float x, const uint64_t *tab) {
    double xd = (double)x;
    double kd = __builtin_fma(QS_EXPF_INVLN2N, xd, QS_EXPF_SHIFT);
    uint64_t ki = qs_d2u(kd);
    kd = kd - QS_EXPF_SHIFT;
    double r = __builtin_fma(QS_EXPF_INVLN2N, xd, -kd);
#ifdef __HIP_DEVICE_COMPILE__
    const uint64_t te = tab[ki & (QS_EXPF_TAB_N - 1)];
    const uint32_t klo = (uint32_t)ki, tlo = (uint32_t)te;
    uint32_t thi = (uint32_t)(te >> 32);
    asm("v_lshl_add_u32 %0, %1, 15, %0" : "+v"(thi) : "v"(klo));
    double s = qs_u2d(((uint64_t)thi << 32) | tlo);
#else
    uint64_t t = tab[ki & (QS_EXPF_TAB_N - 1)] + (ki << 47);
    double s = qs_u2d(t);
#endif
    double z = __builtin_fma(QS_EXPF_C0, r, QS_EXPF_C1);
    double r2 = r * r;
    double y = __builtin_fma(QS_EXPF_C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

/* The same method for arguments in the softmax window, x in [-33.27, 0], with the table
 * index taken straight from the shifter's low word.  Rounding with SHIFT + XOFF instead of
 * SHIFT (XOFF a multiple of 32; both in the binade [2^52, 2^53), where adding rounds to an
 * integer of the same parity, hence the same tie-breaking) leaves r unchanged and makes the
 * low word k + XOFF, which lies in [0, XOFF] for k in [-XOFF, 0].  Entry j of the extended
 * table is the scale itself for k = j - XOFF: T[k & 31] plus k << 47 (modulo 2^64), the bits
 * qs_expf_core forms per element, so the results equal qs_expf_core's bit for bit with one
 * mask and one add fewer per element. */
#define QS_EXPF_XOFF 1536
#define QS_EXPF_XTAB_N (QS_EXPF_XOFF + 1)
#define QS_EXPF_XSHIFT (QS_EXPF_SHIFT + QS_EXPF_XOFF)

QS_EXPF_FN uint64_t qs_expf_xtab_entry(const uint64_t *tab, int j) {
    return tab[j & (QS_EXPF_TAB_N - 1)] + ((uint64_t)(int64_t)(j - QS_EXPF_XOFF) << 47);
}

QS_EXPF_FN float qs_expf_window(float x, const uint64_t *xtab) {
    double xd = (double)x;
    double kd = __builtin_fma(QS_EXPF_INVLN2N, xd, QS_EXPF_XSHIFT);
    uint32_t klo = (uint32_t)qs_d2u(kd);
    kd = kd - QS_EXPF_XSHIFT;
    double r = __builtin_fma(QS_EXPF_INVLN2N, xd, -kd);
    double s = qs_u2d(xtab[klo]);
    double z = __builtin_fma(QS_EXPF_C0, r, QS_EXPF_C1);
    double r2 = r * r;
    double y = __builtin_fma(QS_EXPF_C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

#ifdef __HIPCC__
/* qs_expf_window on four arguments at once, in phases (argument reductions, then the four
 * table reads, then the polynomials, then the scaling), so the table reads are in flight
 * together instead of each waiting out its own latency.  Same operations, same results.
 * A caller with a loop passes the shifter and C1 (the default values) from registers that
 * stay live across it: an operation has room for one scalar operand besides, and a
 * constant would be copied into a vector register for every call. */
__device__ static inline void qs_expf4_window(const float (&x)[4], float (&e)[4],
                                              const uint64_t *xtab,
                                              double kshift = QS_EXPF_XSHIFT,
                                              double c1 = QS_EXPF_C1) {
    double r[4];
    uint32_t klo[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const double xd = (double)x[k];
        double kd = __builtin_fma(QS_EXPF_INVLN2N, xd, kshift);
        klo[k] = (uint32_t)qs_d2u(kd);
        kd = kd - QS_EXPF_XSHIFT;
        r[k] = __builtin_fma(QS_EXPF_INVLN2N, xd, -kd);
    }
    uint64_t te[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) te[k] = xtab[klo[k]];
    double y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const double z = __builtin_fma(QS_EXPF_C0, r[k], c1);
        const double r2 = r[k] * r[k];
        double t = __builtin_fma(QS_EXPF_C2, r[k], 1.0);
        y[k] = __builtin_fma(z, r2, t);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) e[k] = (float)(y[k] * qs_u2d(te[k]));
}
#endif

/* Full routine, including the |x| >= 88, infinity and NaN cases. */
QS_EXPF_FN float qs_expf_tab(float x, const uint64_t *tab) {
    uint32_t top = (qs_f2u(x) >> 20) & 0x7ffu;
    if (top >= 0x42bu) {                      /* |x| >= 88 or NaN */
        if (qs_f2u(x) == 0xff800000u) return 0.0f;            /* -inf */
        if (top >= 0x7f8u) return x + x;                      /* +inf, NaN */
        if (x > 0x1.62e42ep6f) return qs_u2f(0x7f800000u);    /* overflow */
        if (x < -0x1.9fe368p6f) return 0.0f;                  /* underflow */
    }
    return qs_expf_core(x, tab);
}

#ifndef __HIP_DEVICE_COMPILE__
static const uint64_t qs_expf_table_host[QS_EXPF_TAB_N] = QS_EXPF_TABLE_INIT;
QS_EXPF_FN float qs_expf(float x) { return qs_expf_tab(x, qs_expf_table_host); }
#endif

#endif /* QS_EXPF_H */
