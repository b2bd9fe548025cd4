// qs_cert.h - the softmax denominator as a proven interval, and sample.c:153-178 decided
// for every normaliser that interval allows (device code, included by qs_part.hip).
//
// The reference sums (double)expf(sc_i - msc) over the 30-nat window in id order
// (sample.c:146-149) and draws with inv = (float)(1.0 / sum).  The streaming kernel
// instead sums, per part of a row, e^_i = 2^t_i with t_i = fl(sc_i * L - c) (one fma, one
// v_exp_f32), where M is the part's largest scaled logit, L = float(log2 e) and c a float
// at or above M*L; it also sums e^_i * t_i.  From those two sums, the part maxima and the
// rounding bounds below, the row's last workgroup derives [S_lo, S_hi], an interval that
// provably holds the reference's sum, hence [v_lo, v_hi] = [fl(1/S_hi), fl(1/S_lo)], the
// floats the reference's inv can be (both roundings are monotone).  Only the top
// candidates' numerators are computed exactly (qs_expf_core, equal to the host expf).
//
// The decision is then taken once and proved to be the same for every inv in
// [v_lo, v_hi]:
//   order   p_i = fl(e_i * inv) is monotone in e_i, so the (p desc, id asc) order is the
//           (e desc, id asc) order unless two neighbours with ids in descending order
//           round to the same p; excluded when e_i > e_{i+1} (1 + 2^-22) for every such
//           pair the cuts read (fl(e v) lies within e v (1 +- 2^-24)).
//   top-p   the running sums cum_i(v) are monotone in v, so the cut is the same for all v
//           when the first position that may reach top_p at v_hi surely reaches it at
//           v_lo (lane scans stand for the sequential sums up to a 2^-40 margin).
//   min-p   p_i(v) < fl(min_p p_0(v)) holds for all v when e_i < min_p e_0 (1 - 2^-21),
//           and fails for all v when e_i >= min_p e_0 (1 + 2^-21).
//   draw    the accumulated p and u * rsum all scale with v up to 2^-23 relative: the
//           chosen position c is the same for all v when u * E_{n-1} (1 + 2^-22) <= E_c
//           and u * E_{n-1} (1 - 2^-22) > E_{c-1}, E_j the running sums of e.
// Anything not proved (a normaliser interval the cuts cross, neighbours that may swap, a
// cut reading past the proven prefix) is reported and the caller recomputes the row's
// exact sum instead.
//
// Error bound of one part (all logs natural; a_i = M - sc_i >= 0, D = msc - M >= 0,
// rho = L M - c in (-ulp(c), 0], gamma = L ln2 - 1):
//   e_ref_i / (e^_i exp(M - msc) 2^-rho) = exp(-gamma (sc_i - M) - ln2 (L(sc_i - M) + rho) d_i
//                                          + (sc_i - msc) d'_i) (1 + zeta_i) / (1 + eta_i)
// with |d_i|, |d'_i| <= 2^-24 (the fma's and the reference's subtraction's roundings),
// |zeta_i| <= ZETA (host expf) and |eta_i| <= ETA (v_exp_f32), so
//   |log ratio| <= KAPPA_A a_i + 2^-24 (ln2 |rho| + D) + ZETA + ETA,
//   KAPPA_A = |gamma| + (1 + |gamma|) 2^-24 + 2^-24.
// Elements outside the reference's window add at most V exp(thr - msc) in all.
#pragma once

#include "qs_device.h"

namespace qs {

constexpr float CERT_L = 0x1.715476p+0f;          // float(log2 e) = 1.44269502162933349609375
constexpr double CERT_LN2 = 0x1.62e42fefa39efp-1;
// 1 / L in binary64 (folded by the compiler, rounded to nearest): A below is multiplied by
// it instead of divided by L, one rounding of 2^-53 in place of the division's, inside the
// factor 1 + 2^-22 that covers A's arithmetic.
constexpr double CERT_INV_L = 1.0 / (double)CERT_L;
// KAPPA_A above (1.32559e-7), rounded up.
constexpr double CERT_KAPPA_A = 1.3256e-7;
// Host expf (glibc 2.35 x86-64): largest relative error over every float in [-64, 0],
// measured exhaustively against expl: 5.959911e-08 (2^-24.0001); rounded up.
constexpr double CERT_ZETA = 5.9600e-8;
// v_exp_f32 on gfx950: largest relative error against exp2 in binary64 over every float
// t in [-64, 0], measured exhaustively on the device: 8.483877e-08 (2^-23.49); rounded up.
constexpr double CERT_ETA = 8.4840e-8;
// Bound on exp(-t) for t > 64 among the e^ of elements outside the window.
constexpr double CERT_TAIL = 0x1p-62;
// Below this |msc| the window's arguments stay in [-31, 0] and the parts' c and t keep
// the precision the bound assumes; other rows take the exact path.
constexpr float CERT_MSC_MAX = 0x1p20f;

// The part constant c: float(M * L) rounded up, so rho = L M - c is in (-ulp(c), 0] and
// every t = fl(sc L - c) of the part is <= 0 (v_exp_f32's measured range).
__device__ __forceinline__ float cert_c(float M) {
    float c = M * CERT_L;
    if (__builtin_fmaf(M, CERT_L, -c) > 0.0f) {       // c below M*L: the next float up
        const uint32_t b = __float_as_uint(c);         // (c != 0 here: M*L was inexact)
        c = __uint_as_float(c > 0.0f ? b + 1u : b - 1u);
    }
    return c;
}


// ---- per-logit pieces of the streaming kernels ----------------------------------------------

constexpr float T_GUARD = -200.0f;   // t floor in wavefronts with -inf, NaN or huge logits
constexpr float SC_SANE = -1e30f;    // scaled logits at or above this give a finite t

__device__ __forceinline__ float max3n(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
__device__ __forceinline__ float min3n(float a, float b, float c) {
    return __builtin_elementwise_minimum(__builtin_elementwise_minimum(a, b), c);
}
// The largest of four logits (v_max3 without operand canonicalisation; with a NaN among
// them the result may be a NaN).
__device__ __forceinline__ float max4(const float4 &v) {
    float m;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(m) : "v"(v.x), "v"(v.y), "v"(v.z));
    asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(m), "v"(v.w));
    return m;
}

// Pass 2 on one float4: the approximate numerators' quad sum and the e*t sum.
template <bool GUARD>
__device__ __forceinline__ void sum4(const float4 &v, float inv_t, float c, double &S, float &Tn) {
    const float w[4] = {v.x, v.y, v.z, v.w};
    float t[4], e[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float sc = w[k] * inv_t;                // the reference's scaled logit
        t[k] = __builtin_fmaf(sc, CERT_L, -c);
        if (GUARD) t[k] = fmaxf(t[k], T_GUARD);
        e[k] = __builtin_amdgcn_exp2f(t[k]);
    }
    S += (double)((e[0] + e[1]) + (e[2] + e[3]));
#pragma unroll
    for (int k = 0; k < 4; ++k) Tn = __builtin_fmaf(e[k], t[k], Tn);
}

// The m-th largest lane value of a wavefront (wmx: its largest), or a value at most that
// with at least m lane values at or above it.  Uniform.  Up to 6: the lanes holding the
// current largest value drop out (value 0: keys of logits are above it) and the largest of
// the rest is taken; beyond, a sort.
__device__ __forceinline__ uint32_t wave_mth(uint32_t v, uint32_t wmx, int m) {
    if (m <= 6) {
        uint32_t x = wmx;
        for (int i = 1; i < m; ++i) {
            v = v >= x ? 0u : v;
            const uint32_t y = wave_max_u(v);
            if (y == 0u) break;                       // every lane is at or above x
            x = y;
        }
        return x;
    }
    const uint32_t srt = wave_sort_desc_u32(v);
    return (uint32_t)__builtin_amdgcn_readlane((int)srt, m - 1);
}

// Interval of the reference's softmax denominator from one part's sums (per lane, lanes
// past the parts pass S = 0, T = 0, maxw = -inf).  Accumulated by the caller:
// lo += s*(S (1-2^-22.9)) - E, hi += s*(S (1+2^-22.9)) + E.
struct CertPart {
    double lo, hi;
};
__device__ __forceinline__ CertPart cert_part(float maxw, double S, float T, float inv_t,
                                              float msc, float thr) {
    CertPart r{0.0, 0.0};
    const float M = maxw * inv_t;
    // a part whose largest scaled logit is below the threshold has nothing in the window
    if (!(M >= thr) || !(S > 0.0)) return r;
    const float c = cert_c(M);
    const double rho = (double)CERT_L * (double)M - (double)c;     // exact in binary64
    const double D = (double)msc - (double)M;                      // exact, >= 0
    const double s = exp(-D - rho * CERT_LN2);
    const double sup = S * (1.0 + 0x1.12p-23), slo = S * (1.0 - 0x1.12p-23);  // 2^-22.9
    const double arho = -rho;
    // sum of e^_i a_i: a_i <= (|t_i| (1 + 2^-23) + |rho|) / L; T carries at most about
    // 30 roundings of 2^-24 (20 fma steps per thread, then the reductions)
    const double A = ((double)T * (1.0 + 0x1p-18) + arho * sup) * CERT_INV_L * (1.0 + 0x1p-22);
    const double kj = 0x1p-24 * (CERT_LN2 * arho + D) + CERT_ZETA + CERT_ETA + 0x1p-100;
    const double E = s * (1.0 + 0x1p-10) * (CERT_KAPPA_A * A + kj * sup);
    r.lo = s * slo - E;
    r.hi = s * sup + E;
    return r;
}

// An integer exponent base: the least integer-valued float at or above M*L (M finite,
// |M| < 2^22).  Sums taken against such bases are moved to a larger one by an exact
// power of two, so a lane can start its sums before it has seen its largest logit.
__device__ __forceinline__ float cert_cbase(float M) {
    float c = ceilf(M * CERT_L);
    if (__builtin_fmaf(M, CERT_L, -c) > 0.0f) c += 1.0f;   // M*L rounded down onto c
    return c;
}

// cert_part for a part whose sums were taken against an integer base c >= M*L, some of
// them first against smaller integer bases and then scaled by 2^-(difference) exactly
// (rho = L M - c in (-1, 0]).  A term taken against a base c' <= c has the rounding error
// of fl(sc L - c'), at most 2^-24 |sc L - c'| <= 2^-24 |sc L - c|, so the per-element bound
// of cert_part holds with this rho.  T = sum of e^ * (-t) is an approximation whose
// roundings (a float chain per chunk, then binary64 rescaling and sums) stay far inside
// the factor 1 + 2^-12 allowed for them.  cert_part_cs takes the part's scale
// s = exp(-D - rho ln 2) (D = msc - M) from cert_scale_c, which needs neither sum, so a
// caller may compute it while the sums are still being reduced; cert_part_c does both.
__device__ __forceinline__ double cert_scale_c(float maxw, float c, float inv_t, float msc) {
    const float M = maxw * inv_t;
    const double rho = (double)CERT_L * (double)M - (double)c;     // exact in binary64
    const double D = (double)msc - (double)M;                      // exact, >= 0
    return exp(-D - rho * CERT_LN2);
}

__device__ __forceinline__ CertPart cert_part_cs(float maxw, float c, double S, double T,
                                                 float inv_t, float msc, float thr, double s) {
    CertPart r{0.0, 0.0};
    const float M = maxw * inv_t;
    if (!(M >= thr) || !(S > 0.0)) return r;
    const double rho = (double)CERT_L * (double)M - (double)c;     // exact in binary64
    const double D = (double)msc - (double)M;                      // exact, >= 0
    const double sup = S * (1.0 + 0x1.12p-23), slo = S * (1.0 - 0x1.12p-23);
    const double arho = -rho;
    const double A = (T * (1.0 + 0x1p-12) + arho * sup) * CERT_INV_L * (1.0 + 0x1p-22);
    const double kj = 0x1p-24 * (CERT_LN2 * arho + D) + CERT_ZETA + CERT_ETA + 0x1p-100;
    const double E = s * (1.0 + 0x1p-10) * (CERT_KAPPA_A * A + kj * sup);
    r.lo = s * slo - E;
    r.hi = s * sup + E;
    return r;
}
__device__ __forceinline__ CertPart cert_part_c(float maxw, float c, double S, double T,
                                                float inv_t, float msc, float thr) {
    return cert_part_cs(maxw, c, S, T, inv_t, msc, thr, cert_scale_c(maxw, c, inv_t, msc));
}

// The whole-row interval from the per-part sums of lo/hi: the window's outside elements
// (at most V of them, each below exp(thr - msc) or CERT_TAIL), the reference's sequential
// double sum (at most V roundings of 2^-53) and this arithmetic (2^-40).  S_ref >= 1
// always (the max's own term is expf(0) = 1).
__device__ __forceinline__ void cert_interval(double lo, double hi, float msc, float thr, int V,
                                              double &S_lo, double &S_hi) {
    // thr = fl(msc - 30): d = thr - msc + 30 is exact in binary64 and |d| <= 1/16 for
    // |msc| < 2^20 (rows beyond take the exact path), where exp(d) <= 1 + d + d^2;
    // exp(-30) = 0x1.a56e0c2ac7f75p-44, the product rounded up by the factor 1.001
    const double d = ((double)thr - (double)msc) + 30.0;
    double out = 0x1.a56e0c2ac7f75p-44 * 1.001 * (1.0 + d + d * d);
    if (out < CERT_TAIL) out = CERT_TAIL;
    const double seq = (double)V * 0x1p-53;
    S_lo = (lo - (double)V * out) * (1.0 - seq) * (1.0 - 0x1p-40);
    S_hi = hi * (1.0 + seq) * (1.0 + 0x1p-40);
    if (S_lo < 1.0) S_lo = 1.0;
}

// (e, id) sort key: e's bits above, ~id below (descending: e desc, id asc).
__device__ __forceinline__ uint64_t eid_key(float e, int id) {
    return ((uint64_t)__float_as_uint(e) << 32) | (uint32_t)~(uint32_t)id;
}

// sample.c:153-178 for every inv in [v_lo, v_hi], over sorted (e, id) keys held Q per lane
// by one wavefront (position q*64 + lane in k[q]; keys past the candidates are 0).  E: the
// positions [0, E) are positions of the full order for every such inv; nwin: the window
// size, or any value above E when it is not known (every use of it then lies past E).
// Returns CF_NONE with rs advanced, id, and d's keep counts when the cuts and the draw are
// proved the same for every inv of the interval; otherwise the CF_* reason (nothing
// consumed).
// Every lane gets the same results.
__device__ __forceinline__ float lane_f(float v, int i) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}
__device__ __forceinline__ double lane_d(double v, int i) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)u, i);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), i);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Reasons a certified decision hands the row to the exact path (qs_pick_diag.fallback).
enum {
    CF_NONE = 0, CF_INPUT = 1, CF_BRACKET = 2, CF_PREFIX = 3, CF_ORDER = 4, CF_TOPP_EXACT = 5,
    CF_TOPP_SPLIT = 6, CF_TOPP_PAST = 7, CF_MINP_FLOOR = 8, CF_MINP_SPLIT = 9,
    CF_MINP_PAST = 10, CF_KEEP_PAST = 11, CF_DRAW_HI = 12, CF_DRAW_LO = 13, CF_MSC = 14,
    CF_WIDE = 15
};

template <int Q>
__device__ __forceinline__ int cert_prefix(const uint64_t (&k)[Q], int E, int nwin,
                                            const qs_row_param &P, float v_lo, float v_hi,
                                            uint64_t &rs, int &id, qs_pick_diag &d) {
    const int lane = threadIdx.x & 63;
    int n = nwin;                                             // sample.c:153-154
    if (P.top_k > 0 && P.top_k < n) n = P.top_k;
    d.keep_topk = n;
    const int lim = min(n, E);          // positions the cuts can read
    if (lim < 1 || lim > 64 * Q) return CF_PREFIX;
    uint64_t rs2 = rs;                  // the draw's uniform (sample.c:172), consumed only
    const double u = rng_unit(rs2);     // when the row is decided
    float e[Q];
    int idv[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        e[q] = key_p(k[q]);
        idv[q] = key_id(k[q]);
    }
    // the first position in [beg, end) where pred(q) holds, or end
    auto first = [&](int beg, int end, auto &&pred) {
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int i = q * 64 + lane;
            const uint64_t m = __ballot(i >= beg && i < end && pred(q));
            if (m) return q * 64 + (int)__builtin_ctzll(m);
        }
        return end;
    };
    // values at a uniform position
    auto e_at = [&](int i) {
        float v = 0.0f;
#pragma unroll
        for (int q = 0; q < Q; ++q)
            if (q == (i >> 6)) v = lane_f(e[q], i & 63);
        return v;
    };
    // the order: neighbours whose ids descend must keep distinct p for every inv
    {
        bool bad = false;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int i = q * 64 + lane;
            if (q * 64 + 1 >= lim) break;
            float en = __shfl_down(e[q], 1, 64);
            int idn = __shfl_down(idv[q], 1, 64);
            if (q + 1 < Q && lane == 63) {
                en = lane_f(e[q + 1 < Q ? q + 1 : q], 0);
                idn = __builtin_amdgcn_readlane(idv[q + 1 < Q ? q + 1 : q], 0);
            }
            if (i + 1 < lim && idv[q] > idn && !((double)e[q] > (double)en * (1.0 + 0x1p-22)))
                bad = true;
        }
        if (__ballot(bad)) return CF_ORDER;
    }
    QS_TL_HOOK(2);
    // the running sums at both ends of the interval (top-p) and of e (the draw), as lane
    // scans computed together: within lim * 2^-53 of the exact sums, as the reference's
    // sequential sums are, so a sum more than 2^-40 away from top_p compares with it as the
    // reference's does.  Each running sum is monotone in inv.  The sums of e are taken over
    // every position; the draw reads positions below its cut only, where they equal the sums
    // over the kept prefix.
    double clo[Q], chi[Q], ce[Q];
    {
        double carry_lo = 0.0, carry_hi = 0.0, carry_e = 0.0;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int i = q * 64 + lane;
            double a = (double)(i < lim ? e[q] * v_lo : 0.0f);
            double b = (double)(i < lim ? e[q] * v_hi : 0.0f);
            double c = (double)e[q];
            wave_scan3(a, b, c);
            clo[q] = a + carry_lo;
            chi[q] = b + carry_hi;
            ce[q] = c + carry_e;
            carry_lo = lane_d(clo[q], 63);
            carry_hi = lane_d(chi[q], 63);
            carry_e = lane_d(ce[q], 63);
        }
    }
    if (P.top_p < 1.0f) {                                     // sample.c:155-160
        // the cut is proved when the first position that may reach top_p at v_hi surely
        // reaches it at v_lo
        const double tp = (double)P.top_p;
        const double sure = tp * (1.0 + 0x1p-40), maybe = tp * (1.0 - 0x1p-40);
        const int jh = first(0, lim, [&](int q) { return chi[q] >= maybe; });
        if (jh < lim) {
            double cj = 0.0;
#pragma unroll
            for (int q = 0; q < Q; ++q)
                if (q == (jh >> 6)) cj = lane_d(clo[q], jh & 63);
            if (!(cj >= sure)) return CF_TOPP_SPLIT;
            n = jh + 1;
        } else if (n > E) {
            return CF_TOPP_PAST;                              // the cut reads past E
        }
    }
    d.keep_topp = n;
    QS_TL_HOOK(3);
    const float e0 = lane_f(e[0], 0);
    if (P.min_p > 0.0f) {                                     // sample.c:161-168
        const double fl = (double)P.min_p * (double)e0;
        // a floor below the normal range loses the relative bound: not decided here
        if (!(fl * (double)v_lo >= 0x1p-100)) return CF_MINP_FLOOR;
        const double above = fl * (1.0 + 0x1p-21), below = fl * (1.0 - 0x1p-21);
        const int lim2 = min(n, E);
        const int j = first(1, lim2, [&](int q) { return !((double)e[q] >= above); });
        if (j < lim2) {
            if (!((double)e_at(j) < below)) return CF_MINP_SPLIT;
            n = j;
        } else if (n > E) {
            return CF_MINP_PAST;
        }
    }
    if (n < 1) n = 1;
    if (n > E) return CF_KEEP_PAST;
    // the draw (sample.c:170-175) over the running sums of e
    auto ce_at = [&](int i) {
        double v = 0.0;
#pragma unroll
        for (int q = 0; q < Q; ++q)
            if (q == (i >> 6)) v = lane_d(ce[q], i & 63);
        return v;
    };
    const double tot = ce_at(n - 1);
    const double R = u * tot;
    int c = first(0, n, [&](int q) { return R <= ce[q]; });
    if (c >= n) c = n - 1;
    if (c < n - 1 && !(R * (1.0 + 0x1p-22) <= ce_at(c))) return CF_DRAW_HI;
    if (c > 0 && !(R * (1.0 - 0x1p-22) > ce_at(c - 1))) return CF_DRAW_LO;
    int cid = 0;
#pragma unroll
    for (int q = 0; q < Q; ++q)
        if (q == (c >> 6)) cid = __builtin_amdgcn_readlane(idv[q], c & 63);
    rs = rs2;
    id = cid;
    d.keep = n;
    d.rank = c;
    d.u = u;
    d.p0 = e0 * v_lo;
    d.rsum = tot * (double)v_lo;    // the kept mass at v_lo (approximately the reference's)
    return CF_NONE;
}

// The position where the proven prefix ends: the first of [0, m) whose e is not above
// e_rej (1 + 2^-22), the largest numerator any rejected logit can have (0: none of them
// in the window).  Positions before it precede every rejected logit for every inv.
__device__ __forceinline__ bool cert_above_rej(float e, float e_rej) {
    return e_rej <= 0.0f || (double)e > (double)e_rej * (1.0 + 0x1p-22);
}

// Row-level inputs of a certified decision.
struct CertTotals {
    float maxl;      // max penalised logit
    float msc;       // maxl * inv_t
    float v_lo, v_hi;    // the floats the reference's inv can be
    double S_lo, S_hi;   // its softmax denominator lies in [S_lo, S_hi]
    int nwin;        // window size, -1 when unknown
    int cflag;       // some part's candidate list overflowed
    uint32_t rej;    // bound on every logit not among the candidates (key; 0: none)
    int total;       // gathered candidates
};

// The exact numerator of a candidate with penalised logit key `kw` (0 outside the window).
__device__ __forceinline__ float cert_e(uint32_t kw, float inv_t, float msc, float thr,
                                        const uint64_t *tab) {
    const float s = key2f(kw) * inv_t;
    return s >= thr ? qs_expf_core(s - msc, tab) : 0.0f;
}

// Record a decided sampling row (one lane).
__device__ __forceinline__ void cert_record(int row, const qs_row_param &P, const CertTotals &t,
                                            uint64_t rs, int id, int m, qs_pick_diag &d,
                                            int hl, int hh, const RowState &st, int32_t *out,
                                            qs_pick_diag *diag) {
    int32_t *ring = st.ring + (int64_t)row * st.ring_stride;
    st.rng[row] = rs;
    ring_record_at(ring, st.hlen + row, st.hhead + row, P.ring_cap, id, hl, hh);
    out[row] = id;
    if (diag) {
        d.id = id;
        d.path = QS_PATH_CERT;
        d.n_window = t.nwin;
        d.n_cand = m;
        d.maxl = t.maxl;
        d.msc = t.msc;
        d.inv = t.v_lo;
        d.inv_hi = t.v_hi;
        d.sum = t.S_lo;
        d.sum_hi = t.S_hi;
        diag[row] = d;
    }
}

// The end of a one-wavefront certified decision: lane i holds the i-th key of the kept
// candidates in (e desc, id asc) order (0 past them; e = 0 for ids outside the window),
// e_rej bounds the numerator of every id not kept (0: none of them in the window).  The
// proven prefix, then cert_prefix; records the row and returns CF_NONE when decided,
// otherwise the CF_* reason (nothing recorded).
__device__ __forceinline__ int cert_finish_wave(int row, const qs_row_param &P,
                                                const CertTotals &t, uint64_t ek, float e_rej,
                                                const RowState &st, int32_t *out,
                                                qs_pick_diag *diag, const RowHist &h) {
    const int lane = threadIdx.x & 63;
    QS_TL_HOOK(0);
    const int m = __popcll(__ballot((ek >> 32) != 0ull));
    int E = m;
    {
        const uint64_t below = __ballot(lane < m && !cert_above_rej(key_p(ek), e_rej));
        if (below) E = __builtin_ctzll(below);
    }
    const int nwin = t.nwin >= 0 ? t.nwin : (e_rej <= 0.0f ? m : m + 1);
    qs_pick_diag d;
    memset(&d, 0, sizeof d);
    uint64_t rs = h.rng;
    int id = -1;
    const uint64_t kq[1] = {ek};
    QS_TL_HOOK(1);
    const int why = cert_prefix<1>(kq, E, nwin, P, t.v_lo, t.v_hi, rs, id, d);
    QS_TL_HOOK(4);
    if (why != CF_NONE) return why;
    if (lane == 0) {
        CertTotals tt = t;
        tt.nwin = t.nwin >= 0 ? t.nwin : (e_rej <= 0.0f ? m : -1);
        cert_record(row, P, tt, rs, id, m, d, h.len, h.head, st, out, diag);
    }
    return CF_NONE;
}

// The certified decision by one wavefront for rows with top K at most 64 and at most
// WAVE_CAND gathered candidates: the bit-serial bracket keeping the K largest keys and at
// most 64 (dropped keys raise the rejected bound), exact e per lane, a 64-lane sort by
// (e desc, id asc), the proven prefix and cert_prefix.  Returns CF_NONE when decided and
// recorded, otherwise the CF_* reason the caller must take the exact path for.  scratch: 64
// u64 of LDS private to the wavefront.
__device__ __forceinline__ int cert_row_wave(int row, const qs_row_param &P, const CertTotals &t,
                                             const uint32_t *keys, const int32_t *ids,
                                             uint64_t *scratch, const uint64_t *tab,
                                             const RowState &st, int32_t *out,
                                             qs_pick_diag *diag, const RowHist &h) {
    const int lane = threadIdx.x & 63;
    const float inv_t = P.inv_t, msc = t.msc, thr = msc - 30.0f;
    if (t.cflag || t.total > WAVE_CAND || t.total < 1) return CF_INPUT;
    const int K = row_ksel(P);
    if (K > 64) return CF_INPUT;
    uint32_t kk[4];
    int idv[4];
    bool valid[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int j = q * 64 + lane;
        valid[q] = j < t.total;
        kk[q] = valid[q] ? keys[j] : 0u;
        idv[q] = valid[q] ? ids[j] : 0;
    }
    uint32_t th = 0u;
    QS_TL_HOOK(0);
    if (t.total > 64) th = wave_bracket(kk, K, 64, t.total);
    QS_TL_HOOK(1);
    int n_kept = 0;
    uint32_t myrej = 0u;
    bool keep[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        keep[q] = valid[q] && kk[q] >= th;
        if (valid[q] && !keep[q]) myrej = kk[q] > myrej ? kk[q] : myrej;
        n_kept += __popcll(__ballot(keep[q]));
    }
    if (n_kept > 64) return CF_BRACKET;
    const uint32_t wrej = wave_max_u(myrej);
    const uint32_t rej = t.rej > wrej ? t.rej : wrej;
    int base = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint64_t mk = __ballot(keep[q]);
        if (keep[q]) scratch[base + lane_prefix(mk)] = ((uint64_t)kk[q] << 32) | (uint32_t)idv[q];
        base += __popcll(mk);
    }
    __builtin_amdgcn_wave_barrier();
    uint64_t ek = 0ull;
    if (lane < n_kept) {
        const uint64_t v = scratch[lane];
        const float e = cert_e((uint32_t)(v >> 32), inv_t, msc, thr, tab);
        if (e > 0.0f) ek = eid_key(e, (int)(uint32_t)v);
    }
    __builtin_amdgcn_wave_barrier();
    QS_TL_HOOK(2);
    ek = wave_sort_desc(ek);
    QS_TL_HOOK(3);
    const float e_rej = rej > KEY_NEG_INF ? cert_e(rej, inv_t, msc, thr, tab) : 0.0f;
    return cert_finish_wave(row, P, t, ek, e_rej, st, out, diag, h);
}

// The certified decision by the whole block for top K up to K_MAX: radix-select the K
// largest candidate keys (ties kept; the rest raise the rejected bound), exact e, a sort
// of up to 512 (e, id) keys, the proven prefix, then cert_prefix by wavefront 0.  All
// threads call it; returns CF_NONE when decided and recorded, otherwise the CF_* reason.
template <int NT>
__device__ __forceinline__ int cert_row_block(int row, const qs_row_param &P, const CertTotals &t,
                                              uint32_t *keys, int32_t *ids, uint64_t *srt,
                                              DecideLds<NT> &dl, const RowState &st,
                                              int32_t *out, qs_pick_diag *diag,
                                              const RowHist &h) {
    const int tid = threadIdx.x, lane = tid & 63;
    const float inv_t = P.inv_t, msc = t.msc, thr = msc - 30.0f;
    const uint64_t *tab = dl.tab;
    if (t.cflag || t.total < 1) return CF_INPUT;
    const int K = row_ksel(P);
    const uint32_t th = t.total > K ? block_kth<NT>(keys, t.total, K, dl.hist, dl.sh + 4) : 0u;
    if (tid == 0) { dl.sh[3] = 0; dl.shu[0] = t.rej; }
    __syncthreads();
    uint32_t myrej = 0u;
    for (int j0 = 0; j0 < t.total; j0 += NT) {
        const int j = j0 + tid;
        const bool valid = j < t.total;
        const uint32_t kv = valid ? keys[j] : 0u;
        const bool keep = valid && kv >= th;
        if (valid && !keep) myrej = kv > myrej ? kv : myrej;
        const uint64_t mk = __ballot(keep);
        int wbase = 0;
        if (lane == 0 && mk) wbase = atomicAdd(&dl.sh[3], __popcll(mk));
        wbase = __shfl(wbase, 0, 64);
        if (keep) {
            const int pos = wbase + lane_prefix(mk);
            if (pos < 512) {
                const float e = cert_e(kv, inv_t, msc, thr, tab);
                srt[pos] = e > 0.0f ? eid_key(e, ids[j]) : 0ull;
            }
        }
    }
    myrej = wave_max_u(myrej);
    if (lane == 0) atomicMax(&dl.shu[0], myrej);
    __syncthreads();
    const int nkept = dl.sh[3];
    const uint32_t rej = dl.shu[0];
    __syncthreads();
    if (nkept > 512) return CF_WIDE;
    int npad = 64;
    while (npad < nkept) npad <<= 1;
    for (int j = nkept + tid; j < npad; j += NT) srt[j] = 0ull;
    __syncthreads();
    if (npad >= 128 && npad <= NT) {
        block_sort_desc_waves<NT>(srt, npad);
    } else {
        if (tid < 64) {
            if (npad <= 64) wave_sort_lds_desc<1>(srt, npad);
            else if (npad <= 128) wave_sort_lds_desc<2>(srt, npad);
            else if (npad <= 256) wave_sort_lds_desc<4>(srt, npad);
            else wave_sort_lds_desc<8>(srt, npad);
        }
        __syncthreads();
    }
    int status = 1;
    if (tid < 64) {
        uint64_t k8[8];
        const int Q = npad / 64;
#pragma unroll
        for (int q = 0; q < 8; ++q) k8[q] = q < Q ? srt[q * 64 + lane] : 0ull;
        int m = 0;
#pragma unroll
        for (int q = 0; q < 8; ++q) m += __popcll(__ballot((k8[q] >> 32) != 0ull));
        const float e_rej = rej > KEY_NEG_INF ? cert_e(rej, inv_t, msc, thr, tab) : 0.0f;
        int E = m;
        for (int q = 7; q >= 0; --q) {
            const uint64_t b = __ballot(q * 64 + lane < m && !cert_above_rej(key_p(k8[q]), e_rej));
            if (b) E = q * 64 + __builtin_ctzll(b);
        }
        const int nwin = t.nwin >= 0 ? t.nwin : (e_rej <= 0.0f ? m : m + 1);
        qs_pick_diag d;
        memset(&d, 0, sizeof d);
        uint64_t rs = h.rng;
        int id = -1;
        int why;
        if (Q <= 1) {
            const uint64_t kq[1] = {k8[0]};
            why = cert_prefix<1>(kq, E, nwin, P, t.v_lo, t.v_hi, rs, id, d);
        } else if (Q <= 2) {
            const uint64_t kq[2] = {k8[0], k8[1]};
            why = cert_prefix<2>(kq, E, nwin, P, t.v_lo, t.v_hi, rs, id, d);
        } else if (Q <= 4) {
            const uint64_t kq[4] = {k8[0], k8[1], k8[2], k8[3]};
            why = cert_prefix<4>(kq, E, nwin, P, t.v_lo, t.v_hi, rs, id, d);
        } else {
            why = cert_prefix<8>(k8, E, nwin, P, t.v_lo, t.v_hi, rs, id, d);
        }
        const bool ok = why == CF_NONE;
        if (ok && lane == 0) {
            CertTotals tt = t;
            tt.nwin = t.nwin >= 0 ? t.nwin : (e_rej <= 0.0f ? m : -1);
            cert_record(row, P, tt, rs, id, m, d, h.len, h.head, st, out, diag);
        }
        if (lane == 0) dl.sh[7] = why;
    }
    __syncthreads();
    status = dl.sh[7];
    __syncthreads();
    return status;
}

}  // namespace qs
