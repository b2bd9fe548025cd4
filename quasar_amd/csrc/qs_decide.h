// qs_decide.h - what a row's decision needs beside its candidates (device code, included
// by the streaming kernels): the decision workgroup's LDS, the visit of a row's penalised
// logits, the exact softmax denominator and the exact path for rows the certified decision
// does not cover (sample.c:118-178).
//
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "../../include/quasar_sampler.h"
#include "qs_cert.h"
#include "qs_device.h"
#include "qs_launch.h"

namespace qs {
namespace dec {

// The timeline build (make timeline: -DQS_TIMELINE) records the 100 MHz clock at the
// phases of each decision (rows below TL_ROWS; one copy per translation unit).
#ifdef QS_TIMELINE
constexpr int TL_ROWS = 4096;
static __device__ uint64_t g_tl_dec[TL_ROWS * 8];
#define QS_DEC_MARK(e)                                                                        \
    do {                                                                                      \
        if (threadIdx.x == 0 && blockIdx.x < qs::dec::TL_ROWS) {                              \
            qs::dec::g_tl_dec[blockIdx.x * 8 + (e)] = __builtin_amdgcn_s_memrealtime();       \
            if ((e) == 0)                                                                     \
                qs::dec::g_tl_dec[blockIdx.x * 8 + 5] = qs::dec::g_tl_dec[blockIdx.x * 8 + 6] = 0; \
        }                                                                                     \
    } while (0)
#else
#define QS_DEC_MARK(e) ((void)0)
#endif

constexpr int ND = 256;              // threads per decision workgroup
constexpr int FCAP = 2048;           // candidates a row's decision gathers
constexpr int SCAP = 512;            // candidates the exact decision sorts in LDS
constexpr int XUP = 8;               // float4 per thread per chunk of the exact recount
constexpr int XCHUNK = ND * XUP * 4; // elements per load round of the exact recount
constexpr int XBM = 4 * XCHUNK;      // elements per history bitmap block of it

// History bitmap words of `len` logits (one bit per logit, in whole 16-byte groups).
__host__ __device__ constexpr int bitmap_words(int len) { return (len / 32 + 1 + 3) / 4 * 4; }

struct PartArgs {
    const float *logits;
    int64_t stride;
    int vocab;
    int n_rows;
    int parts;
    int part_len;                    // elements per part (a multiple of 4)
    int xcd_map;                     // 1: the parts of a row on one XCD (rows >= 8)
    RowState st;
    Scratch sc;
    int32_t *out;
    qs_pick_diag *diag;
};

// ---- the decision --------------------------------------------------------------------------

struct DecLds {
    uint32_t keys[FCAP];
    int32_t ids[FCAP];
    uint64_t srt[SCAP];
    uint32_t bm[bitmap_words(XBM)];
    DecideLds<ND> dl;
    int offs[QS_PART_MAX_PARTS + 1];
    CertTotals ct;
    double exs[ND / 64];
    int exc[ND / 64];
    float bv[ND / 64];
    int bi[ND / 64];
    uint32_t pmaxk[QS_PART_MAX_PARTS];   // per part: max key, rejection bound, sums, min, NaNs
    uint32_t prej[QS_PART_MAX_PARTS];
    double psum[QS_PART_MAX_PARTS];
    float pterm[QS_PART_MAX_PARTS];
    uint32_t pmin[QS_PART_MAX_PARTS];
    int pnan[QS_PART_MAX_PARTS];
    int gcount;                          // decide_par: candidates gathered
};
static_assert(sizeof(FullLds<ND>) <= sizeof(uint32_t) * 2 * FCAP, "full-window LDS aliases keys/ids");

// Visit the row's penalised logits (f(w, id) on every thread's share; all threads): in
// blocks of XBM logits, each with its history bitmap in LDS, read XUP float4s per thread at
// a time with every load issued before the first is used.
template <typename F>
__device__ __forceinline__ void row_visit(const PartArgs &a, int row, const qs_row_param &P,
                                          DecLds &dl, F &&f) {
    const int tid = threadIdx.x;
    const float rp = P.repeat_penalty;
    const int cap = P.ring_cap;                   // (clamped: row_param)
    int len, head;
    ring_pos(a.st, row, cap, len, head);
    const bool pen = rp > 1.0f && len > 0 && cap > 0;
    const int32_t *ring = a.st.ring + (int64_t)row * a.st.ring_stride;
    const float4 *x4 = (const float4 *)(a.logits + (int64_t)row * a.stride);
    for (int lo = 0; lo < a.vocab; lo += XBM) {
        const int hi = min(lo + XBM, a.vocab), c_hi = hi >> 2;
        if (pen) {                                    // sample.c:118-120: each id once
            for (int j = tid; j < bitmap_words(XBM); j += ND) dl.bm[j] = 0u;
            __syncthreads();
            for (int j = tid; j < len; j += ND) {
                const int id = ring[qs_ring_slot(cap, head, j)];
                if (id >= lo && id < hi) atomicOr(&dl.bm[(id - lo) >> 5], 1u << ((id - lo) & 31));
            }
            __syncthreads();
        }
        for (int c0 = (lo >> 2) + tid; c0 < c_hi; c0 += ND * XUP) {
            float4 v[XUP];
#pragma unroll
            for (int k = 0; k < XUP; ++k) {
                const int c = c0 + k * ND;
                v[k] = c < c_hi ? x4[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int k = 0; k < XUP; ++k) {
                const int c = c0 + k * ND;
                if (c >= c_hi) break;
                float w[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
                const int q = 4 * c - lo;
                const uint32_t nib = pen ? (dl.bm[q >> 5] >> (q & 31)) & 0xFu : 0u;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if ((nib >> e) & 1u) w[e] = penalise(w[e], rp);
                    f(w[e], 4 * c + e);
                }
            }
        }
        if (pen) __syncthreads();                     // the block's bitmap is read
    }
}

// The row's exact softmax denominator and window size (sample.c:136-149), recomputed from
// the logits with the host-libm-equal expf: for rows the certified decision does not cover.
// All threads; the sums reduce in a fixed order.  That order's sum and the reference's
// (ids ascending) are sums of the same n nonnegative binary64 numbers, each within
// (n - 1) 2^-53 of their exact total, so the two differ by at most 2 n 2^-53 of it; where
// (float)(1 / x) is the same float at both ends of that reach it is the reference's inv
// (1 / x and both roundings are monotone), and where it is not (or sc.sum_in_order asks
// for it) the sum is taken again in id order.
__device__ __forceinline__ void exact_totals(const PartArgs &a, int row, const qs_row_param &P, float msc,
                             DecLds &dl, double &sum, int &nwin) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float inv_t = P.inv_t, thr = msc - 30.0f;
    double acc = 0.0;
    int cnt = 0;
    row_visit(a, row, P, dl, [&](float w, int) {
        const float s = w * inv_t;
        if (s >= thr) {
            acc += (double)qs_expf_core(s - msc, dl.dl.tab);
            ++cnt;
        }
    });
    acc = wave_sum_d(acc);
    cnt = wave_sum_i(cnt);
    if (lane == 0) { dl.exs[wv] = acc; dl.exc[wv] = cnt; }
    __syncthreads();
    double s = 0.0;
    int c = 0;
    for (int j = 0; j < ND / 64; ++j) { s += dl.exs[j]; c += dl.exc[j]; }
    sum = s;
    nwin = c;
    __syncthreads();
    if (a.sc.sum_in_order || !inv_settled(s, c))   // (uniform)
        sum = sum_in_id_order<ND, XBM>(a.logits + (int64_t)row * a.stride, a.vocab, a.st, row,
                                       P, msc, dl.bm, dl.dl.tab, &dl.exs[0]);
}

// The block's (largest value, first index) of (v, i) pairs; i < 0: none.  All threads.
__device__ __forceinline__ void block_best(float &v, int &i, DecLds &dl) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    wave_best(v, i);
    if (lane == 0) { dl.bv[wv] = v; dl.bi[wv] = i; }
    __syncthreads();
    v = -INFINITY;
    i = -1;
    for (int j = 0; j < ND / 64; ++j) best_combine(v, i, dl.bv[j], dl.bi[j]);
    __syncthreads();
}

// The exact path (all threads): the row's exact denominator, then the reference's decision
// over the gathered candidates (or the whole window); `status` is the reason the certified
// decision gave up, kept in the diagnostics.
__device__ __forceinline__ void exact_row(const PartArgs &a, int row, const qs_row_param &P,
                                          const CertTotals &t, DecLds &dl, const RowHist &hist,
                                          int status) {
    FullLds<ND> &fl = *(FullLds<ND> *)dl.keys;       // aliases keys/ids (dead by then)
    RowTotals rt;
    rt.maxl = t.maxl;
    rt.sum = 0.0;
    rt.nwin = 0;
    rt.cflag = t.cflag;
    rt.rej = t.rej;
    rt.total = t.total;
    if (isfinite(t.msc)) exact_totals(a, row, P, t.msc, dl, rt.sum, rt.nwin);
    QS_DEC_MARK(5);
    decide_row_fast<ND, SCAP, false>(row, P, rt, FCAP, dl.keys, dl.ids, dl.srt, dl.dl, fl,
                                     a.logits + (int64_t)row * a.stride, a.vocab, a.st, a.sc,
                                     a.out, a.diag, -1, &hist);
    QS_DEC_MARK(6);
    __syncthreads();
    if (threadIdx.x == 0 && a.diag) a.diag[row].fallback = status;
}

}  // namespace dec
}  // namespace qs
