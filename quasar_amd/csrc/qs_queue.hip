// qs_queue.hip - the pick as one persistent kernel over an ordered task queue.
//
// Every row is cut into S slices of at most NT*NF*4 = 10,240 logits and every
// (row, slice) is two tasks (reference semantics sample.c:111-179):
//
//   scan  streams the slice from HBM into registers: the repeat penalty (history logits
//         set aside and re-entered penalised, sample.c:118-128), the slice max and the
//         row max by atomic max, per-wavefront candidate thresholds and the candidates
//         (every logit at or above the threshold; every other one is below it).  Greedy
//         rows: the slice's first argmax (sample.c:130-134).
//   sum   re-reads the slice (from the last-level cache by then) and, with the row max,
//         computes the exact softmax numerators, double partial sums and window counts
//         (sample.c:136-150).
//
// Rows are grouped in blocks of RB; the queue lists the scans of `lag` blocks ahead of
// the sums:
//
//   scan(0) .. scan(lag-1), sum(0), scan(lag), sum(1), scan(lag+1), ..., sum(nb-1)
//
// so the HBM-bound scans of later rows run beside the VALU-bound sums of earlier rows on
// the same CUs.  Workgroups take tickets (GRAB at a time, the next batch requested while
// the current one runs) from one atomic counter.  A sum waits (bounded) only for the
// scans of its own row: they have lower tickets and never wait, so every wait ends
// whatever order the hardware dispatches workgroups in, and with the lag it is normally
// over before it starts.  The task that completes a row's last sum (greedy rows: the last
// scan) finalizes the row with decide_row.

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "../../include/quasar_sampler.h"
#include "qs_device.h"
#include "qs_expf.h"
#include "qs_internal.h"
#include "qs_launch.h"

using namespace qs;

namespace {

constexpr int NT = 256;                   // threads per workgroup (power of two)
constexpr int NW = NT / 64;
constexpr int NF = 10;                    // float4 registers per thread
constexpr int SLICE_MAX = NT * NF * 4;    // logits per slice
constexpr int SLICE_ALIGN = 64;           // slice starts fall on 256-byte boundaries
constexpr int CPS = QS_OP_CPS;            // candidates kept per slice
constexpr int FIN = 2048;                 // candidates the finalizing workgroup gathers
constexpr int SORTN = 1024;               // candidates it sorts by exact p
constexpr int S_MAX = QS_OP_S_MAX;        // slices per row
constexpr int RB = 8;                     // rows per queue block
constexpr int GRAB = 2;                   // tickets taken at a time
constexpr int TARGET_TASKS = 2048;        // small batches: more slices per row, up to this
constexpr int CAND_BUDGET = 1536;         // expected candidates per row (waves * kw)
constexpr float X_OUT = -150.0f;          // expf core of this rounds to +0

static_assert(FIN % NT == 0, "gather loop");
static_assert(S_MAX <= 64, "one lane per slice");

__constant__ uint64_t c_tab[QS_EXPF_TAB_N] = QS_EXPF_TABLE_INIT;

struct QArgs {
    const float *logits;
    int64_t stride;
    int vocab;
    int n_rows;
    int slices;
    int slice_len;
    int blocks;
    int lag;
    int n_tasks;
    RowState st;
    Scratch sc;
    OpScratch op;
    int32_t *out;
    qs_pick_diag *diag;
};

struct StreamLds {
    uint64_t hm[NT];        // history bits per thread: bit 4j+k = component k of float4 j
    double wsum[NW];
    int wcnt[NW];
    uint32_t wrej[NW];
    uint32_t wmax[NW];
    float wbv[NW];
    int wbi[NW];
    int ncand;
};

struct FinLds {
    uint32_t keys[FIN];
    int32_t ids[FIN];
    uint64_t srt[SORTN];
    int offs[S_MAX + 1];
    RowTotals tot;
    DecideLds<NT> dl;
    FullLds<NT> fl;
};

union QLds {
    StreamLds s;
    FinLds f;
};

// Candidates each wavefront keeps: about twice the share of the row's top K one
// wavefront can expect, plus a margin (the decision proves whatever it is given).
__host__ __device__ __forceinline__ int wave_kw(int K, int waves_per_row) {
    const int kw = 2 * ((K + waves_per_row - 1) / waves_per_row) + 6;
    return kw < 64 ? kw : 64;
}

// Element index of bit b (= 4j + k) of thread tid's registers in a slice starting at lo.
__device__ __forceinline__ int bit_index(int lo, int b, int tid) {
    return lo + 4 * ((b >> 2) * NT + tid) + (b & 3);
}

// Greedy combine for one element visited out of index order: strictly greater, or equal
// at a lower index (a NaN never wins, as in sample.c:132).
__device__ __forceinline__ void greedy_take(float &bv, int &bi, float l, int i) {
    if (l > bv || (l == bv && bi >= 0 && i < bi)) { bv = l; bi = i; }
}

// ---- per-row counters ---------------------------------------------------------------------

// A row's counters share one 256-byte line of their own, so the polls of different rows
// go to different memory channels.
enum { CTR_MAX = 0, CTR_SCANS = 1, CTR_SUMS = 2 };

__device__ __forceinline__ uint32_t *row_ctr(const QArgs &a, int row) {
    return a.op.ctr + (int64_t)row * QS_OP_CTR_STRIDE;
}

__device__ __forceinline__ void reset_row(const QArgs &a, int row) {
    uint32_t *c = row_ctr(a, row);
    st_dev(&c[CTR_MAX], 0u);
    st_dev(&c[CTR_SCANS], 0u);
    st_dev(&c[CTR_SUMS], 0u);
}

// ---- the queue ------------------------------------------------------------------------------

struct Task {
    int sum;      // 0: scan, 1: sum
    int row;
    int slice;
};

__device__ __forceinline__ Task decode(const QArgs &a, int t) {
    const int S = a.slices, T1 = RB * S, nb = a.blocks;
    const int lead = (a.lag < nb ? a.lag : nb);
    const int pairs = nb - lead;
    int sum, blk, idx;
    if (t < lead * T1) {
        sum = 0;
        blk = t / T1;
        idx = t - blk * T1;
    } else {
        const int u = t - lead * T1;
        if (u < pairs * 2 * T1) {
            const int b = u / (2 * T1), w = u - b * 2 * T1;
            sum = w < T1 ? 1 : 0;
            blk = w < T1 ? b : b + lead;
            idx = w < T1 ? w : w - T1;
        } else {
            const int v = u - pairs * 2 * T1;
            sum = 1;
            blk = pairs + v / T1;
            idx = v - (v / T1) * T1;
        }
    }
    Task k;
    k.sum = sum;
    k.row = blk * RB + idx / S;
    k.slice = idx - (idx / S) * S;
    return k;
}

// ---- one slice in registers --------------------------------------------------------------

template <bool VEC>
__device__ __forceinline__ void issue_slice(float4 (&v)[NF], const float *x, int lo, int hi) {
    const int tid = threadIdx.x, c0 = lo >> 2;
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        const int c = c0 + j * NT + tid;
        if (VEC) {
            const float q = __builtin_nanf("");
            v[j] = (c << 2) < hi ? *((const float4 *)x + c) : make_float4(q, q, q, q);
        } else {
            v[j] = load4<false>(x, c, hi);
        }
    }
}

// History ids of the slice as bits of their owning thread (returned), with those logits
// set to NaN in the registers: they re-enter, penalised, from the bits.  All threads call
// this; it holds the workgroup barriers of the scatter (at least one).
__device__ __forceinline__ uint64_t set_aside_history(float4 (&v)[NF], const QArgs &a, int row,
                                                      const qs_row_param &P, int lo, int hi,
                                                      StreamLds &ls) {
    const int tid = threadIdx.x;
    const int hlen = a.st.hlen[row];
    const bool pen = P.repeat_penalty > 1.0f && hlen > 0 && P.ring_cap > 0;
    if (!pen) {
        __syncthreads();
        return 0ull;
    }
    ls.hm[tid] = 0ull;
    __syncthreads();
    const int head = a.st.hhead[row], cap = P.ring_cap;
    const int32_t *ring = a.st.ring + (int64_t)row * a.st.ring_stride;
    for (int q = tid; q < hlen; q += NT) {
        const int id = ring[(head + q) % cap];
        if (id >= lo && id < hi) {
            const int p = id - lo, c = p >> 2;
            atomicOr((unsigned long long *)&ls.hm[c & (NT - 1)],
                     1ull << ((c / NT) * 4 + (p & 3)));
        }
    }
    __syncthreads();
    const uint64_t hm = ls.hm[tid];
    const float qnan = __builtin_nanf("");
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        const uint32_t nib = (uint32_t)(hm >> (4 * j)) & 15u;
        if (__ballot(nib != 0u)) {
            if (nib & 1u) v[j].x = qnan;
            if (nib & 2u) v[j].y = qnan;
            if (nib & 4u) v[j].z = qnan;
            if (nib & 8u) v[j].w = qnan;
        }
    }
    return hm;
}

// ---- the finalizing workgroup ----------------------------------------------------------------

__device__ __forceinline__ void finalize_greedy(const QArgs &a, int row, const qs_row_param &P) {
    const int lane = threadIdx.x & 63;
    if (threadIdx.x >= 64) return;
    const int S = a.slices, l0 = row * S;
    float bv = -INFINITY;
    int bi = -1;
    if (lane < S) {
        bv = ld_dev(&a.op.bestv[l0 + lane]);
        bi = ld_dev(&a.op.besti[l0 + lane]);
    }
    wave_best(bv, bi);
    if (lane == 0) {
        const float *x = a.logits + (int64_t)row * a.stride;
        record_greedy(row, P, bv, bi, bv, x[0], a.st, a.out, a.diag);
        reset_row(a, row);
    }
}

__device__ __forceinline__ void finalize_sampling(const QArgs &a, int row, const qs_row_param &P,
                                                  FinLds &f) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int S = a.slices, l0 = row * S;
    if (tid < QS_EXPF_TAB_N) f.dl.tab[tid] = c_tab[tid];
    if (tid < 64) {
        // Row totals from the S slices; the double sum is a butterfly over slice
        // positions, so it does not depend on which workgroup finished when.
        const bool have = lane < S;
        double ps = have ? ld_dev(&a.op.psum[l0 + lane]) : 0.0;
        int pc = have ? ld_dev(&a.op.pcnt[l0 + lane]) : 0;
        int cc = have ? ld_dev(&a.op.ccnt[l0 + lane]) : 0;
        uint32_t cr = have ? ld_dev(&a.op.rej[l0 + lane]) : 0u;
        const int cf = wave_or_i((cc >> 30) & 1);
        cc &= 0x3FFFFFFF;
        ps = wave_sum_d(ps);
        pc = wave_sum_i(pc);
        cr = wave_max_u(cr);
        int incl = cc;
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(incl, o, 64);
            if (lane >= o) incl += t;
        }
        if (have) f.offs[lane] = incl - cc;
        if (lane == 63) f.offs[S] = incl;
        if (lane == 0) {
            f.tot.maxl = key2f(ld_dev(&row_ctr(a, row)[CTR_MAX]));
            f.tot.sum = ps;
            f.tot.nwin = pc;
            f.tot.cflag = cf;
            f.tot.rej = cr;
        }
    }
    __syncthreads();
    RowTotals t = f.tot;
    t.total = f.offs[S];
    if (t.total <= FIN && isfinite(t.maxl * P.inv_t)) {
        // Gather the slice lists: every load is issued before any is stored to LDS.
        uint32_t kk[FIN / NT];
        int32_t ii[FIN / NT];
#pragma unroll
        for (int q = 0; q < FIN / NT; ++q) {
            const int g = q * NT + tid;
            kk[q] = 0u;
            ii[q] = 0;
            if (g < t.total) {
                int lo = 0, hi = S;                          // last s with offs[s] <= g
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (f.offs[mid] <= g) lo = mid; else hi = mid - 1;
                }
                const int64_t src = (int64_t)(l0 + lo) * CPS + (g - f.offs[lo]);
                kk[q] = ld_dev(&a.op.ckey[src]);
                ii[q] = ld_dev(&a.op.cid[src]);
            }
        }
#pragma unroll
        for (int q = 0; q < FIN / NT; ++q) {
            const int g = q * NT + tid;
            if (g < t.total) {
                f.keys[g] = kk[q];
                f.ids[g] = ii[q];
            }
        }
    }
    __syncthreads();
    const float *x = a.logits + (int64_t)row * a.stride;
    decide_row_fast<NT, SORTN>(row, P, t, FIN, f.keys, f.ids, f.srt, f.dl, f.fl, x, a.vocab,
                               a.st, a.sc, a.out, a.diag, -1);
    if (tid == 0) reset_row(a, row);
}

// ---- the two tasks -----------------------------------------------------------------------

template <bool VEC>
__device__ __forceinline__ void scan_task(const QArgs &a, int row, int slice, QLds &u,
                                          int &s_fin) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int S = a.slices, task = row * S + slice;
    const qs_row_param P = a.st.prm[row];
    const int lo = slice * a.slice_len;
    const int hi = min(lo + a.slice_len, a.vocab);
    const float *x = a.logits + (int64_t)row * a.stride;
    const float rp = P.repeat_penalty;

    float4 v[NF];
    issue_slice<VEC>(v, x, lo, hi);
    if (tid == 0) u.s.ncand = 0;
    const uint64_t hm = set_aside_history(v, a, row, P, lo, hi, u.s);

    if (row_greedy(P)) {
        float bv = -INFINITY;
        int bi = -1;
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            const int i0 = lo + 4 * (j * NT + tid);
            if (v[j].x > bv) { bv = v[j].x; bi = i0; }
            if (v[j].y > bv) { bv = v[j].y; bi = i0 + 1; }
            if (v[j].z > bv) { bv = v[j].z; bi = i0 + 2; }
            if (v[j].w > bv) { bv = v[j].w; bi = i0 + 3; }
        }
        for (uint64_t m = hm; m; m &= m - 1) {
            const int i = bit_index(lo, __builtin_ctzll(m), tid);
            greedy_take(bv, bi, penalise(x[i], rp), i);
        }
        wave_best(bv, bi);
        if (lane == 0) {
            u.s.wbv[wv] = bv;
            u.s.wbi[wv] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            float b0 = u.s.wbv[0];
            int i0 = u.s.wbi[0];
            for (int k = 1; k < NW; ++k) best_combine(b0, i0, u.s.wbv[k], u.s.wbi[k]);
            st_dev(&a.op.bestv[task], b0);
            st_dev(&a.op.besti[task], i0);
            stores_done();
            s_fin = add_dev(&row_ctr(a, row)[CTR_SCANS], 1u) == (uint32_t)S - 1;
        }
        __syncthreads();
        if (s_fin) finalize_greedy(a, row, P);
        return;
    }

    // thread maxima (history logits penalised) and the wavefront's threshold
    float m4[NF];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        m4[j] = fmaxf(fmaxf(v[j].x, v[j].y), fmaxf(v[j].z, v[j].w));
        mx = fmaxf(mx, m4[j]);
    }
    for (uint64_t m = hm; m; m &= m - 1) {
        const int i = bit_index(lo, __builtin_ctzll(m), tid);
        mx = fmaxf(mx, penalise(x[i], rp));
    }
    const int kw = wave_kw(row_ksel(P), S * NW);
    const uint32_t mk = f2key(mx);
    uint32_t th = 0u;
    for (int b = 31; b >= 0; --b) {
        const uint32_t c = th | (1u << b);
        if (__popcll(__ballot(mk >= c)) >= kw) th = c;
    }
    if (th <= KEY_NEG_INF) th = KEY_NEG_INF + 1u;   // -inf and NaN never qualify
    const float thf = key2f(th);
    uint32_t *ck = a.op.ckey + (int64_t)task * CPS;
    int32_t *ci = a.op.cid + (int64_t)task * CPS;
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        if (__ballot(m4[j] >= thf)) {
            const int i0 = lo + 4 * (j * NT + tid);
            const float w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (w[k] >= thf) {
                    const int pos = atomicAdd(&u.s.ncand, 1);
                    if (pos < CPS) {
                        st_dev(&ck[pos], f2key(w[k]));
                        st_dev(&ci[pos], i0 + k);
                    }
                }
            }
        }
    }
    for (uint64_t m = hm; m; m &= m - 1) {
        const int i = bit_index(lo, __builtin_ctzll(m), tid);
        const float l = penalise(x[i], rp);
        if (l >= thf) {
            const int pos = atomicAdd(&u.s.ncand, 1);
            if (pos < CPS) {
                st_dev(&ck[pos], f2key(l));
                st_dev(&ci[pos], i);
            }
        }
    }
    const float wmax = wave_max_f(mx);
    if (lane == 0) {
        u.s.wmax[wv] = f2key(wmax);
        u.s.wrej[wv] = th - 1u;
    }
    stores_done();
    __syncthreads();
    if (tid == 0) {
        uint32_t k = u.s.wmax[0], r = u.s.wrej[0];
        for (int q = 1; q < NW; ++q) {
            k = u.s.wmax[q] > k ? u.s.wmax[q] : k;
            r = u.s.wrej[q] > r ? u.s.wrej[q] : r;
        }
        const int n = u.s.ncand;
        uint32_t *c = row_ctr(a, row);
        __hip_atomic_fetch_max(&c[CTR_MAX], k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        st_dev(&a.op.rej[task], r);
        st_dev(&a.op.ccnt[task], (n < CPS ? n : CPS) | (n > CPS ? (1 << 30) : 0));
        stores_done();                      // the max and the lists before the arrival
        add_dev(&c[CTR_SCANS], 1u);
    }
}

template <bool VEC>
__device__ __forceinline__ void sum_task(const QArgs &a, int row, int slice, QLds &u,
                                         const uint64_t *tab, int &s_fin, uint32_t &s_rowmax) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int S = a.slices, task = row * S + slice;
    const qs_row_param P = a.st.prm[row];
    if (row_greedy(P)) return;                      // decided by its scans
    const int lo = slice * a.slice_len;
    const int hi = min(lo + a.slice_len, a.vocab);
    const float *x = a.logits + (int64_t)row * a.stride;
    const float rp = P.repeat_penalty;

    float4 v[NF];
    issue_slice<VEC>(v, x, lo, hi);
    if (tid == 0) {
        // the row's scans (lower tickets, never waiting) have normally finished long ago
        uint32_t *c = row_ctr(a, row);
        for (int it = 0; ld_dev(&c[CTR_SCANS]) < (uint32_t)S; ++it) {
            if (it >= SPIN_LIMIT) {
                atomicOr(a.sc.err, 8);
                break;
            }
            __builtin_amdgcn_s_sleep(8);
        }
        s_rowmax = ld_dev(&c[CTR_MAX]);
    }
    const uint64_t hm = set_aside_history(v, a, row, P, lo, hi, u.s);   // barriers inside

    const float maxl = key2f(s_rowmax);
    const float inv_t = P.inv_t;
    const float msc = maxl * inv_t;
    const float thr = msc - 30.0f;
    double acc0 = 0.0, acc1 = 0.0;
    int cnt = 0;
    if (isfinite(msc)) {
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            const float s0 = v[j].x * inv_t, s1 = v[j].y * inv_t;
            const float s2 = v[j].z * inv_t, s3 = v[j].w * inv_t;
            const bool i0 = s0 >= thr, i1 = s1 >= thr, i2 = s2 >= thr, i3 = s3 >= thr;
            if (__ballot(i0 || i1 || i2 || i3)) {
                const float e0 = qs_expf_core(i0 ? s0 - msc : X_OUT, tab);
                const float e1 = qs_expf_core(i1 ? s1 - msc : X_OUT, tab);
                const float e2 = qs_expf_core(i2 ? s2 - msc : X_OUT, tab);
                const float e3 = qs_expf_core(i3 ? s3 - msc : X_OUT, tab);
                acc0 += (double)e0;
                acc1 += (double)e1;
                acc0 += (double)e2;
                acc1 += (double)e3;
                cnt += (int)i0 + (int)i1 + (int)i2 + (int)i3;
            }
        }
        for (uint64_t m = hm; m; m &= m - 1) {
            const int i = bit_index(lo, __builtin_ctzll(m), tid);
            const float s = penalise(x[i], rp) * inv_t;
            if (s >= thr) {
                acc0 += (double)qs_expf_core(s - msc, tab);
                ++cnt;
            }
        }
    }
    const double ws = wave_sum_d(acc0 + acc1);
    const int wc = wave_sum_i(cnt);
    if (lane == 0) {
        u.s.wsum[wv] = ws;
        u.s.wcnt[wv] = wc;
    }
    __syncthreads();
    if (tid == 0) {
        double tsum = 0.0;
        int tc = 0;
        for (int k = 0; k < NW; ++k) {
            tsum += u.s.wsum[k];
            tc += u.s.wcnt[k];
        }
        st_dev(&a.op.psum[task], tsum);
        st_dev(&a.op.pcnt[task], tc);
        stores_done();
        s_fin = add_dev(&row_ctr(a, row)[CTR_SUMS], 1u) == (uint32_t)S - 1;
    }
    __syncthreads();
    if (s_fin) finalize_sampling(a, row, P, u.f);
}

// ---- the kernel -------------------------------------------------------------------------------

// Four wavefronts per SIMD: 128 VGPRs hold the ten float4 and the exp pipeline unspilled.
template <bool VEC>
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4, 4)))
k_queue(QArgs a) {
    __shared__ QLds u;
    __shared__ uint64_t tab[QS_EXPF_TAB_N];
    __shared__ int s_t, s_fin;
    __shared__ uint32_t s_rowmax;

    const int tid = threadIdx.x;
    if (tid < QS_EXPF_TAB_N) tab[tid] = c_tab[tid];
    __syncthreads();
    (void)s_t;
    for (int t = blockIdx.x; t < a.n_tasks; t += gridDim.x) {
        const Task k = decode(a, t);
        if (k.row >= a.n_rows) continue;
        if (k.sum) sum_task<VEC>(a, k.row, k.slice, u, tab, s_fin, s_rowmax);
        else scan_task<VEC>(a, k.row, k.slice, u, s_fin);
        __syncthreads();
    }
}

int slices_min(int n_vocab) { return (n_vocab + SLICE_MAX - 1) / SLICE_MAX; }

}  // namespace

// ---- host side ----------------------------------------------------------------------------------

int qs_queue_geometry(int n_rows, int n_vocab, int kmax, int *slice_len) {
    const int s_min = slices_min(n_vocab);
    if (s_min > S_MAX) return 0;
    int s = (TARGET_TASKS + n_rows - 1) / n_rows;
    if (s > S_MAX) s = S_MAX;
    if (s < s_min) s = s_min;
    for (;;) {
        int len = (n_vocab + s - 1) / s;
        len = (len + SLICE_ALIGN - 1) / SLICE_ALIGN * SLICE_ALIGN;
        const int slices = (n_vocab + len - 1) / len;
        const int waves = slices * NW;
        if (slices <= s_min || waves * wave_kw(kmax, waves) <= CAND_BUDGET) {
            *slice_len = len;
            return slices;
        }
        s = slices - 1;
        if (s < s_min) s = s_min;
    }
}

int qs_queue_slice_cap(int max_rows, int max_vocab) {
    const int a = ((max_rows + RB - 1) / RB * RB) * slices_min(max_vocab);
    const int b = TARGET_TASKS + max_rows + RB * S_MAX;
    return a > b ? a : b;
}

int qs_queue_grid(void) {
    int dev = 0, ncu = 0, nb0 = 0, nb1 = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb0, k_queue<true>, NT, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb1, k_queue<false>, NT, 0) != hipSuccess)
        return 0;
    const int nb = nb0 < nb1 ? nb0 : nb1;
    return nb * ncu;
}

int qs_queue_launch(const float *logits, int64_t row_stride, int n_rows, int n_vocab, int kmax,
                    const RowState &st, const Scratch &sc, const OpScratch &op, int32_t *out,
                    qs_pick_diag *diag, int grid_cap, int lag_rows, hipStream_t stream) {
    int slice_len = 0;
    const int slices = qs_queue_geometry(n_rows, n_vocab, kmax, &slice_len);
    if (slices < 1 || slices > S_MAX || slice_len > SLICE_MAX || grid_cap < 1) {
        qs_set_error("queue pick: vocabulary %d does not fit %d slices of %d", n_vocab, S_MAX,
                     SLICE_MAX);
        return QS_EINVAL;
    }
    QArgs a;
    a.logits = logits;
    a.stride = row_stride;
    a.vocab = n_vocab;
    a.n_rows = n_rows;
    a.slices = slices;
    a.slice_len = slice_len;
    a.blocks = (n_rows + RB - 1) / RB;
    if ((int64_t)a.blocks * RB * slices > op.slice_cap) {
        qs_set_error("queue pick: %d rows x %d slices exceed the scratch (%d)", n_rows, slices,
                     op.slice_cap);
        return QS_EDEVICE;
    }
    // scans run `lag` blocks ahead of the sums: about half a grid of tasks by default
    int lag = lag_rows > 0 ? (lag_rows + RB - 1) / RB
                           : (grid_cap / 2 + RB * slices - 1) / (RB * slices);
    if (lag < 1) lag = 1;
    a.lag = lag;
    a.n_tasks = 2 * a.blocks * RB * slices;
    a.st = st;
    a.sc = sc;
    a.op = op;
    a.out = out;
    a.diag = diag;
    const int grid = a.n_tasks < grid_cap ? a.n_tasks : grid_cap;
    const bool vec = ((uintptr_t)logits % 16 == 0) && (row_stride % 4 == 0) && (n_vocab % 4 == 0);
    if (vec)
        hipLaunchKernelGGL(k_queue<true>, dim3(grid), dim3(NT), 0, stream, a);
    else
        hipLaunchKernelGGL(k_queue<false>, dim3(grid), dim3(NT), 0, stream, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        qs_set_error("queue pick launch: %s", hipGetErrorString(e));
        return QS_EDEVICE;
    }
    return 0;
}
