// qs_onepass.hip - the one-pass pick: every logit is read from HBM once.
//
// A pick of B rows is B*S tasks, one per (row, slice) of at most NT*NF*4 = 10,240 logits.
// The grid is resident (sized from the occupancy) and split into gangs of S workgroups
// with the same index mod 8, i.e. on one XCD when workgroups are dealt to the XCDs
// round-robin.  Gang q handles rows q, q + gangs, q + 2*gangs, ...: its S members load
// the S slices of a row together, so the one wait of a task (for the row max) lasts about
// as long as the atomics that carry it.
//
// Per task (256 threads, 10 float4 registers each), reference semantics sample.c:111-179:
//   1. Load the slice into registers with 16-byte loads; scatter the row's history ids
//      that fall in the slice into per-thread LDS bit masks.
//   2. History logits are set aside in the registers (NaN) and handled from the bit masks
//      with the repeat penalty applied (sample.c:118-128), so the register pass needs no
//      per-element penalty test.
//   3. Slice max (greedy rows: the first argmax, sample.c:130-134).  Per wavefront, a
//      candidate threshold: the kw-th largest of the 64 lane maxima, so kw distinct
//      logits of the wavefront reach it; every logit at or above it is written out as a
//      candidate, and every other one is below it.
//   4. The row max is combined with atomics over the row's wavefronts; each wavefront
//      waits (bounded) until all of them have published.
//   5. Exact softmax numerators expf(x*inv_t - msc) straight from the registers, double
//      partial sums and window counts (sample.c:136-150).
//   6. The workgroup that completes a row's last task finalizes the row: totals in fixed
//      slice order, decide_row over the gathered candidates (top-K by logit, exact p,
//      proof of the prefix, cuts, draw), the history record.

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
constexpr int SLICE_MAX = NT * NF * 4;    // logits per task
constexpr int SLICE_ALIGN = 64;           // slice starts fall on 256-byte boundaries
constexpr int CPS = QS_OP_CPS;            // candidates kept per slice
constexpr int FIN = 2048;                 // candidates the finalizing workgroup gathers
constexpr int SORTN = 1024;               // candidates it sorts by exact p
constexpr int S_MAX = QS_OP_S_MAX;        // slices per row
constexpr int TARGET_TASKS = 2048;        // small batches: more slices per row, up to this
constexpr int CAND_BUDGET = 1536;         // expected candidates per row (waves * kw)
constexpr float X_OUT = -150.0f;          // expf core of this rounds to +0

static_assert(FIN % NT == 0, "gather loop");
static_assert(S_MAX <= 64, "one lane per slice");

__constant__ uint64_t c_tab[QS_EXPF_TAB_N] = QS_EXPF_TABLE_INIT;

struct OpArgs {
    const float *logits;
    int64_t stride;
    int vocab;
    int n_rows;
    int slices;
    int slice_len;
    int gangs;
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

union OpLds {
    StreamLds s;
    FinLds f;
};

// Candidates each wavefront keeps: about twice the share of the row's top K one
// wavefront can expect, plus a margin (the decision proves whatever it is given).
__host__ __device__ __forceinline__ int wave_kw(int K, int waves_per_row) {
    const int kw = 2 * ((K + waves_per_row - 1) / waves_per_row) + 6;
    return kw < 64 ? kw : 64;
}

template <bool VEC>
__device__ __forceinline__ float4 slice_load(const float *x, int c, int hi) {
    if (VEC) {
        if ((c << 2) < hi) return *((const float4 *)x + c);
        const float q = __builtin_nanf("");
        return make_float4(q, q, q, q);
    }
    return load4<false>(x, c, hi);
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

// ---- the finalizing workgroup ----------------------------------------------------------------

// A row's counters share one 256-byte line of their own: rows poll different lines, so
// no memory channel serves every poll of the grid.
__device__ __forceinline__ uint32_t *row_ctr(const OpArgs &a, int row) {
    return a.op.ctr + (int64_t)row * QS_OP_CTR_STRIDE;
}
enum { CTR_MAX = 0, CTR_ARRIVE = 1, CTR_DONE = 2 };

__device__ __forceinline__ void reset_row(const OpArgs &a, int row) {
    uint32_t *c = row_ctr(a, row);
    st_dev(&c[CTR_MAX], 0u);
    st_dev(&c[CTR_ARRIVE], 0u);
    st_dev(&c[CTR_DONE], 0u);
}

__device__ __forceinline__ void finalize_row(const OpArgs &a, int row, const qs_row_param &P,
                                             bool greedy, FinLds &f) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int S = a.slices, l0 = row * S;
    const float *x = a.logits + (int64_t)row * a.stride;
    if (greedy) {                                            // sample.c:130-134
        if (tid < 64) {
            float bv = -INFINITY;
            int bi = -1;
            if (lane < S) {
                bv = ld_dev(&a.op.bestv[l0 + lane]);
                bi = ld_dev(&a.op.besti[l0 + lane]);
            }
            wave_best(bv, bi);
            if (lane == 0) {
                record_greedy(row, P, bv, bi, bv, x[0], a.st, a.out, a.diag);
                reset_row(a, row);
            }
        }
        return;
    }
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
    decide_row_fast<NT, SORTN>(row, P, t, FIN, f.keys, f.ids, f.srt, f.dl, f.fl, x, a.vocab,
                               a.st, a.sc, a.out, a.diag, -1);
    if (tid == 0) reset_row(a, row);
}

// ---- the kernel -------------------------------------------------------------------------------

// Four wavefronts per SIMD: 128 VGPRs hold the ten float4 and the exp pipeline unspilled.
template <bool VEC>
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4, 4)))
k_onepass(OpArgs a) {
    __shared__ OpLds u;
    __shared__ uint64_t tab[QS_EXPF_TAB_N];
    __shared__ int s_fin;
    __shared__ uint32_t s_wmax[NW], s_rowmax;

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int S = a.slices;
    const float qnan = __builtin_nanf("");
    if (tid < QS_EXPF_TAB_N) tab[tid] = c_tab[tid];
    const int xcd = blockIdx.x & 7, j8 = blockIdx.x >> 3;
    const int gang = (j8 / S) * 8 + xcd;
    const int slice = j8 % S;

    for (int row = gang; row < a.n_rows; row += a.gangs) {
        const int task = row * S + slice;
        const qs_row_param P = a.st.prm[row];
        const bool greedy = row_greedy(P);
        const int lo = slice * a.slice_len;
        const int hi = min(lo + a.slice_len, a.vocab);
        const float *x = a.logits + (int64_t)row * a.stride;
        const int c0 = lo >> 2;

        // 1. the slice, into registers
        float4 v[NF];
#pragma unroll
        for (int j = 0; j < NF; ++j) v[j] = slice_load<VEC>(x, c0 + j * NT + tid, hi);

        // history ids of the slice, as bits of the owning thread
        const float rp = P.repeat_penalty;
        const int hlen = a.st.hlen[row];
        const bool pen = rp > 1.0f && hlen > 0 && P.ring_cap > 0;
        if (tid == 0) u.s.ncand = 0;
        uint64_t hm = 0ull;
        if (pen) {
            u.s.hm[tid] = 0ull;
            __syncthreads();
            const int head = a.st.hhead[row], cap = P.ring_cap;
            const int32_t *ring = a.st.ring + (int64_t)row * a.st.ring_stride;
            for (int q = tid; q < hlen; q += NT) {
                const int id = ring[(head + q) % cap];
                if (id >= lo && id < hi) {
                    const int p = id - lo, c = p >> 2;
                    atomicOr((unsigned long long *)&u.s.hm[c & (NT - 1)],
                             1ull << ((c / NT) * 4 + (p & 3)));
                }
            }
            __syncthreads();
            hm = u.s.hm[tid];
            // 2. set the history logits aside: they re-enter penalised from the bit list
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
        } else {
            __syncthreads();
        }

        if (greedy) {
            // 3g. first argmax of the slice
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
            }
        } else {
            // 3s. thread maxima (history logits penalised) and the wave's threshold
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

            // 4. the row max over every workgroup of the row: one atomic max and one
            // arrival per workgroup, one poller
            const float wmax = wave_max_f(mx);
            if (lane == 0) s_wmax[wv] = f2key(wmax);
            __syncthreads();
            if (tid == 0) {
                uint32_t k = s_wmax[0];
                for (int q = 1; q < NW; ++q) k = s_wmax[q] > k ? s_wmax[q] : k;
                uint32_t *c = row_ctr(a, row);
                // the max is performed before the arrival that announces it
                __hip_atomic_fetch_max(&c[CTR_MAX], k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                stores_done();
                add_dev(&c[CTR_ARRIVE], 1u);
                for (int it = 0; ld_dev(&c[CTR_ARRIVE]) < (uint32_t)S; ++it) {
                    if (it >= SPIN_LIMIT) {
                        atomicOr(a.sc.err, 4);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(4);
                }
                s_rowmax = ld_dev(&c[CTR_MAX]);
            }
            __syncthreads();
            const uint32_t rk = s_rowmax;

            // 5. softmax numerators from the registers
            const float maxl = key2f(rk);
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
                u.s.wrej[wv] = th - 1u;
            }
            __syncthreads();
            if (tid == 0) {
                double tsum = 0.0;
                int tc = 0;
                uint32_t tr = 0u;
                for (int k = 0; k < NW; ++k) {
                    tsum += u.s.wsum[k];
                    tc += u.s.wcnt[k];
                    tr = u.s.wrej[k] > tr ? u.s.wrej[k] : tr;
                }
                const int n = u.s.ncand;
                st_dev(&a.op.psum[task], tsum);
                st_dev(&a.op.pcnt[task], tc);
                st_dev(&a.op.rej[task], tr);
                st_dev(&a.op.ccnt[task], (n < CPS ? n : CPS) | (n > CPS ? (1 << 30) : 0));
            }
        }

        // 6. publish the task; the last of the row finalizes it
        stores_done();
        __syncthreads();
        if (tid == 0) s_fin = add_dev(&row_ctr(a, row)[CTR_DONE], 1u) == (uint32_t)S - 1;
        __syncthreads();
        if (s_fin) finalize_row(a, row, P, greedy, u.f);
        __syncthreads();
    }
}

int slices_min(int n_vocab) { return (n_vocab + SLICE_MAX - 1) / SLICE_MAX; }

}  // namespace

// ---- host side ----------------------------------------------------------------------------------

int qs_onepass_geometry(int n_rows, int n_vocab, int kmax, int per_xcd, int *slice_len) {
    int s_min = slices_min(n_vocab);
    if (s_min > S_MAX) return 0;
    // the smallest slice count that divides the per-XCD capacity, when there is one
    for (int d = s_min; d <= S_MAX && d <= per_xcd; ++d)
        if (per_xcd % d == 0) { s_min = d; break; }
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

int qs_onepass_slice_cap(int max_rows, int max_vocab) {
    // slices per row never exceed twice the minimum (the divisor search) or S_MAX
    int s = 2 * slices_min(max_vocab);
    if (s > S_MAX) s = S_MAX;
    const int a = max_rows * s;
    const int b = TARGET_TASKS + max_rows;
    return a > b ? a : b;
}

int qs_onepass_grid(void) {
    int dev = 0, ncu = 0, nb0 = 0, nb1 = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb0, k_onepass<true>, NT, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb1, k_onepass<false>, NT, 0) != hipSuccess)
        return 0;
    const int nb = nb0 < nb1 ? nb0 : nb1;
    return nb * ncu;
}

int qs_onepass_launch(const float *logits, int64_t row_stride, int n_rows, int n_vocab, int kmax,
                      const RowState &st, const Scratch &sc, const OpScratch &op, int32_t *out,
                      qs_pick_diag *diag, int grid_cap, hipStream_t stream) {
    int slice_len = 0;
    const int per_xcd = grid_cap / 8;
    const int slices = qs_onepass_geometry(n_rows, n_vocab, kmax, per_xcd, &slice_len);
    if (slices < 1 || slices > S_MAX || slice_len > SLICE_MAX || per_xcd < slices) {
        qs_set_error("one-pass pick: vocabulary %d does not fit %d slices of %d", n_vocab,
                     S_MAX, SLICE_MAX);
        return QS_EINVAL;
    }
    if ((int64_t)n_rows * slices > op.slice_cap) {
        qs_set_error("one-pass pick: %d rows x %d slices exceed the scratch (%d)", n_rows,
                     slices, op.slice_cap);
        return QS_EDEVICE;
    }
    OpArgs a;
    a.logits = logits;
    a.stride = row_stride;
    a.vocab = n_vocab;
    a.n_rows = n_rows;
    a.slices = slices;
    a.slice_len = slice_len;
    // gangs of `slices` workgroups, the same number on every XCD, all resident
    const int per_xcd_gangs = per_xcd / slices;
    int gx = (n_rows + 7) / 8;
    if (gx > per_xcd_gangs) gx = per_xcd_gangs;
    a.gangs = 8 * gx;
    a.st = st;
    a.sc = sc;
    a.op = op;
    a.out = out;
    a.diag = diag;
    const int grid = a.gangs * slices;
    const bool vec = ((uintptr_t)logits % 16 == 0) && (row_stride % 4 == 0) && (n_vocab % 4 == 0);
    if (vec)
        hipLaunchKernelGGL(k_onepass<true>, dim3(grid), dim3(NT), 0, stream, a);
    else
        hipLaunchKernelGGL(k_onepass<false>, dim3(grid), dim3(NT), 0, stream, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        qs_set_error("one-pass pick launch: %s", hipGetErrorString(e));
        return QS_EDEVICE;
    }
    return 0;
}
