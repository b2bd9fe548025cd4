// qs_batch.hip - the device batch: per-row state in HBM, the split-row kernels, and the C
// ABI (include/quasar_sampler.h, parts 2 and 3).
//
// One pick of B rows (reference semantics: sample.c:111-179), each row cut into S slices:
//
//   k_scan     grid S x B  Stream the slice once with 16-byte loads, apply the repeat
//                          penalty from an LDS bitmap of the history, reduce the slice max
//                          (greedy rows: the first argmax).  Sampling rows also record a
//                          candidate threshold: the 2K-th largest of the 256 per-thread
//                          maxima, so at least 2K logits of the slice reach it.
//   k_expsum   grid S x B  Second pass over the slice (from the last-level cache at these
//                          sizes): exact softmax numerators expf(x*inv_t - msc) with the
//                          host-libm-equal expf, double partial sums, window counts, and
//                          every logit at or above the threshold kept as a candidate.
//   k_finalize grid B      Row totals; radix-select the row's top K candidates by logit,
//                          their exact p, a bitonic sort by (p desc, id asc), a proof that
//                          no rejected logit can reach a position the cuts read, then
//                          top-k / top-p / min-p / the draw exactly as sample.c, and the
//                          history record.  Rows the proof does not cover (large nucleus,
//                          probability ties across the threshold, non-finite maxima) are
//                          finished in the same workgroup over the whole window, sorted in
//                          a scratch slot.
//
// Generator states and history rings stay on the device.  Floating point follows the
// reference bit for bit: -ffp-contract=off, correctly rounded float division, IEEE
// denormals, the expf of qs_expf.h.

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/quasar_sampler.h"
#include "qs_device.h"
#include "qs_expf.h"
#include "qs_gen.h"
#include "qs_internal.h"
#include "qs_launch.h"

using namespace qs;

namespace {

constexpr int WG = 256;              // threads per workgroup of the split kernels
constexpr int NW = WG / 64;
constexpr int U = 4;                 // 16-byte loads in flight per thread per step
constexpr int SLOTS = 16;            // full-window scratch slots (2V u64 + V bits each)
constexpr int S_MAX = 64;            // slices per row
constexpr int SLICE_QUANT = 1024;    // slice length granularity (elements)
constexpr int TARGET_WGS = 2048;     // workgroups k_scan aims for
constexpr int SLICE_MAX = 1 << 18;   // longest slice (its history bitmap lives in LDS)
constexpr int CCAP = 2048;           // candidates kept per slice
constexpr int FIN_CAP = 4096;        // candidates k_finalize gathers per row

__constant__ uint64_t c_exp_tab[QS_EXPF_TAB_N] = QS_EXPF_TABLE_INIT;

// ---- streaming helpers ---------------------------------------------------------------------

// One group of U float4 per thread: float4 c = cb + u*WG + tid; logits at or past `hi`
// read as NaN.
template <bool VEC>
__device__ __forceinline__ void load_group(float4 (&v)[U], const float *x, int cb, int hi) {
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = load4<VEC>(x, cb + u * WG + (int)threadIdx.x, hi);
}

// A group that lies wholly inside the slice: plain 16-byte loads, no tests.
__device__ __forceinline__ void load_full(float4 (&v)[U], const float *x, int cb) {
    const float4 *x4 = (const float4 *)x;
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = x4[cb + u * WG + (int)threadIdx.x];
}

// Stream [lo, hi) of row x through fn(group, cb) in groups of WG*U float4, in index
// order.  With 16-byte loads (VEC: aligned rows, hi a multiple of 4) the full groups run
// in a branch-free loop that always has the next group's loads in flight, so each wait
// names the exact count of loads still outstanding; the partial tail group is loaded
// with bounds tests.
template <bool VEC, typename Fn>
__device__ __forceinline__ void stream_slice(const float *x, int lo, int hi, Fn &&fn) {
    constexpr int G = WG * U;
    const int c0 = lo >> 2, c1 = (hi + 3) >> 2;
    int cb = c0;
    float4 va[U], vb[U];
    if (VEC) {
        const int nfull = (c1 - c0) / G;
        if (nfull >= 1) {
            load_full(va, x, cb);
            int g = 0;
            for (; g + 2 < nfull; g += 2) {       // va holds group g; g+1, g+2 exist
                load_full(vb, x, cb + G);
                fn(va, cb);
                load_full(va, x, cb + 2 * G);
                fn(vb, cb + G);
                cb += 2 * G;
            }
            if (g + 1 < nfull) {
                load_full(vb, x, cb + G);
                fn(va, cb);
                fn(vb, cb + G);
                cb += 2 * G;
            } else {
                fn(va, cb);
                cb += G;
            }
        }
    }
    for (; cb < c1; cb += G) {
        load_group<VEC>(va, x, cb, hi);
        fn(va, cb);
    }
}

// History bits of the four logits starting at element i0 (LDS bitmap of [lo, hi)).
__device__ __forceinline__ uint32_t hist_nibble(const uint32_t *bm, int i0, int lo, int hi) {
    if (i0 >= hi) return 0u;
    const int r = i0 - lo;
    return (bm[r >> 5] >> (r & 31)) & 0xFu;
}

// sample.c:124 on the flagged components of one float4 (a wave-uniform skip when no lane
// of the wavefront has a flagged component).
__device__ __forceinline__ void penalise4(float (&w)[4], uint32_t nib, float rp) {
    if (__ballot(nib != 0u)) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            if ((nib >> k) & 1u) w[k] = penalise(w[k], rp);
    }
}

// ---- k_scan --------------------------------------------------------------------------------

// Max (greedy: first argmax) over one group of a slice.
template <bool GREEDY>
__device__ __forceinline__ void scan_group(const float4 (&v)[U], int cb, int lo, int hi,
                                           const uint32_t *bm, bool pen, float rp, float &mx,
                                           float &bv, int &bi) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int i0 = (cb + u * WG + (int)threadIdx.x) << 2;
        float w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
        if (pen) penalise4(w, hist_nibble(bm, i0, lo, hi), rp);
#pragma unroll
        for (int k = 0; k < 4; ++k) mx = w[k] > mx ? w[k] : mx;
        if (GREEDY) {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (w[k] > bv) { bv = w[k]; bi = i0 + k; }
        }
    }
}

template <bool VEC, bool GREEDY>
__device__ __forceinline__ void scan_slice(const float *x, int lo, int hi, const uint32_t *bm,
                                           bool pen, float rp, float &mx, float &bv, int &bi) {
    stream_slice<VEC>(x, lo, hi, [&](const float4 (&v)[U], int cb) {
        scan_group<GREEDY>(v, cb, lo, hi, bm, pen, rp, mx, bv, bi);
    });
}

template <bool VEC>
__global__ void __launch_bounds__(WG) k_scan(Geometry g, RowState st, Scratch sc) {
    extern __shared__ uint32_t lds[];
    __shared__ float red_f[NW];
    __shared__ int red_i[NW];
    __shared__ uint32_t tmax[WG];
    __shared__ uint32_t hist[256];
    __shared__ int sh[2];

    const int slice = blockIdx.x, row = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const qs_row_param P = row_param(st, row);
    const bool greedy = row_greedy(P);
    const int lo = slice * g.slice_len;
    const int hi = min(lo + g.slice_len, g.vocab);
    const float rp = P.repeat_penalty;
    const bool pen = rp > 1.0f && st.hlen[row] > 0 && P.ring_cap > 0;
    uint32_t *bm = lds;
    if (pen) build_bitmap<WG>(bm, g.bm_words, lo, hi, st, row, P.ring_cap);

    const float *x = g.logits + (int64_t)row * g.stride;
    float mx = -INFINITY;                 // max penalised logit of this thread
    float bv = -INFINITY;                 // greedy: best value, first index
    int bi = -1;
    if (greedy) scan_slice<VEC, true>(x, lo, hi, bm, pen, rp, mx, bv, bi);
    else scan_slice<VEC, false>(x, lo, hi, bm, pen, rp, mx, bv, bi);

    const float m = wave_max_f(mx);
    if (lane == 0) red_f[wv] = m;
    __syncthreads();
    if (tid == 0) {
        float t = red_f[0];
        for (int k = 1; k < NW; ++k) t = fmaxf(t, red_f[k]);
        sc.smax[row * g.slices + slice] = t;
    }
    if (greedy) {
        wave_best(bv, bi);
        __syncthreads();
        if (lane == 0) { red_f[wv] = bv; red_i[wv] = bi; }
        __syncthreads();
        if (tid == 0) {
            float v0 = red_f[0];
            int i0 = red_i[0];
            for (int k = 1; k < NW; ++k) best_combine(v0, i0, red_f[k], red_i[k]);
            sc.bestv[row * g.slices + slice] = v0;
            sc.besti[row * g.slices + slice] = i0;
        }
        return;
    }
    // Candidate threshold: the k-th largest thread maximum.  Those k maxima are k distinct
    // logits of the slice, so the slice's top k all lie at or above it.  k is about twice
    // the slice's share of the row's top K plus a margin: the decision proves whatever it
    // gets, and a row whose top K crowd into one slice takes the full-window path.
    tmax[tid] = f2key(mx);
    __syncthreads();
    const int k2 = min(2 * ((row_ksel(P) + g.slices - 1) / g.slices) + 8, WG);
    const uint32_t th = block_kth<WG>(tmax, WG, k2, hist, sh);
    if (tid == 0) sc.sth[row * g.slices + slice] = th;
}

// ---- k_expsum ------------------------------------------------------------------------------

constexpr float X_OUT = -150.0f;     // qs_expf_core of this rounds to +0

struct SumState {
    double acc0, acc1;               // partial softmax denominators (two chains)
    int cnt;                         // window count of the wavefront (uniform)
    int ovf;                         // candidate list overflowed
};

// Softmax numerators, window count and candidates of one group (sample.c:136-148 per
// element).  Out-of-window lanes evaluate the exp core at X_OUT, which is exactly +0.
__device__ __forceinline__ void sum_group(const float4 (&v)[U], int cb, int lo, int hi,
                                          const uint32_t *bm, bool pen, float rp, float inv_t,
                                          float msc, float thr, float thf, const uint64_t *tab,
                                          uint32_t *ckey, int32_t *cid, int *ncand,
                                          SumState &ss) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int i0 = (cb + u * WG + (int)threadIdx.x) << 2;
        float w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
        if (pen) penalise4(w, hist_nibble(bm, i0, lo, hi), rp);
        float s[4];
        bool in[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            s[k] = w[k] * inv_t;
            in[k] = s[k] >= thr;
            ss.cnt += __popcll(__ballot(in[k]));
        }
        if (__ballot(in[0] | in[1] | in[2] | in[3])) {
            float e[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) e[k] = qs_expf_core(in[k] ? s[k] - msc : X_OUT, tab);
            ss.acc0 += (double)e[0];
            ss.acc1 += (double)e[1];
            ss.acc0 += (double)e[2];
            ss.acc1 += (double)e[3];
        }
        const float m4 = fmaxf(fmaxf(w[0], w[1]), fmaxf(w[2], w[3]));
        if (__ballot(m4 >= thf)) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const bool cand = w[k] >= thf;
                const uint64_t mk = __ballot(cand);
                if (mk) {
                    int base = 0;
                    if (lane == 0) base = atomicAdd(ncand, __popcll(mk));
                    base = __shfl(base, 0, 64);
                    if (cand) {
                        const int pos = base + lane_prefix(mk);
                        if (pos < CCAP) {
                            ckey[pos] = f2key(w[k]);
                            cid[pos] = i0 + k;
                        } else {
                            ss.ovf = 1;
                        }
                    }
                }
            }
        }
    }
}

template <bool VEC>
__global__ void __launch_bounds__(WG) k_expsum(Geometry g, RowState st, Scratch sc) {
    extern __shared__ uint32_t lds[];
    __shared__ uint64_t tab[QS_EXPF_TAB_N];
    __shared__ double red_d[NW];
    __shared__ int red_i[NW];
    __shared__ int ncand;

    const int slice = blockIdx.x, row = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const qs_row_param P = row_param(st, row);
    if (row_greedy(P)) return;
    const int li = row * g.slices + slice;

    float maxl = -INFINITY;
    for (int s = 0; s < g.slices; ++s) maxl = fmaxf(maxl, sc.smax[row * g.slices + s]);
    const float inv_t = P.inv_t;
    const float msc = maxl * inv_t;
    const float thr = msc - 30.0f;
    if (!isfinite(msc)) {                  // k_finalize handles these rows on its own
        if (tid == 0) {
            sc.psum[li] = 0.0;
            sc.pcnt[li] = 0;
            sc.ccnt[li] = 0;
            sc.cflag[li] = 0;
            sc.crej[li] = 0u;
        }
        return;
    }
    const int lo = slice * g.slice_len;
    const int hi = min(lo + g.slice_len, g.vocab);
    const float *x = g.logits + (int64_t)row * g.stride;
    if (tid < QS_EXPF_TAB_N) tab[tid] = c_exp_tab[tid];
    if (tid == 0) ncand = 0;
    const float rp = P.repeat_penalty;
    const bool pen = rp > 1.0f && st.hlen[row] > 0 && P.ring_cap > 0;
    uint32_t *bm = lds;
    uint32_t *ckey = lds + g.bm_words;
    int32_t *cid = (int32_t *)(ckey + CCAP);
    if (pen) build_bitmap<WG>(bm, g.bm_words, lo, hi, st, row, P.ring_cap);
    __syncthreads();
    const uint32_t th = sc.sth[li];
    const float thf = th > KEY_NEG_INF ? key2f(th) : -INFINITY;

    SumState ss{0.0, 0.0, 0, 0};
    stream_slice<VEC>(x, lo, hi, [&](const float4 (&v)[U], int cb) {
        sum_group(v, cb, lo, hi, bm, pen, rp, inv_t, msc, thr, thf, tab, ckey, cid, &ncand, ss);
    });
    const double a = wave_sum_d(ss.acc0 + ss.acc1);
    const int o = wave_or_i(ss.ovf);
    if (lane == 0) { red_d[wv] = a; red_i[wv] = ss.cnt | (o << 30); }
    __syncthreads();
    const int n = min(ncand, CCAP);
    uint32_t *gk = sc.ckey + (int64_t)li * sc.ccap;
    int32_t *gi = sc.cid + (int64_t)li * sc.ccap;
    for (int j = tid; j < n; j += WG) {
        gk[j] = ckey[j];
        gi[j] = cid[j];
    }
    if (tid == 0) {
        double t = 0.0;
        int ct = 0, fl = 0;
        for (int k = 0; k < NW; ++k) {
            t += red_d[k];
            ct += red_i[k] & 0x3FFFFFFF;
            fl |= red_i[k] >> 30;
        }
        sc.psum[li] = t;
        sc.pcnt[li] = ct;
        sc.ccnt[li] = n;
        sc.cflag[li] = fl;
        // every logit of the slice below the threshold was rejected
        sc.crej[li] = th > KEY_NEG_INF ? th - 1u : 0u;
    }
}

// ---- k_finalize ----------------------------------------------------------------------------

struct FinArgs {
    Geometry g;
    RowState st;
    Scratch sc;
    int32_t *out;
    qs_pick_diag *diag;
};

__global__ void __launch_bounds__(WG) k_finalize(FinArgs a) {
    __shared__ uint32_t keys[FIN_CAP];
    __shared__ int32_t ids[FIN_CAP];
    __shared__ uint64_t srt[SORT_CAP];
    __shared__ int offs[S_MAX + 1];
    __shared__ RowTotals tot;
    __shared__ float gbv;
    __shared__ int gbi;
    __shared__ DecideLds<WG> dl;
    __shared__ FullLds<WG> fl;

    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const Geometry &g = a.g;
    const Scratch &sc = a.sc;
    const RowState &st = a.st;
    const qs_row_param P = row_param(st, row);
    const int S = g.slices;
    const int l0 = row * S;
    if (tid < QS_EXPF_TAB_N) dl.tab[tid] = c_exp_tab[tid];

    // Row totals from the S slices (wave 0; S <= 64).  The double sum is a fixed
    // butterfly over slice positions, so it does not depend on timing.
    if (tid < 64) {
        const bool have = lane < S;
        float mx = have ? sc.smax[l0 + lane] : -INFINITY;
        mx = wave_max_f(mx);
        if (row_greedy(P)) {
            float bv = have ? sc.bestv[l0 + lane] : -INFINITY;
            int bi = have ? sc.besti[l0 + lane] : -1;
            wave_best(bv, bi);
            if (lane == 0) { gbv = bv; gbi = bi; tot.maxl = mx; }
        } else {
            double ps = have ? sc.psum[l0 + lane] : 0.0;
            int pc = have ? sc.pcnt[l0 + lane] : 0;
            int cc = have ? sc.ccnt[l0 + lane] : 0;
            int cf = have ? sc.cflag[l0 + lane] : 0;
            uint32_t cr = have ? sc.crej[l0 + lane] : 0u;
            ps = wave_sum_d(ps);
            pc = wave_sum_i(pc);
            cf = wave_or_i(cf);
            cr = wave_max_u(cr);
            int incl = cc;                     // prefix of candidate counts over slices
            for (int o = 1; o < 64; o <<= 1) {
                const int t = __shfl_up(incl, o, 64);
                if (lane >= o) incl += t;
            }
            if (have) offs[lane] = incl - cc;
            if (lane == 63) offs[S] = incl;
            if (lane == 0) {
                tot.maxl = mx;
                tot.sum = ps;
                tot.nwin = pc;
                tot.cflag = cf;
                tot.rej = cr;
            }
        }
    }
    __syncthreads();
    const float *x = g.logits + (int64_t)row * g.stride;
    if (row_greedy(P)) {                                   // sample.c:130-134
        if (tid == 0) record_greedy(row, P, gbv, gbi, tot.maxl, x[0], st, a.out, a.diag);
        return;
    }
    // the reference's inv where the slices' fixed-order sum does not settle it
    {
        constexpr int BLK = 32768;                         // bitmap block: in fl (not yet used)
        static_assert(sizeof(FullLds<WG>) >= BLK / 8, "the bitmap in fl");
        const float msc = tot.maxl * P.inv_t;
        if (isfinite(msc) && (sc.sum_in_order || !inv_settled(tot.sum, tot.nwin))) {
            __shared__ double xch;
            const double s = sum_in_id_order<WG, BLK>(x, g.vocab, st, row, P, msc,
                                                      (uint32_t *)&fl, dl.tab, &xch);
            if (tid == 0) tot.sum = s;
            __syncthreads();
        }
    }
    RowTotals t = tot;
    t.total = offs[S];
    if (t.total <= FIN_CAP && isfinite(t.maxl * P.inv_t)) {
        // Gather the slice lists: every load is issued before any is stored to LDS.
        uint32_t kk[FIN_CAP / WG];
        int32_t ii[FIN_CAP / WG];
#pragma unroll
        for (int q = 0; q < FIN_CAP / WG; ++q) {
            const int j = q * WG + tid;
            kk[q] = 0u;
            ii[q] = 0;
            if (j < t.total) {
                int lo = 0, hi = S;                        // last s with offs[s] <= j
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (offs[mid] <= j) lo = mid; else hi = mid - 1;
                }
                const int64_t src = (int64_t)(l0 + lo) * sc.ccap + (j - offs[lo]);
                kk[q] = sc.ckey[src];
                ii[q] = sc.cid[src];
            }
        }
#pragma unroll
        for (int q = 0; q < FIN_CAP / WG; ++q) {
            const int j = q * WG + tid;
            if (j < t.total) {
                keys[j] = kk[q];
                ids[j] = ii[q];
            }
        }
    }
    __syncthreads();
    decide_row_fast<WG, SORT_CAP, true>(row, P, t, FIN_CAP, keys, ids, srt, dl, fl, x, g.vocab, st, sc, a.out,
                        a.diag, -1);
}

// ---- synthetic inputs and the expf check ---------------------------------------------------

__global__ void __launch_bounds__(WG) k_gen(float *out, int64_t stride, int64_t row0,
                                            int n_rows, int vocab, qs_gen_spec spec) {
    const int64_t idx = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (idx >= (int64_t)n_rows * vocab) return;
    const int64_t r = idx / vocab;
    const int c = (int)(idx - r * vocab);
    out[r * stride + c] = qs_gen_logit(&spec, (uint64_t)(row0 + r), c, vocab);
}

// A plain streaming copy (16-byte loads and stores), for calibrating memory counters.
__global__ void __launch_bounds__(WG) k_copy(const float4 *x, float4 *y, int64_t n4) {
    for (int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x; i < n4; i += (int64_t)gridDim.x * WG)
        y[i] = x[i];
}

// The copy in 4-byte elements (plain global loads of one dword).
__global__ void __launch_bounds__(WG) k_copy1(const float *x, float *y, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x; i < n; i += (int64_t)gridDim.x * WG)
        y[i] = x[i];
}

// The same copy with the loads of the sampler's streaming kernels, for counter calibration:
// a raw buffer load of 16 bytes, nontemporal (the row kernel's), or that load written
// straight into LDS (the streaming part kernel's), each over a buffer resource spanning the
// workgroup's float4s (loads past it read no memory).
constexpr int CP_WORD3 = 0x00020000;     // raw buffer, 32-bit data format
constexpr int CP_NT = 2;                 // nontemporal
typedef unsigned int cp_u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void cp_lds_void;
template <bool LDS>
__global__ void __launch_bounds__(WG) k_copy_buf(const float4 *x, float4 *y, int64_t n4) {
    __shared__ float4 st[WG];
    const int tid = threadIdx.x;
    for (int64_t c = (int64_t)blockIdx.x * WG; c < n4; c += (int64_t)gridDim.x * WG) {
        const int64_t left = n4 - c;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(x + c), 0, (int)((left < WG ? left : WG) * 16), CP_WORD3);
        float4 v;
        if constexpr (LDS) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (cp_lds_void *)(st + (tid & ~63)), 16,
                                                     tid * 16, 0, 0, CP_NT);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            const volatile float *q = (const volatile float *)&st[tid];
            v = make_float4(q[0], q[1], q[2], q[3]);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // read before reloaded
        } else {
            const cp_u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(rs, tid * 16, 0, CP_NT);
            v = make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                            __uint_as_float(u.w));
        }
        if (tid < left) y[c + tid] = v;
    }
}

// A one-row pick's result for the host: its id and the batch's error flag stored by one
// thread into pinned host memory (h: the device's address of it), in place of two
// device-to-host copies.
__global__ void __launch_bounds__(64) k_result1(const int32_t *out, const int32_t *err,
                                                int32_t *h) {
    if (threadIdx.x == 0) {
        h[0] = out[0];
        h[1] = err[0];
    }
}

// The kernels' expf, element by element.  Inside [-33, 0] the pipelined kernel's 4-wide
// window variant (qs_expf4_window, extended table) runs too, and a result different from
// qs_expf_tab's is reported as NaN, so the comparison with the host C library covers both.
__global__ void __launch_bounds__(WG) k_expf(const float *x, float *y, int64_t n) {
    __shared__ uint64_t tab[QS_EXPF_TAB_N];
    __shared__ uint64_t xtab[QS_EXPF_XTAB_N];
    if (threadIdx.x < QS_EXPF_TAB_N) tab[threadIdx.x] = c_exp_tab[threadIdx.x];
    __syncthreads();
    for (int j = threadIdx.x; j < QS_EXPF_XTAB_N; j += WG) xtab[j] = qs_expf_xtab_entry(tab, j);
    __syncthreads();
    const int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (i < n) {
        const float v = x[i];
        float r = qs_expf_tab(v, tab);
        if (v <= 0.0f && v >= -33.0f) {
            const float a[4] = {v, v, v, v};
            float e[4];
            qs_expf4_window(a, e, xtab);
            if (__float_as_uint(e[0]) != __float_as_uint(r)) r = __builtin_nanf("");
        }
        y[i] = r;
    }
}

// ---- host side ----------------------------------------------------------------------------

int hip_fail(hipError_t e, const char *what) {
    qs_set_error("%s: %s", what, hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? QS_ENOMEM : QS_EDEVICE;
}

#define HIP_TRY(call, what)                                  \
    do {                                                     \
        hipError_t e_ = (call);                              \
        if (e_ != hipSuccess) return hip_fail(e_, (what));   \
    } while (0)

template <typename T>
int dev_alloc(T **p, size_t n, const char *what) {
    *p = nullptr;
    if (n == 0) n = 1;
    hipError_t e = hipMalloc((void **)p, n * sizeof(T));
    if (e != hipSuccess) { *p = nullptr; return hip_fail(e, what); }
    return 0;
}

int slices_for(int n_rows, int vocab, int kmax_sel, int *slice_len) {
    int s = (TARGET_WGS + n_rows - 1) / n_rows;
    if (s > S_MAX) s = S_MAX;
    // each slice contributes about 2K candidates; k_finalize gathers FIN_CAP
    const int cap = FIN_CAP / (3 * kmax_sel);
    if (s > cap) s = cap;
    if (s < 1) s = 1;
    const int s_min = (vocab + SLICE_MAX - 1) / SLICE_MAX;
    if (s < s_min) s = s_min;
    int len = (vocab + s - 1) / s;
    len = (len + SLICE_QUANT - 1) / SLICE_QUANT * SLICE_QUANT;
    *slice_len = len;
    return (vocab + len - 1) / len;
}

}  // namespace

struct qs_batch {
    int max_rows = 0, max_vocab = 0, max_last_n = 0;
    int mode = QS_MODE_AUTO;               // QS_MODE_*: which kernels a pick uses
    int slice_rows = 0;                    // capacity of the per-slice / per-part scratch
    int part_resident = 0;                 // resident workgroups of the streaming kernel
    int n_cu = 0;                          // the device's CUs (the row kernel's batch floor)
    bool row8 = false;                     // two 8-wavefront row workgroups fit on a CU
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    hipEvent_t mid = nullptr;              // recorded between the streaming pick's kernels
    std::vector<qs_row_param> h_prm;
    qs_row_param *d_prm = nullptr;
    uint64_t *d_rng = nullptr;
    int32_t *d_ring = nullptr, *d_hlen = nullptr, *d_hhead = nullptr;
    Scratch sc{};
    HeadRec *d_hrec = nullptr;             // the output layer's per-(row, tile) records
    uint32_t *d_hbits = nullptr;           // its history bitmap (zero between picks)
    bool hbits_dirty = false;              // a fused pick failed after marking it: clear
                                           // it before the next one
    int32_t *h_pin = nullptr;              // pinned: a one-row pick's id and error flag
    int32_t *d_pin = nullptr;              // the device's address of h_pin
};

static void batch_release(qs_batch *b) {
    if (!b) return;
    if (b->stream) (void)hipStreamSynchronize(b->stream);
    void *ptrs[] = {b->d_prm, b->d_rng, b->d_ring, b->d_hlen, b->d_hhead, b->sc.smax,
                    b->sc.bestv, b->sc.besti, b->sc.sth, b->sc.ckey, b->sc.cid, b->sc.ccnt,
                    b->sc.crej, b->sc.cflag, b->sc.psum, b->sc.pcnt, b->sc.locks,
                    b->sc.full_keys, b->sc.full_bm, b->sc.err, b->sc.wrec,
                    b->sc.pcand, b->sc.gbest, b->sc.gmaxk, b->sc.gcnt, b->d_hrec,
                    b->d_hbits};
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    if (b->h_pin) (void)hipHostFree(b->h_pin);
    if (b->ev0) (void)hipEventDestroy(b->ev0);
    if (b->ev1) (void)hipEventDestroy(b->ev1);
    if (b->stream) (void)hipStreamDestroy(b->stream);
    delete b;
}

static int batch_alloc(qs_batch *b) {
    const int R = b->max_rows, V = b->max_vocab;
    // rows*slices is at most max(R, min(TARGET_WGS, S_MAX*R)); the streaming kernel needs
    // rows*parts
    int sr = R;
    const int many = TARGET_WGS < S_MAX * R ? TARGET_WGS : S_MAX * R;
    if (many > sr) sr = many;
    const int np = qs_part_parts(V);
    if ((int64_t)np * R > sr) sr = np * R;
    b->slice_rows = sr;
    b->part_resident = qs_part_resident();
    if (b->part_resident < 1) b->part_resident = 512;
    {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&b->n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            b->n_cu < 1)
            b->n_cu = 256;
    }
    b->row8 = qs_row_resident(8) >= 2;
    // a few whole-window slots behind the slot locks: rows that need one are rare and
    // each holder is a running workgroup
    b->sc.nslots = R < SLOTS ? R : SLOTS;
    b->sc.ccap = CCAP;
    b->sc.spin_limit = SPIN_LIMIT;
    int rc = 0;
    if (!rc) rc = dev_alloc(&b->d_prm, R, "params");
    if (!rc) rc = dev_alloc(&b->d_rng, R, "rng");
    if (!rc) rc = dev_alloc(&b->d_ring, (size_t)R * (b->max_last_n > 0 ? b->max_last_n : 1), "ring");
    if (!rc) rc = dev_alloc(&b->d_hlen, R, "hlen");
    if (!rc) rc = dev_alloc(&b->d_hhead, R, "hhead");
    if (!rc) rc = dev_alloc(&b->sc.smax, sr, "smax");
    if (!rc) rc = dev_alloc(&b->sc.bestv, sr, "bestv");
    if (!rc) rc = dev_alloc(&b->sc.besti, sr, "besti");
    if (!rc) rc = dev_alloc(&b->sc.sth, sr, "sth");
    if (!rc) rc = dev_alloc(&b->sc.ckey, (size_t)sr * CCAP, "ckey");
    if (!rc) rc = dev_alloc(&b->sc.cid, (size_t)sr * CCAP, "cid");
    if (!rc) rc = dev_alloc(&b->sc.ccnt, sr, "ccnt");
    if (!rc) rc = dev_alloc(&b->sc.crej, sr, "crej");
    if (!rc) rc = dev_alloc(&b->sc.cflag, sr, "cflag");
    if (!rc) rc = dev_alloc(&b->sc.psum, sr, "psum");
    if (!rc) rc = dev_alloc(&b->sc.pcnt, sr, "pcnt");
    const size_t np_rows = (size_t)np * R;          // parts of the streaming kernel
    if (!rc) rc = dev_alloc(&b->sc.wrec, np_rows * QS_PART_WAVES, "part records");
    if (!rc) rc = dev_alloc(&b->sc.pcand, np_rows * QS_PART_CANDS, "part candidates");
    if (!rc) rc = dev_alloc(&b->sc.locks, b->sc.nslots, "locks");
    if (!rc) rc = dev_alloc(&b->sc.full_keys, (size_t)b->sc.nslots * 2 * V, "full_keys");
    if (!rc) rc = dev_alloc(&b->sc.full_bm, (size_t)b->sc.nslots * (V / 32 + 1), "full_bm");
    if (!rc) rc = dev_alloc(&b->sc.err, 1, "err");
    if (!rc) rc = dev_alloc(&b->sc.gbest, R, "greedy bests");
    if (!rc) rc = dev_alloc(&b->sc.gmaxk, R, "greedy maxima");
    if (!rc) rc = dev_alloc(&b->sc.gcnt, R, "greedy part counts");
    if (!rc && hipMemset(b->sc.locks, 0, sizeof(int32_t) * b->sc.nslots) != hipSuccess) rc = QS_EDEVICE;
    if (!rc && hipMemset(b->sc.err, 0, sizeof(int32_t)) != hipSuccess) rc = QS_EDEVICE;
    if (!rc && hipMemset(b->sc.gbest, 0, sizeof(uint64_t) * R) != hipSuccess) rc = QS_EDEVICE;
    if (!rc && hipMemset(b->sc.gmaxk, 0, sizeof(uint32_t) * R) != hipSuccess) rc = QS_EDEVICE;
    if (!rc && hipMemset(b->sc.gcnt, 0, sizeof(uint32_t) * R) != hipSuccess) rc = QS_EDEVICE;
    return rc;
}

static int upload_rows(qs_batch *b, int row0, int n_rows) {
    HIP_TRY(hipStreamSynchronize(b->stream), "sync");
    HIP_TRY(hipMemcpy(b->d_prm + row0, b->h_prm.data() + row0, sizeof(qs_row_param) * n_rows,
                      hipMemcpyHostToDevice),
            "upload params");
    return 0;
}

static bool rows_ok(const qs_batch *b, int row0, int n_rows) {
    if (!b || row0 < 0 || n_rows < 1 || row0 + n_rows > b->max_rows) {
        qs_set_error("rows [%d, %d) outside the batch", row0, row0 + n_rows);
        return false;
    }
    return true;
}

// The kernels a pick with these arguments takes: the batch's mode, or for AUTO the row
// kernel when the batch has a row for at least a quarter of the CUs and every sampling row
// aims at most QS_ROW_AUTO_KSEL candidates (its per-wavefront candidate lists hold a few
// hundred entries; a row that overflows them takes the full-window path), the streaming
// kernels when the rows allow them, the split-row kernels otherwise.  `kmax` is the largest
// candidate target among the sampling rows (1 when every row is greedy).  The quarter: on
// MI355X (256 CUs) at 151,936 logits a row, a pick of the row kernel takes about 23 us
// from 8 to 64 rows (one workgroup per row, each row's latency), the streaming pair 17 us at
// 8 rows rising to 22 at 48 and 28 at 64.
static int auto_mode(const qs_batch *b, const float *d_logits, int64_t row_stride, int n_rows,
                     int n_vocab, int kmax) {
    if (b->mode != QS_MODE_AUTO) return b->mode;
    if (4 * (int64_t)n_rows >= b->n_cu && kmax <= QS_ROW_AUTO_KSEL &&
        qs_row_supported(n_rows, n_vocab, row_stride, d_logits))
        return QS_MODE_ROW;
    return qs_part_supported(n_rows, n_vocab, row_stride, d_logits) ? QS_MODE_STREAM
                                                                    : QS_MODE_SPLIT;
}

// Wavefronts per row of the row kernel: 16 (one workgroup per CU) up to a row per CU, 8
// (two per CU, one deciding while the other streams) beyond, when two fit (at 300 rows of
// 151,936 logits: 48.4 us a pick against 51.5 with a second round of 16-wavefront rows).
static int row_waves(const qs_batch *b, int n_rows) {
    return n_rows <= b->n_cu || !b->row8 ? 16 : 8;
}

extern "C" {

qs_batch *qs_batch_new(int max_rows, int max_vocab, int max_last_n) {
    if (max_rows < 1 || max_vocab < 1 || max_last_n < 0) {
        qs_set_error("qs_batch_new: bad sizes (%d, %d, %d)", max_rows, max_vocab, max_last_n);
        return nullptr;
    }
    qs_batch *b = new (std::nothrow) qs_batch();
    if (!b) return nullptr;
    b->max_rows = max_rows;
    b->max_vocab = max_vocab;
    b->max_last_n = max_last_n;
    hipError_t e = hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking);
    if (e != hipSuccess) { hip_fail(e, "stream"); b->stream = nullptr; batch_release(b); return nullptr; }
    if (hipEventCreate(&b->ev0) != hipSuccess || hipEventCreate(&b->ev1) != hipSuccess) {
        qs_set_error("qs_batch_new: event creation failed");
        batch_release(b);
        return nullptr;
    }
    if (batch_alloc(b) != 0) { batch_release(b); return nullptr; }
    b->h_prm.resize(max_rows);
    std::vector<uint64_t> rng(max_rows);
    for (int r = 0; r < max_rows; ++r) qs_default_param(&b->h_prm[r], &rng[r]);
    std::vector<int32_t> zero(max_rows, 0);
    if (hipMemcpy(b->d_prm, b->h_prm.data(), sizeof(qs_row_param) * max_rows, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(b->d_rng, rng.data(), sizeof(uint64_t) * max_rows, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(b->d_hlen, zero.data(), sizeof(int32_t) * max_rows, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(b->d_hhead, zero.data(), sizeof(int32_t) * max_rows, hipMemcpyHostToDevice) != hipSuccess) {
        qs_set_error("qs_batch_new: initial upload failed");
        batch_release(b);
        return nullptr;
    }
    return b;
}

void qs_batch_free(qs_batch *b) { batch_release(b); }

int qs_batch_config(qs_batch *b, int row0, int n_rows, float temperature, float top_p,
                    int top_k, float min_p, float repeat_penalty, int repeat_last_n,
                    const uint64_t *seeds) {
    if (!rows_ok(b, row0, n_rows)) return QS_EINVAL;
    if (repeat_last_n > b->max_last_n) {
        qs_set_error("repeat_last_n %d exceeds the batch's ring capacity %d", repeat_last_n,
                     b->max_last_n);
        return QS_EINVAL;
    }
    std::vector<uint64_t> rng(n_rows);
    for (int r = 0; r < n_rows; ++r) {
        qs_row_param &p = b->h_prm[row0 + r];
        qs_clamp_config(temperature, top_p, top_k, min_p, repeat_penalty, repeat_last_n,
                        seeds ? seeds[r] : 0ull, p.ring_cap, &p, &rng[r]);
    }
    int rc = upload_rows(b, row0, n_rows);
    if (rc) return rc;
    std::vector<int32_t> zero(n_rows, 0);
    HIP_TRY(hipMemcpy(b->d_rng + row0, rng.data(), sizeof(uint64_t) * n_rows, hipMemcpyHostToDevice), "rng");
    HIP_TRY(hipMemcpy(b->d_hlen + row0, zero.data(), sizeof(int32_t) * n_rows, hipMemcpyHostToDevice), "hlen");
    HIP_TRY(hipMemcpy(b->d_hhead + row0, zero.data(), sizeof(int32_t) * n_rows, hipMemcpyHostToDevice), "hhead");
    return 0;
}

int qs_batch_reset(qs_batch *b, int row0, int n_rows) {
    if (!rows_ok(b, row0, n_rows)) return QS_EINVAL;
    HIP_TRY(hipStreamSynchronize(b->stream), "sync");
    std::vector<int32_t> zero(n_rows, 0);
    HIP_TRY(hipMemcpy(b->d_hlen + row0, zero.data(), sizeof(int32_t) * n_rows, hipMemcpyHostToDevice), "hlen");
    HIP_TRY(hipMemcpy(b->d_hhead + row0, zero.data(), sizeof(int32_t) * n_rows, hipMemcpyHostToDevice), "hhead");
    return 0;
}

// Lay out `n` ids into a ring of capacity cap exactly as n successive records would.
static void ring_fill(const int32_t *ids, int n, int cap, int32_t *ring, int32_t *len,
                      int32_t *head) {
    *len = 0;
    *head = 0;
    if (cap <= 0) return;
    for (int i = 0; i < n; ++i) {
        if (*len < cap) {
            ring[(*head + *len) % cap] = ids[i];
            ++*len;
        } else {
            ring[*head] = ids[i];
            *head = (*head + 1) % cap;
        }
    }
}

int qs_batch_set_history(qs_batch *b, int row0, int n_rows, const int32_t *ids,
                         int n_per_row) {
    if (!rows_ok(b, row0, n_rows)) return QS_EINVAL;
    if (n_per_row < 0 || (n_per_row > 0 && !ids)) {
        qs_set_error("qs_batch_set_history: bad ids");
        return QS_EINVAL;
    }
    const int L = b->max_last_n > 0 ? b->max_last_n : 1;
    std::vector<int32_t> ring((size_t)n_rows * L, 0), len(n_rows), head(n_rows);
    for (int r = 0; r < n_rows; ++r)
        ring_fill(ids + (size_t)r * n_per_row, n_per_row, b->h_prm[row0 + r].ring_cap,
                  ring.data() + (size_t)r * L, &len[r], &head[r]);
    HIP_TRY(hipStreamSynchronize(b->stream), "sync");
    HIP_TRY(hipMemcpy(b->d_ring + (size_t)row0 * L, ring.data(), sizeof(int32_t) * ring.size(), hipMemcpyHostToDevice), "ring");
    HIP_TRY(hipMemcpy(b->d_hlen + row0, len.data(), sizeof(int32_t) * n_rows, hipMemcpyHostToDevice), "hlen");
    HIP_TRY(hipMemcpy(b->d_hhead + row0, head.data(), sizeof(int32_t) * n_rows, hipMemcpyHostToDevice), "hhead");
    return 0;
}

int qs_batch_set_state(qs_batch *b, int row, uint64_t rng, const int32_t *hist, int n) {
    if (!rows_ok(b, row, 1)) return QS_EINVAL;
    int rc = qs_batch_set_history(b, row, 1, hist, n);
    if (rc) return rc;
    HIP_TRY(hipMemcpy(b->d_rng + row, &rng, sizeof rng, hipMemcpyHostToDevice), "rng");
    return 0;
}

int qs_batch_get_state(qs_batch *b, int row, uint64_t *rng, int32_t *hist, int cap,
                       int *hist_len) {
    if (!rows_ok(b, row, 1)) return QS_EINVAL;
    HIP_TRY(hipStreamSynchronize(b->stream), "sync");
    const int L = b->max_last_n > 0 ? b->max_last_n : 1;
    std::vector<int32_t> ring(L);
    int32_t len = 0, head = 0;
    uint64_t r = 0;
    HIP_TRY(hipMemcpy(&r, b->d_rng + row, sizeof r, hipMemcpyDeviceToHost), "rng");
    HIP_TRY(hipMemcpy(&len, b->d_hlen + row, sizeof len, hipMemcpyDeviceToHost), "hlen");
    HIP_TRY(hipMemcpy(&head, b->d_hhead + row, sizeof head, hipMemcpyDeviceToHost), "hhead");
    HIP_TRY(hipMemcpy(ring.data(), b->d_ring + (size_t)row * L, sizeof(int32_t) * L, hipMemcpyDeviceToHost), "ring");
    if (rng) *rng = r;
    if (hist_len) *hist_len = len;
    const int ringcap = b->h_prm[row].ring_cap;
    if (hist)
        for (int i = 0; i < len && i < cap; ++i) hist[i] = ring[(head + i) % ringcap];
    return 0;
}

// The largest top-k among the sampling rows of [row0, row0 + n_rows) and whether any row
// samples; QS_EINVAL when a row's ring is larger than the batch holds.
static int batch_kmax(const qs_batch *b, int n_rows, int *kmax, bool *any_sample,
                      int row0 = 0) {
    *kmax = 1;
    *any_sample = false;
    for (int r = row0; r < row0 + n_rows; ++r) {
        const qs_row_param &p = b->h_prm[r];
        if (row_greedy(p)) continue;
        *any_sample = true;
        const int k = row_ksel(p);
        if (k > *kmax) *kmax = k;
        if (p.ring_cap > b->max_last_n) { qs_set_error("ring capacity"); return QS_EINVAL; }
    }
    return 0;
}

int qs_batch_resolve_mode(qs_batch *b, const float *d_logits, int64_t row_stride, int n_rows,
                          int n_vocab) {
    if (!b || n_rows < 1 || n_rows > b->max_rows || n_vocab < 1 || n_vocab > b->max_vocab ||
        row_stride < n_vocab) {
        qs_set_error("qs_batch_resolve_mode: bad arguments");
        return QS_EINVAL;
    }
    int kmax = 1;
    bool any_sample = false;
    if (const int rc = batch_kmax(b, n_rows, &kmax, &any_sample)) return rc;
    return auto_mode(b, d_logits, row_stride, n_rows, n_vocab, kmax);
}

// The pick of the batch's rows [row0, row0 + n_rows) from logits rows 0 .. n_rows - 1: the
// kernels see the rows' state from row0 on (parameters, generators, rings, lengths and
// heads are arrays over the batch's rows), their scratch from its start.
static int pick_range(qs_batch *b, int row0, const float *d_logits, int64_t row_stride,
                      int n_rows, int n_vocab, int32_t *d_out, qs_pick_diag *d_diag) {
    if (!b || !d_logits || !d_out) { qs_set_error("qs_batch_pick: null argument"); return QS_EINVAL; }
    if (row0 < 0 || n_rows < 1 || n_rows > b->max_rows - row0 || n_vocab < 1 ||
        n_vocab > b->max_vocab || row_stride < n_vocab) {
        qs_set_error("qs_batch_pick: rows [%d, %d) (max %d), vocab %d (max %d), stride %lld",
                     row0, row0 + n_rows, b->max_rows, n_vocab, b->max_vocab,
                     (long long)row_stride);
        return QS_EINVAL;
    }
    int kmax = 1;
    bool any_sample = false;
    if (const int rc = batch_kmax(b, n_rows, &kmax, &any_sample, row0)) return rc;
    const int rs = b->max_last_n > 0 ? b->max_last_n : 1;
    RowState st0{b->d_prm + row0, b->d_rng + row0, b->d_ring + (int64_t)row0 * rs,
                 b->d_hlen + row0, b->d_hhead + row0, rs};
    const int mode = auto_mode(b, d_logits, row_stride, n_rows, n_vocab, kmax);
    if (mode == QS_MODE_ROW) {
        if (!qs_row_supported(n_rows, n_vocab, row_stride, d_logits)) {
            qs_set_error("qs_batch_pick: the row kernel does not support this pick");
            return QS_EINVAL;
        }
        return qs_row_launch(d_logits, row_stride, n_rows, n_vocab, st0, b->sc, d_out, d_diag,
                             row_waves(b, n_rows), b->stream);
    }
    if (mode == QS_MODE_STREAM) {
        if (!qs_part_supported(n_rows, n_vocab, row_stride, d_logits)) {
            qs_set_error("qs_batch_pick: the streaming kernel does not support this pick");
            return QS_EINVAL;
        }
        return qs_part_launch(d_logits, row_stride, n_rows, n_vocab, st0, b->sc, d_out, d_diag,
                              b->part_resident, b->stream, b->mid, !any_sample);
    }
    Geometry g;
    g.logits = d_logits;
    g.stride = row_stride;
    g.vocab = n_vocab;
    g.n_rows = n_rows;
    g.slices = slices_for(n_rows, n_vocab, kmax, &g.slice_len);
    if (g.slices * n_rows > b->slice_rows) {
        qs_set_error("qs_batch_pick: slice scratch too small");
        return QS_EDEVICE;
    }
    g.bm_words = g.slice_len / 32;
    const RowState st = st0;
    const bool vec = ((uintptr_t)d_logits % 16 == 0) && (row_stride % 4 == 0) &&
                     (n_vocab % 4 == 0);
    const dim3 grid(g.slices, n_rows);
    const size_t lds_scan = sizeof(uint32_t) * (size_t)g.bm_words;
    const size_t lds_exp = sizeof(uint32_t) * ((size_t)g.bm_words + 2 * (size_t)CCAP);
    if (vec) {
        hipLaunchKernelGGL(k_scan<true>, grid, dim3(WG), lds_scan, b->stream, g, st, b->sc);
    } else {
        hipLaunchKernelGGL(k_scan<false>, grid, dim3(WG), lds_scan, b->stream, g, st, b->sc);
    }
    HIP_TRY(hipGetLastError(), "k_scan launch");
    if (any_sample) {
        if (vec) {
            hipLaunchKernelGGL(k_expsum<true>, grid, dim3(WG), lds_exp, b->stream, g, st, b->sc);
        } else {
            hipLaunchKernelGGL(k_expsum<false>, grid, dim3(WG), lds_exp, b->stream, g, st, b->sc);
        }
        HIP_TRY(hipGetLastError(), "k_expsum launch");
    }
    FinArgs fa{g, st, b->sc, d_out, d_diag};
    hipLaunchKernelGGL(k_finalize, dim3(n_rows), dim3(WG), 0, b->stream, fa);
    HIP_TRY(hipGetLastError(), "k_finalize launch");
    return 0;
}

int qs_batch_pick(qs_batch *b, const float *d_logits, int64_t row_stride, int n_rows,
                  int n_vocab, int32_t *d_out, qs_pick_diag *d_diag) {
    return pick_range(b, 0, d_logits, row_stride, n_rows, n_vocab, d_out, d_diag);
}

int qs_batch_pick_rows(qs_batch *b, int row0, const float *d_logits, int64_t row_stride,
                       int n_rows, int n_vocab, int32_t *d_out, qs_pick_diag *d_diag) {
    return pick_range(b, row0, d_logits, row_stride, n_rows, n_vocab, d_out, d_diag);
}

int qs_batch_set_mode(qs_batch *b, int mode) {
    if (!b || mode < QS_MODE_AUTO || mode > QS_MODE_ROW) {
        qs_set_error("qs_batch_set_mode: bad mode %d", mode);
        return QS_EINVAL;
    }
    b->mode = mode;
    return 0;
}

int qs_batch_synchronize(qs_batch *b) {
    if (!b) return QS_EINVAL;
    HIP_TRY(hipStreamSynchronize(b->stream), "qs_batch_synchronize");
    int32_t err = 0;
    HIP_TRY(hipMemcpy(&err, b->sc.err, sizeof err, hipMemcpyDeviceToHost), "error flag");
    if (err) {
        const int32_t zero = 0;
        (void)hipMemcpy(b->sc.err, &zero, sizeof zero, hipMemcpyHostToDevice);
        qs_set_error("a whole-window scratch slot was not free in time (flags %d): the rows "
                     "involved returned -3 and kept their generator state and history; "
                     "pick them again", err);
        return QS_EAGAIN;
    }
    return 0;
}

int qs_batch_pick1_host(qs_batch *b, float *d_logits, const float *logits, int n_vocab,
                        int32_t *d_out, int32_t *id) {
    if (!b || !d_logits || !logits || !d_out || !id) return QS_EINVAL;
    if (!b->h_pin) {
        HIP_TRY(hipHostMalloc((void **)&b->h_pin, 2 * sizeof(int32_t), hipHostMallocDefault),
                "pinned id buffer");
        if (hipHostGetDevicePointer((void **)&b->d_pin, b->h_pin, 0) != hipSuccess) {
            (void)hipHostFree(b->h_pin);
            b->h_pin = nullptr;
            b->d_pin = nullptr;
            qs_set_error("pinned id buffer: no device address");
            return QS_EDEVICE;
        }
    }
    HIP_TRY(hipMemcpyAsync(d_logits, logits, sizeof(float) * (size_t)n_vocab,
                           hipMemcpyHostToDevice, b->stream), "logits to the device");
    if (const int rc = qs_batch_pick(b, d_logits, n_vocab, 1, n_vocab, d_out, nullptr)) return rc;
    hipLaunchKernelGGL(k_result1, dim3(1), dim3(64), 0, b->stream, d_out, b->sc.err, b->d_pin);
    HIP_TRY(hipGetLastError(), "k_result1 launch");
    HIP_TRY(hipStreamSynchronize(b->stream), "one-row pick");
    if (b->h_pin[1]) {
        const int32_t zero = 0;
        (void)hipMemcpy(b->sc.err, &zero, sizeof zero, hipMemcpyHostToDevice);
        qs_set_error("a whole-window scratch slot was not free in time (flags %d): the row "
                     "returned -3 and kept its generator state and history; pick it again",
                     b->h_pin[1]);
        return QS_EAGAIN;
    }
    *id = b->h_pin[0];
    return 0;
}

void *qs_batch_stream(qs_batch *b) { return b ? (void *)b->stream : nullptr; }

int qs_batch_set_sum_in_order(qs_batch *b, int always) {
    if (!b || always < 0 || always > 1) {
        qs_set_error("qs_batch_set_sum_in_order: bad arguments");
        return QS_EINVAL;
    }
    b->sc.sum_in_order = always;
    return 0;
}

int qs_batch_set_spin_limit(qs_batch *b, int attempts) {
    if (!b || attempts < 0) {
        qs_set_error("qs_batch_set_spin_limit: bad arguments");
        return QS_EINVAL;
    }
    b->sc.spin_limit = attempts;
    return 0;
}

// The output layer's arguments, checked; allocates its records and history bitmap on the
// first call (zeroed once: each pick leaves the bitmap zero).
static int head_records(qs_batch *b, int n_rows);

static int head_check(qs_batch *b, const void *d_hidden, const void *d_weight, int n_embd,
                      int n_rows, int n_vocab, const float *d_logits, bool pick) {
    if (!b || !d_hidden || !d_weight || !d_logits) {
        qs_set_error("output layer: null argument");
        return QS_EINVAL;
    }
    const int rmax = b->max_rows < QS_HEAD_MAX_ROWS ? b->max_rows : QS_HEAD_MAX_ROWS;
    const int vmax = b->max_vocab < QS_HEAD_MAX_VOCAB ? b->max_vocab : QS_HEAD_MAX_VOCAB;
    if (n_rows < 1 || n_rows > rmax || n_vocab < 4 || n_vocab > vmax || n_vocab % 4 != 0 ||
        n_embd < 64 || n_embd % 64 != 0 || (uintptr_t)d_hidden % 16 != 0 ||
        (uintptr_t)d_weight % 16 != 0 || (uintptr_t)d_logits % 16 != 0) {
        qs_set_error("output layer: rows %d (1..%d), vocab %d (a multiple of 4 up to %d), "
                     "embedding %d (a multiple of 64), 16-byte aligned buffers", n_rows, rmax,
                     n_vocab, vmax, n_embd);
        return QS_EINVAL;
    }
    if (!pick) return 0;
    return head_records(b, n_rows);
}

// A fused pick's tile records and history bitmap: allocated on the first such pick (for
// min(max_rows, 256) rows and the batch's vocabulary; the bitmap zeroed once, each pick
// leaving it zero) or cleared after a failed one; then the rows' parameters checked.
static int head_records(qs_batch *b, int n_rows) {
    const int rmax = b->max_rows < QS_HEAD_MAX_ROWS ? b->max_rows : QS_HEAD_MAX_ROWS;
    if (!b->d_hrec) {
        const size_t nt = (size_t)(b->max_vocab + QS_HEAD_TILE - 1) / QS_HEAD_TILE;
        int rc = dev_alloc(&b->d_hrec, (size_t)rmax * nt, "output layer records");
        if (!rc) rc = dev_alloc(&b->d_hbits, (size_t)(QS_HEAD_MAX_ROWS / 32) * b->max_vocab,
                                "output layer history bits");
        if (!rc && hipMemset(b->d_hbits, 0, sizeof(uint32_t) * (QS_HEAD_MAX_ROWS / 32) *
                                                (size_t)b->max_vocab) != hipSuccess) {
            qs_set_error("output layer: clearing the history bits failed");
            rc = QS_EDEVICE;
        }
        if (rc) {
            if (b->d_hrec) (void)hipFree(b->d_hrec);
            if (b->d_hbits) (void)hipFree(b->d_hbits);
            b->d_hrec = nullptr;
            b->d_hbits = nullptr;
            return rc;
        }
    }
    if (b->hbits_dirty) {
        // the bitmap kernel of a failed fused pick may have left bits that only the output
        // layer's kernel clears
        HIP_TRY(hipStreamSynchronize(b->stream), "sync");
        HIP_TRY(hipMemset(b->d_hbits, 0, sizeof(uint32_t) * (QS_HEAD_MAX_ROWS / 32) *
                                             (size_t)b->max_vocab), "clearing the history bits");
        b->hbits_dirty = false;
    }
    int kmax = 1;
    bool any = false;
    return batch_kmax(b, n_rows, &kmax, &any);
}

int qs_batch_head_logits(qs_batch *b, const void *d_hidden, const void *d_weight, int n_embd,
                         int n_rows, int n_vocab, float *d_logits) {
    if (const int rc = head_check(b, d_hidden, d_weight, n_embd, n_rows, n_vocab, d_logits,
                                  false))
        return rc;
    RowState st{b->d_prm, b->d_rng, b->d_ring, b->d_hlen, b->d_hhead,
                b->max_last_n > 0 ? b->max_last_n : 1};
    return qs_head_launch(d_hidden, d_weight, n_embd, n_rows, n_vocab, d_logits, st, b->sc,
                          nullptr, nullptr, nullptr, nullptr, b->stream);
}

int qs_batch_pick_head(qs_batch *b, const void *d_hidden, const void *d_weight, int n_embd,
                       int n_rows, int n_vocab, float *d_logits, int32_t *d_out,
                       qs_pick_diag *d_diag) {
    if (!d_out) { qs_set_error("qs_batch_pick_head: null output"); return QS_EINVAL; }
    if (const int rc = head_check(b, d_hidden, d_weight, n_embd, n_rows, n_vocab, d_logits,
                                  true))
        return rc;
    RowState st{b->d_prm, b->d_rng, b->d_ring, b->d_hlen, b->d_hhead,
                b->max_last_n > 0 ? b->max_last_n : 1};
    const int rc = qs_head_launch(d_hidden, d_weight, n_embd, n_rows, n_vocab, d_logits, st,
                                  b->sc, b->d_hrec, b->d_hbits, d_out, d_diag, b->stream);
    if (rc) b->hbits_dirty = true;
    return rc;
}

size_t qs_head_packed_bytes(int n_embd, int n_vocab) {
    if (n_embd < 64 || n_embd % 64 != 0 || n_vocab < 4 || n_vocab > QS_HEAD_MAX_VOCAB ||
        n_vocab % 4 != 0)
        return 0;
    return 2 * qs_head_packed_elems(n_embd, n_vocab);
}

int qs_batch_head_pack(qs_batch *b, const void *d_weight, int n_embd, int n_vocab,
                       void *d_packed) {
    if (!b || !d_weight || !d_packed || !qs_head_packed_bytes(n_embd, n_vocab) ||
        (uintptr_t)d_weight % 16 != 0 || (uintptr_t)d_packed % 16 != 0) {
        qs_set_error("qs_batch_head_pack: vocab %d (a multiple of 4 up to %d), embedding %d "
                     "(a multiple of 64), non-null 16-byte aligned buffers", n_vocab,
                     QS_HEAD_MAX_VOCAB, n_embd);
        return QS_EINVAL;
    }
    return qs_head_pack_launch(d_weight, n_embd, n_vocab, d_packed, b->stream);
}

int qs_batch_time_head(qs_batch *b, const void *d_hidden, const void *d_weight, int n_embd,
                       int n_rows, int n_vocab, float *d_logits, int32_t *d_out, int iters,
                       int fused, float *ms) {
    if (!b || iters < 1 || !ms || fused < 0 || fused > 2) return QS_EINVAL;
    HIP_TRY(hipEventRecord(b->ev0, b->stream), "event");
    for (int i = 0; i < iters; ++i) {
        int rc;
        if (fused == 1) {
            rc = qs_batch_pick_head(b, d_hidden, d_weight, n_embd, n_rows, n_vocab, d_logits,
                                    d_out, nullptr);
        } else if (fused == 2) {
            rc = qs_batch_head_logits(b, d_hidden, d_weight, n_embd, n_rows, n_vocab, d_logits);
        } else {
            rc = qs_batch_head_logits(b, d_hidden, d_weight, n_embd, n_rows, n_vocab, d_logits);
            if (!rc) rc = qs_batch_pick(b, d_logits, n_vocab, n_rows, n_vocab, d_out, nullptr);
        }
        if (rc) return rc;
    }
    HIP_TRY(hipEventRecord(b->ev1, b->stream), "event");
    HIP_TRY(hipEventSynchronize(b->ev1), "event sync");
    HIP_TRY(hipEventElapsedTime(ms, b->ev0, b->ev1), "elapsed");
    return 0;
}

// The exact output layer's arguments, checked (with `pick`, its records as head_check).
static int head_exact_check(qs_batch *b, int wtype, const void *d_packed, const float *d_xn,
                            int n_embd, int n_rows, int n_vocab, const float *d_logits,
                            bool pick) {
    if (!b || !d_packed || !d_xn || !d_logits) {
        qs_set_error("exact output layer: null argument");
        return QS_EINVAL;
    }
    const int rmax = b->max_rows < QS_HEAD_EXACT_MAX_ROWS ? b->max_rows : QS_HEAD_EXACT_MAX_ROWS;
    const int vmax = b->max_vocab < QS_HEAD_MAX_VOCAB ? b->max_vocab : QS_HEAD_MAX_VOCAB;
    if (!qs_head_exact_shape_ok(wtype, n_embd) || n_rows < 1 || n_rows > rmax ||
        (int64_t)n_rows * n_embd > QS_HEAD_EXACT_MAX_EMBD || n_vocab < 4 || n_vocab > vmax ||
        n_vocab % 4 != 0 || (uintptr_t)d_packed % 16 != 0 || (uintptr_t)d_xn % 16 != 0 ||
        (uintptr_t)d_logits % 16 != 0) {
        qs_set_error("exact output layer: type %d with embedding %d (F32/F16: a multiple of 16, "
                     "Q8_0: 32, Q6_K: 256), rows %d (1..%d, rows x embedding at most %d), "
                     "vocab %d (a multiple of 4 up to %d), 16-byte aligned buffers", wtype,
                     n_embd, n_rows, rmax, QS_HEAD_EXACT_MAX_EMBD, n_vocab, vmax);
        return QS_EINVAL;
    }
    return pick ? head_records(b, n_rows) : 0;
}

size_t qs_head_exact_packed_bytes(int wtype, int n_embd, int n_vocab) {
    if (n_vocab > QS_HEAD_MAX_VOCAB) return 0;
    return qs_head_exact_bytes(wtype, n_embd, n_vocab);
}

int qs_batch_head_exact_pack(qs_batch *b, int wtype, const void *d_weight, int n_embd,
                             int n_vocab, void *d_packed) {
    if (!b || !d_weight || !d_packed || !qs_head_exact_packed_bytes(wtype, n_embd, n_vocab) ||
        (uintptr_t)d_packed % 16 != 0) {
        qs_set_error("qs_batch_head_exact_pack: type %d, embedding %d, vocab %d (up to %d), "
                     "non-null buffers, the packed one 16-byte aligned", wtype, n_embd, n_vocab,
                     QS_HEAD_MAX_VOCAB);
        return QS_EINVAL;
    }
    return qs_head_exact_pack_launch(d_weight, wtype, n_embd, n_vocab, d_packed, b->stream);
}

int qs_batch_head_exact_logits(qs_batch *b, int wtype, const void *d_packed,
                               const float *d_xn, int n_embd, int n_rows, int n_vocab,
                               float *d_logits) {
    if (const int rc = head_exact_check(b, wtype, d_packed, d_xn, n_embd, n_rows, n_vocab,
                                        d_logits, false))
        return rc;
    RowState st{b->d_prm, b->d_rng, b->d_ring, b->d_hlen, b->d_hhead,
                b->max_last_n > 0 ? b->max_last_n : 1};
    return qs_head_exact_launch(d_packed, wtype, d_xn, n_embd, n_rows, n_vocab, d_logits, st,
                                nullptr, b->stream);
}

int qs_batch_pick_head_exact(qs_batch *b, int wtype, const void *d_packed, const float *d_xn,
                             int n_embd, int n_rows, int n_vocab, float *d_logits,
                             int32_t *d_out, qs_pick_diag *d_diag) {
    if (!d_out) { qs_set_error("qs_batch_pick_head_exact: null output"); return QS_EINVAL; }
    if (const int rc = head_exact_check(b, wtype, d_packed, d_xn, n_embd, n_rows, n_vocab,
                                        d_logits, true))
        return rc;
    RowState st{b->d_prm, b->d_rng, b->d_ring, b->d_hlen, b->d_hhead,
                b->max_last_n > 0 ? b->max_last_n : 1};
    const int rc = qs_head_exact_launch(d_packed, wtype, d_xn, n_embd, n_rows, n_vocab,
                                        d_logits, st, b->d_hrec, b->stream);
    if (rc) return rc;
    return qs_head_decide_launch(d_logits, n_rows, n_vocab, st, b->sc, b->d_hrec, d_out, d_diag,
                                 b->stream);
}

int qs_batch_time_head_exact(qs_batch *b, int wtype, const void *d_packed, const float *d_xn,
                             int n_embd, int n_rows, int n_vocab, float *d_logits,
                             int32_t *d_out, int iters, int fused, float *ms) {
    if (!b || iters < 1 || !ms || fused < 0 || fused > 2) return QS_EINVAL;
    HIP_TRY(hipEventRecord(b->ev0, b->stream), "event");
    for (int i = 0; i < iters; ++i) {
        int rc;
        if (fused == 1) {
            rc = qs_batch_pick_head_exact(b, wtype, d_packed, d_xn, n_embd, n_rows, n_vocab,
                                          d_logits, d_out, nullptr);
        } else {
            rc = qs_batch_head_exact_logits(b, wtype, d_packed, d_xn, n_embd, n_rows, n_vocab,
                                            d_logits);
            if (!rc && fused == 0)
                rc = qs_batch_pick(b, d_logits, n_vocab, n_rows, n_vocab, d_out, nullptr);
        }
        if (rc) return rc;
    }
    HIP_TRY(hipEventRecord(b->ev1, b->stream), "event");
    HIP_TRY(hipEventSynchronize(b->ev1), "event sync");
    HIP_TRY(hipEventElapsedTime(ms, b->ev0, b->ev1), "elapsed");
    return 0;
}

int qs_batch_time_picks(qs_batch *b, const float *const *d_logits, int n_buffers,
                        int64_t row_stride, int n_rows, int n_vocab, int32_t *d_out, int iters,
                        float *ms) {
    if (!b || !d_logits || n_buffers < 1 || iters < 1 || !ms) return QS_EINVAL;
    HIP_TRY(hipEventRecord(b->ev0, b->stream), "event");
    for (int i = 0; i < iters; ++i) {
        const int rc = qs_batch_pick(b, d_logits[i % n_buffers], row_stride, n_rows, n_vocab,
                                     d_out, nullptr);
        if (rc) return rc;
    }
    HIP_TRY(hipEventRecord(b->ev1, b->stream), "event");
    HIP_TRY(hipEventSynchronize(b->ev1), "event sync");
    HIP_TRY(hipEventElapsedTime(ms, b->ev0, b->ev1), "elapsed");
    return 0;
}

int qs_batch_time_kernels(qs_batch *b, const float *const *d_logits, int n_buffers,
                          int64_t row_stride, int n_rows, int n_vocab, int32_t *d_out,
                          int iters, float *ms_stream) {
    if (!b || !d_logits || n_buffers < 1 || iters < 1 || !ms_stream) return QS_EINVAL;
    const int mode = qs_batch_resolve_mode(b, d_logits[0], row_stride, n_rows, n_vocab);
    if (mode != QS_MODE_STREAM && mode != QS_MODE_ROW) {
        qs_set_error("qs_batch_time_kernels: the pick takes neither the streaming nor the row "
                     "kernel");
        return mode < 0 ? mode : QS_EINVAL;
    }
    std::vector<hipEvent_t> ev(2 * (size_t)iters, nullptr);
    int rc = 0;
    for (auto &e : ev)
        if (!rc && hipEventCreate(&e) != hipSuccess) rc = QS_EDEVICE;
    for (int i = 0; i < iters && !rc; ++i) {
        if (hipEventRecord(ev[2 * i], b->stream) != hipSuccess) { rc = QS_EDEVICE; break; }
        b->mid = ev[2 * i + 1];
        rc = qs_batch_pick(b, d_logits[i % n_buffers], row_stride, n_rows, n_vocab, d_out,
                           nullptr);
        b->mid = nullptr;
        // the row kernel is the whole pick: its end is the pick's
        if (!rc && mode == QS_MODE_ROW && hipEventRecord(ev[2 * i + 1], b->stream) != hipSuccess)
            rc = QS_EDEVICE;
    }
    if (!rc && hipStreamSynchronize(b->stream) != hipSuccess) rc = QS_EDEVICE;
    double total = 0.0;
    for (int i = 0; i < iters && !rc; ++i) {
        float t = 0.0f;
        if (hipEventElapsedTime(&t, ev[2 * i], ev[2 * i + 1]) != hipSuccess) rc = QS_EDEVICE;
        total += t;
    }
    for (auto &e : ev)
        if (e) (void)hipEventDestroy(e);
    if (rc) {
        if (rc == QS_EDEVICE) qs_set_error("qs_batch_time_kernels: event failure");
        return rc;
    }
    *ms_stream = (float)total;
    return 0;
}

int qs_row_workgroups_per_cu(int waves) {
    if (waves != 16 && waves != 8) {
        qs_set_error("qs_row_workgroups_per_cu: waves %d (16 or 8)", waves);
        return QS_EINVAL;
    }
    return qs_row_resident(waves);
}

void *qs_device_alloc(size_t bytes) {
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) { hip_fail(e, "qs_device_alloc"); return nullptr; }
    return p;
}

void qs_device_free(void *p) {
    if (p) (void)hipFree(p);
}

int qs_memcpy_h2d(void *d_dst, const void *src, size_t bytes) {
    HIP_TRY(hipMemcpy(d_dst, src, bytes, hipMemcpyHostToDevice), "qs_memcpy_h2d");
    return 0;
}

int qs_memcpy_d2h(void *dst, const void *d_src, size_t bytes) {
    HIP_TRY(hipMemcpy(dst, d_src, bytes, hipMemcpyDeviceToHost), "qs_memcpy_d2h");
    return 0;
}

int qs_device_synchronize(void) {
    HIP_TRY(hipDeviceSynchronize(), "qs_device_synchronize");
    return 0;
}

int qs_device_info(char *name, int name_cap, size_t *total_mem, int *n_cu) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
    hipDeviceProp_t pr;
    HIP_TRY(hipGetDeviceProperties(&pr, dev), "hipGetDeviceProperties");
    if (name && name_cap > 0) {
        snprintf(name, (size_t)name_cap, "%s (%s)", pr.name, pr.gcnArchName);
    }
    if (total_mem) *total_mem = pr.totalGlobalMem;
    if (n_cu) *n_cu = pr.multiProcessorCount;
    return 0;
}

int qs_gen_row_seeds(uint64_t seed, int64_t row0, int n_rows, uint64_t *out) {
    if (!out || n_rows < 0 || row0 < 0) {
        qs_set_error("qs_gen_row_seeds: bad arguments");
        return QS_EINVAL;
    }
    for (int r = 0; r < n_rows; ++r) out[r] = qs_gen_row_seed(seed, (uint64_t)(row0 + r));
    return 0;
}

int qs_gen_history(uint64_t seed, int64_t row0, int n_rows, int hist_n, int n_vocab, int pool,
                   int32_t *out) {
    if (!out || n_rows < 0 || row0 < 0 || hist_n < 0 || n_vocab < 1 || pool < 0) {
        qs_set_error("qs_gen_history: bad arguments");
        return QS_EINVAL;
    }
    for (int r = 0; r < n_rows; ++r)
        for (int j = 0; j < hist_n; ++j)
            out[(int64_t)r * hist_n + j] =
                qs_gen_hist_id(seed, (uint64_t)(row0 + r), j, n_vocab, pool);
    return 0;
}

int qs_gen_logits_device(float *d_out, int64_t row_stride, int64_t row0, int n_rows,
                         int n_vocab, int dist, float sigma, float boost, uint64_t seed) {
    if (!d_out || n_rows < 1 || n_vocab < 1 || row_stride < n_vocab || dist < 0 || dist > 2) {
        qs_set_error("qs_gen_logits_device: bad arguments");
        return QS_EINVAL;
    }
    qs_gen_spec spec;
    memset(&spec, 0, sizeof spec);
    spec.dist = dist;
    spec.sigma = sigma;
    spec.boost = boost;
    spec.seed = seed;
    const int64_t n = (int64_t)n_rows * n_vocab;
    const int64_t blocks = (n + WG - 1) / WG;
    hipLaunchKernelGGL(k_gen, dim3((unsigned)blocks), dim3(WG), 0, 0, d_out, row_stride, row0,
                       n_rows, n_vocab, spec);
    HIP_TRY(hipGetLastError(), "k_gen launch");
    HIP_TRY(hipDeviceSynchronize(), "k_gen");
    return 0;
}

int qs_copy_device(void *d_dst, const void *d_src, size_t bytes, int iters) {
    return qs_copy_device_kind(d_dst, d_src, bytes, iters, 0);
}

int qs_copy_device_kind(void *d_dst, const void *d_src, size_t bytes, int iters, int kind) {
    if (!d_dst || !d_src || bytes % 16 != 0 || bytes == 0 || iters < 1 || kind < 0 ||
        kind > 3 || (uintptr_t)d_dst % 16 != 0 || (uintptr_t)d_src % 16 != 0) {
        qs_set_error("qs_copy_device: bad arguments");
        return QS_EINVAL;
    }
    int dev = 0, ncu = 0;
    HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
    HIP_TRY(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev), "CUs");
    const int64_t n4 = (int64_t)(bytes / 16);
    int64_t blocks = (n4 + WG - 1) / WG;
    if (blocks > (int64_t)ncu * 16) blocks = (int64_t)ncu * 16;
    for (int i = 0; i < iters; ++i) {
        const dim3 g((unsigned)blocks), t(WG);
        if (kind == 0)
            hipLaunchKernelGGL(k_copy, g, t, 0, 0, (const float4 *)d_src, (float4 *)d_dst, n4);
        else if (kind == 1)
            hipLaunchKernelGGL(k_copy_buf<false>, g, t, 0, 0, (const float4 *)d_src,
                               (float4 *)d_dst, n4);
        else if (kind == 2)
            hipLaunchKernelGGL(k_copy_buf<true>, g, t, 0, 0, (const float4 *)d_src,
                               (float4 *)d_dst, n4);
        else
            hipLaunchKernelGGL(k_copy1, g, t, 0, 0, (const float *)d_src, (float *)d_dst,
                               4 * n4);
    }
    HIP_TRY(hipGetLastError(), "k_copy launch");
    HIP_TRY(hipDeviceSynchronize(), "k_copy");
    return 0;
}

int qs_expf_device(const float *d_x, float *d_y, int64_t n) {
    if (!d_x || !d_y || n < 1) { qs_set_error("qs_expf_device: bad arguments"); return QS_EINVAL; }
    const int64_t blocks = (n + WG - 1) / WG;
    hipLaunchKernelGGL(k_expf, dim3((unsigned)blocks), dim3(WG), 0, 0, d_x, d_y, n);
    HIP_TRY(hipGetLastError(), "k_expf launch");
    HIP_TRY(hipDeviceSynchronize(), "k_expf");
    return 0;
}

}  // extern "C"
