// qs_batch.hip - the device batch: per-row state in HBM, the gfx950 kernels, and the C ABI
// (include/quasar_sampler.h, parts 2 and 3).
//
// One pick of a batch of B rows (reference semantics: sample.c:111-179) runs as
//
//   k_scan     grid S x B  Stream each row slice once with 16-byte loads; apply the
//                          repeat penalty from an LDS bitmap of the history; reduce the
//                          slice max (and, for greedy rows, the first argmax); keep each
//                          wavefront's top-K penalised logits in an LDS buffer by ballot
//                          compaction plus a bit-serial select, tracking the largest logit
//                          it rejected.
//   k_expsum   grid S x B  Second pass (served from the last-level cache at the workload
//                          sizes): exact softmax numerators expf(x*inv_t - msc) with the
//                          host-libm-equal expf, double partial sums, window counts.
//   k_finalize grid B      Gather the per-wave top-K lists, radix-select the row's top K by
//                          logit, compute their exact p, bitonic-sort by (p desc, id asc),
//                          prove that no rejected logit can reach the prefix the cuts read,
//                          then run top-k / top-p / min-p / the xorshift draw exactly as
//                          sample.c does and record the id.  Rows where the proof fails
//                          (large nucleus, ties across the boundary, non-finite maxima)
//                          go to a work list.
//   k_full     grid <=256  For each listed row: materialise the whole window as 64-bit
//                          (p, id) keys, LSD-radix-sort them on the device, and run the
//                          reference's sequential cuts and draw over the sorted window.
//
// Everything a pick changes (generator state, history ring) stays on the device.
// Floating-point semantics follow the reference bit for bit: the build uses
// -ffp-contract=off, correctly rounded float division, IEEE denormals, and the expf in
// qs_expf.h.

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/quasar_sampler.h"
#include "qs_expf.h"
#include "qs_gen.h"
#include "qs_internal.h"

namespace {

constexpr int WG = 256;              // threads per workgroup
constexpr int NW = WG / 64;          // wavefronts per workgroup
constexpr int U = 4;                 // 16-byte loads in flight per thread per step
constexpr int K_MAX = 512;           // largest top-k preselected on the fast path
constexpr int K_OFF = 64;            // candidates kept per wave when top-k is off
constexpr int FIN_CAP = 4096;        // candidates k_finalize gathers into LDS
constexpr int SORT_CAP = 2048;       // kept candidates k_finalize sorts
constexpr int SLOTS = 256;           // rows k_full works on at once (scratch slots)
constexpr int S_MAX = 64;            // slices per row
constexpr int SLICE_QUANT = 1024;    // slice length granularity (elements)
constexpr int TARGET_WGS = 2048;     // workgroups k_scan aims for
constexpr int SLICE_MAX = 1 << 18;   // longest slice (its history bitmap lives in LDS)

__constant__ uint64_t c_exp_tab[QS_EXPF_TAB_N] = QS_EXPF_TABLE_INIT;

// ---- small device helpers --------------------------------------------------------------

// Order-preserving map of float bit patterns to unsigned keys (-0 sorts below +0).
__device__ __forceinline__ uint32_t f2key(float f) {
    uint32_t b = __float_as_uint(f);
    return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

__device__ __forceinline__ int lane_prefix(uint64_t m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ int wave_sum_i(int v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max_f(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
    for (int o = 32; o > 0; o >>= 1) {
        uint32_t t = __shfl_xor(v, o, 64);
        v = t > v ? t : v;
    }
    return v;
}

// sample.c:124: a flagged logit is divided by the penalty when positive, multiplied
// otherwise (so -0, NaN and -inf stay as they are, +inf stays +inf).
__device__ __forceinline__ float penalise(float l, float rp) {
    return l > 0.0f ? l / rp : l * rp;
}

// sample.c:72-81.
__device__ __forceinline__ double rng_unit(uint64_t &st) {
    uint64_t x = st;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    st = x;
    return (double)((x * 0x2545F4914F6CDD1Dull) >> 11) * (1.0 / 9007199254740992.0);
}

// sample.c:83-92.
__device__ __forceinline__ void ring_record(int32_t *ring, int32_t *hlen, int32_t *hhead,
                                            int cap, int id) {
    if (cap <= 0) return;
    int len = *hlen, head = *hhead;
    if (len < cap) {
        ring[(head + len) % cap] = id;
        *hlen = len + 1;
    } else {
        ring[head] = id;
        *hhead = (head + 1) % cap;
    }
}

// Candidates kept per wavefront for a sampling row.  Any value is correct (k_finalize
// proves or rejects the preselection); this one covers top_k exactly when it is small.
__host__ __device__ __forceinline__ int row_ksel(const qs_row_param &p) {
    return p.top_k > 0 ? (p.top_k < K_MAX ? p.top_k : K_MAX) : K_OFF;
}

__host__ __device__ __forceinline__ bool row_greedy(const qs_row_param &p) {
    return p.temperature <= 0.0f;      // sample.c:130 (a NaN temperature samples)
}

struct RowState {
    const qs_row_param *prm;
    uint64_t *rng;
    int32_t *ring;
    int32_t *hlen;
    int32_t *hhead;
    int ring_stride;
};

struct Scratch {
    float *smax;          // [B*S] slice max of penalised logits
    float *bestv;         // [B*S] greedy: slice max value
    int32_t *besti;       // [B*S] greedy: its first index (-1: none)
    uint32_t *ckey;       // [B*S*NW*capw] candidate keys (f2key of penalised logit)
    int32_t *cid;         // [B*S*NW*capw] candidate ids
    int32_t *ccnt;        // [B*S*NW] candidates per list
    uint32_t *crej;       // [B*S*NW] largest rejected key (0: none)
    int32_t *cflag;       // [B*S*NW] 1: list overflowed (ties), proof impossible
    double *psum;         // [B*S] double partial softmax denominators
    int32_t *pcnt;        // [B*S] window counts
    int32_t *full_list;   // [B] rows for k_full
    int32_t *full_count;  // [1]
    uint64_t *full_keys;  // [SLOTS][2][vocab]
    uint32_t *full_bm;    // [SLOTS][vocab/32+1]
};

struct Geometry {
    const float *logits;
    int64_t stride;
    int vocab;
    int n_rows;
    int slices;
    int slice_len;
    int capw;             // per-wave candidate buffer entries
    int bm_words;         // LDS bitmap words per slice
};

// History membership of [lo, lo + 32*words) as a bitmap in LDS (ids outside are skipped;
// duplicates set the same bit, so each id is penalised once, as sample.c:120 does).
__device__ void build_bitmap(uint32_t *bm, int words, int lo, int hi, const RowState &st,
                             int row, int cap) {
    for (int j = threadIdx.x; j < words; j += WG) bm[j] = 0u;
    __syncthreads();
    const int len = st.hlen[row], head = st.hhead[row];
    const int32_t *ring = st.ring + (int64_t)row * st.ring_stride;
    for (int j = threadIdx.x; j < len; j += WG) {
        int id = ring[(head + j) % cap];
        if (id >= lo && id < hi) atomicOr(&bm[(id - lo) >> 5], 1u << ((id - lo) & 31));
    }
    __syncthreads();
}

// Four consecutive logits starting at element 4c; elements at or past `hi` read as NaN
// (NaN never raises a max, never passes a filter and never enters the window).
template <bool VEC>
__device__ __forceinline__ float4 load4(const float *x, int c, int hi) {
    const int i = c << 2;
    if (VEC && i + 3 < hi) return *((const float4 *)x + c);
    const float q = __builtin_nanf("");
    float4 v;
    v.x = i < hi ? x[i] : q;
    v.y = i + 1 < hi ? x[i + 1] : q;
    v.z = i + 2 < hi ? x[i + 2] : q;
    v.w = i + 3 < hi ? x[i + 3] : q;
    return v;
}

// K-th largest key among the n entries of one wavefront's buffer (bit-serial search:
// the largest t with #(key >= t) >= k).  Wave-uniform result.
__device__ uint32_t wave_kth(const uint32_t *keys, int n, int k, int lane) {
    uint32_t prefix = 0u;
    for (int b = 31; b >= 0; --b) {
        const uint32_t cand = prefix | (1u << b);
        int c = 0;
        for (int j = lane; j < n; j += 64) c += keys[j] >= cand ? 1 : 0;
        c = wave_sum_i(c);
        if (c >= k) prefix = cand;
    }
    return prefix;
}

// Keep the entries with key >= th (in place, order preserved); returns the new count and
// raises `rej` (per lane) to the largest dropped logit.
__device__ int wave_compact(uint32_t *keys, int32_t *ids, int n, uint32_t th, int lane,
                            float &rej) {
    int w = 0;
    for (int base = 0; base < n; base += 64) {
        const int j = base + lane;
        const bool valid = j < n;
        const uint32_t k = valid ? keys[j] : 0u;
        const int32_t id = valid ? ids[j] : 0;
        const bool keep = valid && k >= th;
        if (valid && !keep) rej = fmaxf(rej, key2f(k));
        const uint64_t m = __ballot(keep);
        if (keep) {
            const int pos = w + lane_prefix(m);
            keys[pos] = k;
            ids[pos] = id;
        }
        w += __popcll(m);
    }
    return w;
}

// ---- k_scan -------------------------------------------------------------------------------

template <bool VEC>
__global__ void __launch_bounds__(WG) k_scan(Geometry g, RowState st, Scratch sc) {
    extern __shared__ uint32_t lds[];
    __shared__ float red_f[NW];
    __shared__ int red_i[NW];

    const int slice = blockIdx.x, row = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const qs_row_param P = st.prm[row];
    const bool greedy = row_greedy(P);
    const int lo = slice * g.slice_len;
    const int hi = min(lo + g.slice_len, g.vocab);
    if (row == 0 && slice == 0 && tid == 0) *sc.full_count = 0;

    const float rp = P.repeat_penalty;
    const bool pen = rp > 1.0f && st.hlen[row] > 0 && P.ring_cap > 0;
    uint32_t *bm = lds;
    if (pen) build_bitmap(bm, g.bm_words, lo, hi, st, row, P.ring_cap);

    const int capw = g.capw;
    uint32_t *kbuf = lds + g.bm_words + wv * 2 * capw;
    int32_t *ibuf = (int32_t *)(kbuf + capw);
    const int K = greedy ? 1 : row_ksel(P);

    const float *x = g.logits + (int64_t)row * g.stride;
    float mx = -INFINITY;                 // max penalised logit
    float bv = -INFINITY;                 // greedy: best value, first index
    int bi = -1;
    int n = 0;                            // wave buffer count (wave-uniform)
    float thf = -FLT_MAX;                 // wave filter threshold (wave-uniform)
    float rej = -INFINITY;                // largest logit this lane rejected
    int ovf = 0;

    const int c0 = lo >> 2, c1 = (hi + 3) >> 2;
    for (int cb = c0; cb < c1; cb += WG * U) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = load4<VEC>(x, cb + u * WG + tid, hi);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i0 = (cb + u * WG + tid) << 2;
            float w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
            if (pen) {
                uint32_t nib = 0u;
                if (i0 < hi) {
                    const int r = i0 - lo;
                    nib = (bm[r >> 5] >> (r & 31)) & 0xFu;
                }
                if (__ballot(nib != 0u)) {
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if ((nib >> k) & 1u) w[k] = penalise(w[k], rp);
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) mx = w[k] > mx ? w[k] : mx;
            if (greedy) {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (w[k] > bv) { bv = w[k]; bi = i0 + k; }
            } else {
                bool ps[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) ps[k] = w[k] >= thf;
#pragma unroll
                for (int k = 0; k < 4; ++k) rej = fmaxf(rej, ps[k] ? -INFINITY : w[k]);
                if (__ballot(ps[0] | ps[1] | ps[2] | ps[3])) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const uint64_t m = __ballot(ps[k]);
                        if (ps[k]) {
                            const int pos = n + lane_prefix(m);
                            kbuf[pos] = f2key(w[k]);
                            ibuf[pos] = i0 + k;
                        }
                        n += __popcll(m);
                    }
                    if (n > capw - 256) {
                        uint32_t th = wave_kth(kbuf, n, K, lane);
                        n = wave_compact(kbuf, ibuf, n, th, lane, rej);
                        if (n > capw - 256) {
                            // Too many exact ties to keep: drop them all and give up the
                            // proof for this row (k_finalize sends it to k_full).
                            ovf = 1;
                            n = wave_compact(kbuf, ibuf, n, th + 1u, lane, rej);
                            th = th + 1u;
                        }
                        thf = key2f(th);
                    }
                }
            }
        }
    }

    // slice max
    float m = wave_max_f(mx);
    if (lane == 0) red_f[wv] = m;
    __syncthreads();
    if (tid == 0) {
        float t = red_f[0];
        for (int k = 1; k < NW; ++k) t = fmaxf(t, red_f[k]);
        sc.smax[row * g.slices + slice] = t;
    }
    const int list = (row * g.slices + slice) * NW + wv;
    if (greedy) {
        // first index of the slice maximum: (value desc, index asc), -1 = none
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            const bool better = oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi));
            if (better) { bv = ov; bi = oi; }
        }
        __syncthreads();
        if (lane == 0) { red_f[wv] = bv; red_i[wv] = bi; }
        __syncthreads();
        if (tid == 0) {
            float v0 = red_f[0];
            int i0 = red_i[0];
            for (int k = 1; k < NW; ++k) {
                const float ov = red_f[k];
                const int oi = red_i[k];
                if (oi >= 0 && (i0 < 0 || ov > v0 || (ov == v0 && oi < i0))) { v0 = ov; i0 = oi; }
            }
            sc.bestv[row * g.slices + slice] = v0;
            sc.besti[row * g.slices + slice] = i0;
        }
        return;
    }
    // final prune of this wave's list to its top K (ties kept)
    if (n > K) {
        const uint32_t th = wave_kth(kbuf, n, K, lane);
        n = wave_compact(kbuf, ibuf, n, th, lane, rej);
    }
    const float r = wave_max_f(rej);
    uint32_t *okey = sc.ckey + (int64_t)list * capw;
    int32_t *oid = sc.cid + (int64_t)list * capw;
    for (int j = lane; j < n; j += 64) {
        okey[j] = kbuf[j];
        oid[j] = ibuf[j];
    }
    if (lane == 0) {
        sc.ccnt[list] = n;
        sc.crej[list] = r > -INFINITY ? f2key(r) : 0u;
        sc.cflag[list] = ovf;
    }
}

// ---- k_expsum -----------------------------------------------------------------------------

template <bool VEC>
__global__ void __launch_bounds__(WG) k_expsum(Geometry g, RowState st, Scratch sc) {
    extern __shared__ uint32_t lds[];
    __shared__ uint64_t tab[QS_EXPF_TAB_N];
    __shared__ double red_d[NW];
    __shared__ int red_i[NW];

    const int slice = blockIdx.x, row = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const qs_row_param P = st.prm[row];
    if (row_greedy(P)) return;

    float maxl = -INFINITY;
    for (int s = 0; s < g.slices; ++s) maxl = fmaxf(maxl, sc.smax[row * g.slices + s]);
    const float inv_t = P.inv_t;
    const float msc = maxl * inv_t;
    const float thr = msc - 30.0f;
    if (!isfinite(msc)) {                          // k_finalize / k_full handle these rows
        if (tid == 0) {
            sc.psum[row * g.slices + slice] = 0.0;
            sc.pcnt[row * g.slices + slice] = 0;
        }
        return;
    }
    if (tid < QS_EXPF_TAB_N) tab[tid] = c_exp_tab[tid];
    const int lo = slice * g.slice_len;
    const int hi = min(lo + g.slice_len, g.vocab);
    const float rp = P.repeat_penalty;
    const bool pen = rp > 1.0f && st.hlen[row] > 0 && P.ring_cap > 0;
    uint32_t *bm = lds;
    if (pen) build_bitmap(bm, g.bm_words, lo, hi, st, row, P.ring_cap);
    __syncthreads();

    const float *x = g.logits + (int64_t)row * g.stride;
    double acc = 0.0;
    int cnt = 0;
    const int c0 = lo >> 2, c1 = (hi + 3) >> 2;
    for (int cb = c0; cb < c1; cb += WG * U) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = load4<VEC>(x, cb + u * WG + tid, hi);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i0 = (cb + u * WG + tid) << 2;
            float w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
            if (pen) {
                uint32_t nib = 0u;
                if (i0 < hi) {
                    const int r = i0 - lo;
                    nib = (bm[r >> 5] >> (r & 31)) & 0xFu;
                }
                if (__ballot(nib != 0u)) {
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if ((nib >> k) & 1u) w[k] = penalise(w[k], rp);
                }
            }
            float s[4];
            bool in[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                s[k] = w[k] * inv_t;
                in[k] = s[k] >= thr;
                cnt += in[k] ? 1 : 0;
            }
            if (__ballot(in[0] | in[1] | in[2] | in[3])) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float e = qs_expf_core(s[k] - msc, tab);
                    acc += in[k] ? (double)e : 0.0;
                }
            }
        }
    }
    const double a = wave_sum_d(acc);
    const int c = wave_sum_i(cnt);
    if (lane == 0) { red_d[wv] = a; red_i[wv] = c; }
    __syncthreads();
    if (tid == 0) {
        double t = 0.0;
        int ct = 0;
        for (int k = 0; k < NW; ++k) { t += red_d[k]; ct += red_i[k]; }
        sc.psum[row * g.slices + slice] = t;
        sc.pcnt[row * g.slices + slice] = ct;
    }
}

// ---- block-level select and sort (k_finalize) -------------------------------------------

// K-th largest of n keys in LDS, by 8-bit radix select (4 rounds of a 256-bin histogram).
__device__ uint32_t block_kth(const uint32_t *keys, int n, int k, uint32_t *hist, int *sh) {
    const int tid = threadIdx.x, lane = tid & 63;
    uint32_t prefix = 0u, pmask = 0u;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int j = tid; j < 256; j += WG) hist[j] = 0u;
        __syncthreads();
        for (int j = tid; j < n; j += WG) {
            const uint32_t u = keys[j];
            if ((u & pmask) == prefix) atomicAdd(&hist[(u >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid < 64) {
            uint32_t c[4];
            for (int q = 0; q < 4; ++q) c[q] = hist[4 * lane + q];
            const uint32_t mine = c[0] + c[1] + c[2] + c[3];
            uint32_t incl = mine;           // sum over lanes >= this one
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_down(incl, o, 64);
                if (lane + o < 64) incl += t;
            }
            const uint32_t excl = incl - mine;
            const bool here = excl < (uint32_t)k && (uint32_t)k <= incl;
            if (here) {
                uint32_t run = excl;
                for (int q = 3; q >= 0; --q) {
                    if (run + c[q] >= (uint32_t)k) {
                        sh[0] = 4 * lane + q;
                        sh[1] = k - (int)run;
                        break;
                    }
                    run += c[q];
                }
            }
        }
        __syncthreads();
        prefix |= (uint32_t)sh[0] << shift;
        pmask |= 255u << shift;
        k = sh[1];
        __syncthreads();
    }
    return prefix;
}

// Sort n_pad (power of two) 64-bit keys in LDS, descending.
__device__ void bitonic_desc(uint64_t *s, int n_pad) {
    for (int size = 2; size <= n_pad; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < (n_pad >> 1); i += WG) {
                const int pos = 2 * i - (i & (stride - 1));
                const int par = pos + stride;
                const bool desc = (pos & size) == 0;
                const uint64_t a = s[pos], b = s[par];
                if ((a < b) == desc) { s[pos] = b; s[par] = a; }
            }
            __syncthreads();
        }
    }
}

struct FinArgs {
    Geometry g;
    RowState st;
    Scratch sc;
    int32_t *out;
    qs_pick_diag *diag;
    int gcap;             // LDS gather capacity (entries)
};

__device__ void write_diag(qs_pick_diag *diag, int row, const qs_pick_diag &d) {
    if (diag) diag[row] = d;
}

// The reference's row sums in slice order (deterministic).
__device__ void row_totals(const Scratch &sc, const Geometry &g, int row, float &maxl,
                           double &sum, int &nwin) {
    maxl = -INFINITY;
    sum = 0.0;
    nwin = 0;
    for (int s = 0; s < g.slices; ++s) {
        maxl = fmaxf(maxl, sc.smax[row * g.slices + s]);
        sum += sc.psum[row * g.slices + s];
        nwin += sc.pcnt[row * g.slices + s];
    }
}

__global__ void __launch_bounds__(WG) k_finalize(FinArgs a) {
    extern __shared__ uint32_t lds[];
    __shared__ uint64_t tab[QS_EXPF_TAB_N];
    __shared__ uint32_t hist[256];
    __shared__ int sh[8];
    __shared__ uint32_t shu[4];

    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const Geometry &g = a.g;
    const Scratch &sc = a.sc;
    const RowState &st = a.st;
    const qs_row_param P = st.prm[row];
    int32_t *ring = st.ring + (int64_t)row * st.ring_stride;
    qs_pick_diag d;
    memset(&d, 0, sizeof d);

    if (row_greedy(P)) {                                   // sample.c:130-134
        if (tid == 0) {
            float v0 = -INFINITY;
            int i0 = -1;
            for (int s = 0; s < g.slices; ++s) {
                const float ov = sc.bestv[row * g.slices + s];
                const int oi = sc.besti[row * g.slices + s];
                if (oi >= 0 && (i0 < 0 || ov > v0 || (ov == v0 && oi < i0))) { v0 = ov; i0 = oi; }
            }
            // sample.c scans from index 0 with a strict '>': nothing beats a NaN at 0, and
            // a row with no value above -inf stays at 0.
            const float x0 = g.logits[(int64_t)row * g.stride];
            int id = (i0 < 0 || isnan(x0)) ? 0 : i0;
            ring_record(ring, st.hlen + row, st.hhead + row, P.ring_cap, id);
            a.out[row] = id;
            d.id = id;
            d.path = QS_PATH_GREEDY;
            float mx = -INFINITY;
            for (int s = 0; s < g.slices; ++s) mx = fmaxf(mx, sc.smax[row * g.slices + s]);
            d.maxl = mx;
            d.keep = 1;
            write_diag(a.diag, row, d);
        }
        return;
    }

    float maxl;
    double sum;
    int nwin;
    row_totals(sc, g, row, maxl, sum, nwin);
    const float inv_t = P.inv_t;
    const float msc = maxl * inv_t;
    const float thr = msc - 30.0f;
    if (isnan(msc)) {
        // Empty window (thr is NaN): sample.c returns whatever id its scratch holds; here 0.
        if (tid == 0) {
            uint64_t rs = st.rng[row];
            d.u = rng_unit(rs);
            st.rng[row] = rs;
            ring_record(ring, st.hlen + row, st.hhead + row, P.ring_cap, 0);
            a.out[row] = 0;
            d.id = 0;
            d.path = QS_PATH_EMPTY;
            d.maxl = maxl;
            d.msc = msc;
            d.keep = 1;
            write_diag(a.diag, row, d);
        }
        return;
    }
    bool full = !isfinite(msc);

    // gather the per-wave lists
    const int nlist = g.slices * NW;
    const int list0 = row * nlist;
    uint32_t *keys = lds;
    int32_t *ids = (int32_t *)(lds + a.gcap);
    if (tid == 0) {
        int tot = 0, flag = 0;
        uint32_t rj = 0u;
        for (int l = 0; l < nlist; ++l) {
            tot += sc.ccnt[list0 + l];
            flag |= sc.cflag[list0 + l];
            const uint32_t r = sc.crej[list0 + l];
            rj = r > rj ? r : rj;
        }
        sh[0] = tot;
        sh[1] = flag;
        shu[0] = rj;
    }
    if (tid < QS_EXPF_TAB_N) tab[tid] = c_exp_tab[tid];
    __syncthreads();
    const int total = sh[0];
    if (sh[1] || total > a.gcap) full = true;
    uint32_t rej = shu[0];
    __syncthreads();

    if (!full) {
        // copy lists into LDS: list l starts at the prefix of counts before it
        if (wv == 0) {
            int base = 0;
            for (int l0 = 0; l0 < nlist; l0 += 64) {
                const int l = l0 + lane;
                const int c = l < nlist ? sc.ccnt[list0 + l] : 0;
                int incl = c;
                for (int o = 1; o < 64; o <<= 1) {
                    const int t = __shfl_up(incl, o, 64);
                    if (lane >= o) incl += t;
                }
                if (l < nlist) lds[a.gcap * 2 + l] = (uint32_t)(base + incl - c);
                base += __shfl(incl, 63, 64);
            }
        }
        __syncthreads();
        const uint32_t *offs = lds + a.gcap * 2;
        for (int l = wv; l < nlist; l += NW) {
            const int c = sc.ccnt[list0 + l];
            const uint32_t o = offs[l];
            const uint32_t *sk = sc.ckey + (int64_t)(list0 + l) * g.capw;
            const int32_t *si = sc.cid + (int64_t)(list0 + l) * g.capw;
            for (int j = lane; j < c; j += 64) {
                keys[o + j] = sk[j];
                ids[o + j] = si[j];
            }
        }
        __syncthreads();
    }

    // top-K of the gathered logits (ties kept); everything below goes into `rej`
    const int K = row_ksel(P);
    uint32_t th = 0u;
    if (!full && total > K) th = block_kth(keys, total, K, hist, sh);
    uint64_t *srt = (uint64_t *)(lds + a.gcap * 2 + ((nlist + 1) & ~1));
    if (tid == 0) sh[2] = 0;
    __syncthreads();
    // compact kept entries into the sort buffer as (p, ~id) keys
    const float inv = (float)(1.0 / sum);
    if (!full) {
        uint32_t myrej = 0u;
        for (int j0 = 0; j0 < total; j0 += WG) {
            const int j = j0 + tid;
            const bool valid = j < total;
            const uint32_t k = valid ? keys[j] : 0u;
            const bool keep = valid && k >= th;
            if (valid && !keep) myrej = k > myrej ? k : myrej;
            const uint64_t m = __ballot(keep);
            int wbase = 0;
            if (lane == 0 && m) wbase = atomicAdd(&sh[2], __popcll(m));
            wbase = __shfl(wbase, 0, 64);
            if (keep) {
                const int pos = wbase + lane_prefix(m);
                if (pos < SORT_CAP) {
                    const float w = key2f(k);
                    const float s = w * inv_t;
                    uint64_t key = 0ull;
                    if (s >= thr) {
                        const float e = qs_expf_core(s - msc, tab);
                        const float p = e * inv;
                        key = ((uint64_t)__float_as_uint(p) << 32) | (uint32_t)~(uint32_t)ids[j];
                    }
                    srt[pos] = key;
                }
            }
        }
        myrej = wave_max_u(myrej);
        if (lane == 0) atomicMax(&shu[0], myrej);
    }
    __syncthreads();
    const int nkept = sh[2];
    rej = shu[0];
    if (nkept > SORT_CAP) full = true;
    int npad = 1;
    while (npad < nkept) npad <<= 1;
    if (!full) {
        for (int j = nkept + tid; j < npad; j += WG) srt[j] = 0ull;
        __syncthreads();
        bitonic_desc(srt, npad);
    }

    if (tid == 0) {
        uint64_t rs = st.rng[row];
        int id = -1;
        if (!full) {
            // number of in-window kept entries (sorted first; p > 0 for all of them)
            int m = 0;
            while (m < nkept && (srt[m] >> 32) != 0ull) ++m;
            // Largest probability any rejected logit can have (monotone in the logit).
            float p_rej = -1.0f;
            if (rej != 0u) {
                const float s = key2f(rej) * inv_t;
                if (s >= thr) p_rej = qs_expf_core(s - msc, tab) * inv;
            }
            // Positions [0, E) of the sorted candidates are positions of the full order.
            int E = m;
            for (int i = 0; i < m; ++i)
                if (__uint_as_float((uint32_t)(srt[i] >> 32)) <= p_rej) { E = i; break; }
            if (m == nwin) E = m;
#define PAT(i) __uint_as_float((uint32_t)(srt[(i)] >> 32))
            bool ok = E >= 1;
            int n = nwin;                                         // sample.c:153-154
            if (P.top_k > 0 && P.top_k < n) n = P.top_k;
            d.keep_topk = n;
            if (ok && P.top_p < 1.0f) {                           // sample.c:155-160
                double cum = 0.0;
                int keep = n;
                for (int i = 0; i < n; ++i) {
                    if (i >= E) { ok = false; break; }
                    cum += PAT(i);
                    if (cum >= P.top_p) { keep = i + 1; break; }
                }
                n = keep;
            }
            d.keep_topp = n;
            if (ok && P.min_p > 0.0f) {                           // sample.c:161-168
                const float floor_p = P.min_p * PAT(0);
                int keep = n;
                for (int i = 1; i < n; ++i) {
                    if (i >= E) { ok = false; break; }
                    if (PAT(i) < floor_p) { keep = i; break; }
                }
                n = keep;
            }
            if (n < 1) n = 1;
            if (n > E) ok = false;
            if (ok) {                                             // sample.c:170-178
                double rsum = 0.0;
                for (int i = 0; i < n; ++i) rsum += PAT(i);
                const double u = rng_unit(rs);
                const double r = u * rsum;
                double acc = 0.0;
                int rank = n - 1;
                for (int i = 0; i < n; ++i) {
                    acc += PAT(i);
                    if (r <= acc) { rank = i; break; }
                }
                id = (int)~(uint32_t)(srt[rank] & 0xFFFFFFFFull);
                d.rank = rank;
                d.keep = n;
                d.rsum = rsum;
                d.u = u;
                d.p0 = PAT(0);
            }
#undef PAT
            d.n_cand = m;
            if (!ok) full = true;
        }
        if (full) {
            const int k = atomicAdd(a.sc.full_count, 1);
            a.sc.full_list[k] = row;
        } else {
            st.rng[row] = rs;
            ring_record(ring, st.hlen + row, st.hhead + row, P.ring_cap, id);
            a.out[row] = id;
            d.id = id;
            d.path = QS_PATH_FAST;
            d.n_window = nwin;
            d.maxl = maxl;
            d.msc = msc;
            d.inv = inv;
            d.sum = sum;
            write_diag(a.diag, row, d);
        }
    }
}

// ---- k_full: the whole window on the device ----------------------------------------------

struct FullArgs {
    Geometry g;
    RowState st;
    Scratch sc;
    int32_t *out;
    qs_pick_diag *diag;
};

// Stable LSD radix sort of n 64-bit keys, descending, 8 bits per pass; each wavefront
// owns a contiguous range and ranks equal digits by lane order (ballot multisplit).
// Returns the buffer holding the result (a or b).
__device__ uint64_t *radix_sort_desc(uint64_t *a, uint64_t *b, int n, uint32_t *whist,
                                     int *sh) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int ch = (n + NW - 1) / NW;
    const int beg = min(wv * ch, n), end = min(beg + ch, n);
    const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
    uint64_t *src = a, *dst = b;
    for (int shift = 0; shift < 64; shift += 8) {
        for (int j = tid; j < NW * 256; j += WG) whist[j] = 0u;
        __syncthreads();
        for (int base = beg; base < end; base += 64) {
            const int j = base + lane;
            if (j < end) atomicAdd(&whist[wv * 256 + 255 - (int)((src[j] >> shift) & 255u)], 1u);
        }
        __syncthreads();
        // exclusive offsets in (digit, wave) order; skip passes with a single digit
        {
            const int dg = tid;                 // one digit per thread (WG == 256)
            uint32_t tot = 0;
            for (int w = 0; w < NW; ++w) tot += whist[w * 256 + dg];
            if (tid == 0) sh[0] = 0;
            __syncthreads();
            if (tot == (uint32_t)n) sh[0] = 1;
            // block exclusive scan of tot over digits
            uint32_t incl = tot;
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_up(incl, o, 64);
                if (lane >= o) incl += t;
            }
            __shared__ uint32_t wsum[NW];
            if (lane == 63) wsum[wv] = incl;
            __syncthreads();
            uint32_t base = 0;
            for (int w = 0; w < wv; ++w) base += wsum[w];
            uint32_t run = base + incl - tot;
            for (int w = 0; w < NW; ++w) {
                const uint32_t c = whist[w * 256 + dg];
                whist[w * 256 + dg] = run;
                run += c;
            }
        }
        __syncthreads();
        if (sh[0]) { __syncthreads(); continue; }
        for (int base = beg; base < end; base += 64) {
            const int j = base + lane;
            const bool valid = j < end;
            const uint64_t key = valid ? src[j] : 0ull;
            const int dg = 255 - (int)((key >> shift) & 255u);
            uint64_t peers = __ballot(valid);
            for (int bit = 0; bit < 8; ++bit) {
                const bool on = (dg >> bit) & 1;
                const uint64_t bb = __ballot(on);
                peers &= on ? bb : ~bb;
            }
            if (valid) {
                const int rank = __popcll(peers & lt);
                const uint32_t pos = whist[wv * 256 + dg] + (uint32_t)rank;
                dst[pos] = key;
                const bool leader = (peers >> lane) == 1ull;
                if (leader) whist[wv * 256 + dg] += (uint32_t)__popcll(peers);
            }
        }
        __syncthreads();
        uint64_t *t = src;
        src = dst;
        dst = t;
    }
    return src;
}

__global__ void __launch_bounds__(WG) k_full(FullArgs a) {
    __shared__ uint64_t tab[QS_EXPF_TAB_N];
    __shared__ uint32_t whist[NW * 256];
    __shared__ int sh[4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int count = *a.sc.full_count;
    if (tid < QS_EXPF_TAB_N) tab[tid] = c_exp_tab[tid];
    const Geometry &g = a.g;
    const RowState &st = a.st;
    const int V = g.vocab;
    uint64_t *ka = a.sc.full_keys + (int64_t)blockIdx.x * 2 * V;
    uint64_t *kb = ka + V;
    uint32_t *bm = a.sc.full_bm + (int64_t)blockIdx.x * (V / 32 + 1);
    for (int q = blockIdx.x; q < count; q += gridDim.x) {
        const int row = a.sc.full_list[q];
        const qs_row_param P = st.prm[row];
        int32_t *ring = st.ring + (int64_t)row * st.ring_stride;
        float maxl;
        double sum;
        int nwin_unused;
        row_totals(a.sc, g, row, maxl, sum, nwin_unused);
        const float inv_t = P.inv_t;
        const float msc = maxl * inv_t;
        const float thr = msc - 30.0f;
        const bool deg = !isfinite(msc);           // every p is NaN (sample.c:148 on inf-inf)
        const float inv = (float)(1.0 / sum);
        const float rp = P.repeat_penalty;
        const bool pen = rp > 1.0f && st.hlen[row] > 0 && P.ring_cap > 0;
        if (pen) {
            for (int j = tid; j < V / 32 + 1; j += WG) bm[j] = 0u;
            __syncthreads();
            const int len = st.hlen[row], head = st.hhead[row];
            for (int j = tid; j < len; j += WG) {
                const int id = ring[(head + j) % P.ring_cap];
                if (id >= 0 && id < V) atomicOr(&bm[id >> 5], 1u << (id & 31));
            }
            __syncthreads();
        }
        if (tid == 0) sh[0] = 0;
        __syncthreads();
        const float *x = g.logits + (int64_t)row * g.stride;
        for (int i0 = 0; i0 < V; i0 += WG) {
            const int i = i0 + tid;
            bool in = false;
            uint64_t key = 0ull;
            if (i < V) {
                float w = x[i];
                if (pen && ((bm[i >> 5] >> (i & 31)) & 1u)) w = penalise(w, rp);
                const float s = w * inv_t;
                if (s >= thr) {
                    in = true;
                    uint32_t pb = 0u;
                    if (!deg) pb = __float_as_uint(qs_expf_core(s - msc, tab) * inv);
                    key = ((uint64_t)pb << 32) | (uint32_t)~(uint32_t)i;
                }
            }
            const uint64_t m = __ballot(in);
            int base = 0;
            if (lane == 0 && m) base = atomicAdd(&sh[0], __popcll(m));
            base = __shfl(base, 0, 64);
            if (in) ka[base + lane_prefix(m)] = key;
        }
        __syncthreads();
        const int nw = sh[0];
        __syncthreads();
        const uint64_t *srt = radix_sort_desc(ka, kb, nw, whist, sh + 1);
        if (tid == 0) {
            qs_pick_diag d;
            memset(&d, 0, sizeof d);
            uint64_t rs = st.rng[row];
            int id = 0;
            if (nw == 0) {
                d.u = rng_unit(rs);
                d.path = QS_PATH_EMPTY;
                d.keep = 1;
            } else {
                const float qnan = __builtin_nanf("");
#define PF(i) (deg ? qnan : __uint_as_float((uint32_t)(srt[(i)] >> 32)))
                int n = nw;                                       // sample.c:153-168
                if (P.top_k > 0 && P.top_k < n) n = P.top_k;
                d.keep_topk = n;
                if (P.top_p < 1.0f) {
                    double cum = 0.0;
                    int keep = n;
                    for (int i = 0; i < n; ++i) {
                        cum += PF(i);
                        if (cum >= P.top_p) { keep = i + 1; break; }
                    }
                    n = keep;
                }
                d.keep_topp = n;
                if (P.min_p > 0.0f) {
                    const float floor_p = P.min_p * PF(0);
                    int keep = n;
                    for (int i = 1; i < n; ++i)
                        if (PF(i) < floor_p) { keep = i; break; }
                    n = keep;
                }
                if (n < 1) n = 1;
                double rsum = 0.0;                                // sample.c:170-175
                for (int i = 0; i < n; ++i) rsum += PF(i);
                const double u = rng_unit(rs);
                const double r = u * rsum;
                double acc = 0.0;
                int rank = n - 1;
                for (int i = 0; i < n; ++i) {
                    acc += PF(i);
                    if (r <= acc) { rank = i; break; }
                }
                id = (int)~(uint32_t)(srt[rank] & 0xFFFFFFFFull);
                d.keep = n;
                d.rank = rank;
                d.rsum = rsum;
                d.u = u;
                d.p0 = PF(0);
#undef PF
                d.path = QS_PATH_FULL;
            }
            st.rng[row] = rs;
            ring_record(ring, st.hlen + row, st.hhead + row, P.ring_cap, id);
            a.out[row] = id;
            d.id = id;
            d.n_window = nw;
            d.n_cand = nw;
            d.maxl = maxl;
            d.msc = msc;
            d.inv = deg ? __builtin_nanf("") : inv;
            d.sum = deg ? (double)__builtin_nanf("") : sum;
            write_diag(a.diag, row, d);
        }
        __syncthreads();
    }
}

// ---- synthetic inputs ---------------------------------------------------------------------

__global__ void __launch_bounds__(WG) k_gen(float *out, int64_t stride, int64_t row0,
                                            int n_rows, int vocab, qs_gen_spec spec) {
    const int64_t idx = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (idx >= (int64_t)n_rows * vocab) return;
    const int64_t r = idx / vocab;
    const int c = (int)(idx - r * vocab);
    out[r * stride + c] = qs_gen_logit(&spec, (uint64_t)(row0 + r), c, vocab);
}

__global__ void __launch_bounds__(WG) k_expf(const float *x, float *y, int64_t n) {
    __shared__ uint64_t tab[QS_EXPF_TAB_N];
    if (threadIdx.x < QS_EXPF_TAB_N) tab[threadIdx.x] = c_exp_tab[threadIdx.x];
    __syncthreads();
    const int64_t i = (int64_t)blockIdx.x * WG + threadIdx.x;
    if (i < n) y[i] = qs_expf_tab(x[i], tab);
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
    const int cap = FIN_CAP / (NW * kmax_sel);
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
    int slice_rows = 0;                    // capacity of the per-slice scratch (rows*S)
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    std::vector<qs_row_param> h_prm;
    qs_row_param *d_prm = nullptr;
    uint64_t *d_rng = nullptr;
    int32_t *d_ring = nullptr, *d_hlen = nullptr, *d_hhead = nullptr;
    Scratch sc{};
    int slots = 0;
};

static void batch_release(qs_batch *b) {
    if (!b) return;
    if (b->stream) (void)hipStreamSynchronize(b->stream);
    void *ptrs[] = {b->d_prm, b->d_rng, b->d_ring, b->d_hlen, b->d_hhead, b->sc.smax,
                    b->sc.bestv, b->sc.besti, b->sc.ckey, b->sc.cid, b->sc.ccnt, b->sc.crej,
                    b->sc.cflag, b->sc.psum, b->sc.pcnt, b->sc.full_list, b->sc.full_count,
                    b->sc.full_keys, b->sc.full_bm};
    for (void *p : ptrs)
        if (p) (void)hipFree(p);
    if (b->ev0) (void)hipEventDestroy(b->ev0);
    if (b->ev1) (void)hipEventDestroy(b->ev1);
    if (b->stream) (void)hipStreamDestroy(b->stream);
    delete b;
}

static int batch_alloc(qs_batch *b) {
    const int R = b->max_rows, V = b->max_vocab;
    // rows*slices is at most max(R, min(TARGET_WGS, S_MAX*R))
    int sr = R;
    const int many = TARGET_WGS < S_MAX * R ? TARGET_WGS : S_MAX * R;
    if (many > sr) sr = many;
    b->slice_rows = sr;
    const int capw_max = K_MAX + 512;
    b->slots = R < SLOTS ? R : SLOTS;
    int rc = 0;
    if (!rc) rc = dev_alloc(&b->d_prm, R, "params");
    if (!rc) rc = dev_alloc(&b->d_rng, R, "rng");
    if (!rc) rc = dev_alloc(&b->d_ring, (size_t)R * (b->max_last_n > 0 ? b->max_last_n : 1), "ring");
    if (!rc) rc = dev_alloc(&b->d_hlen, R, "hlen");
    if (!rc) rc = dev_alloc(&b->d_hhead, R, "hhead");
    if (!rc) rc = dev_alloc(&b->sc.smax, sr, "smax");
    if (!rc) rc = dev_alloc(&b->sc.bestv, sr, "bestv");
    if (!rc) rc = dev_alloc(&b->sc.besti, sr, "besti");
    if (!rc) rc = dev_alloc(&b->sc.ckey, (size_t)sr * NW * capw_max, "ckey");
    if (!rc) rc = dev_alloc(&b->sc.cid, (size_t)sr * NW * capw_max, "cid");
    if (!rc) rc = dev_alloc(&b->sc.ccnt, (size_t)sr * NW, "ccnt");
    if (!rc) rc = dev_alloc(&b->sc.crej, (size_t)sr * NW, "crej");
    if (!rc) rc = dev_alloc(&b->sc.cflag, (size_t)sr * NW, "cflag");
    if (!rc) rc = dev_alloc(&b->sc.psum, sr, "psum");
    if (!rc) rc = dev_alloc(&b->sc.pcnt, sr, "pcnt");
    if (!rc) rc = dev_alloc(&b->sc.full_list, R, "full_list");
    if (!rc) rc = dev_alloc(&b->sc.full_count, 1, "full_count");
    if (!rc) rc = dev_alloc(&b->sc.full_keys, (size_t)b->slots * 2 * V, "full_keys");
    if (!rc) rc = dev_alloc(&b->sc.full_bm, (size_t)b->slots * (V / 32 + 1), "full_bm");
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

int qs_batch_pick(qs_batch *b, const float *d_logits, int64_t row_stride, int n_rows,
                  int n_vocab, int32_t *d_out, qs_pick_diag *d_diag) {
    if (!b || !d_logits || !d_out) { qs_set_error("qs_batch_pick: null argument"); return QS_EINVAL; }
    if (n_rows < 1 || n_rows > b->max_rows || n_vocab < 1 || n_vocab > b->max_vocab ||
        row_stride < n_vocab) {
        qs_set_error("qs_batch_pick: rows %d (max %d), vocab %d (max %d), stride %lld", n_rows,
                     b->max_rows, n_vocab, b->max_vocab, (long long)row_stride);
        return QS_EINVAL;
    }
    int kmax = 1;
    bool any_sample = false;
    for (int r = 0; r < n_rows; ++r) {
        const qs_row_param &p = b->h_prm[r];
        if (row_greedy(p)) continue;
        any_sample = true;
        const int k = row_ksel(p);
        if (k > kmax) kmax = k;
        if (p.ring_cap > b->max_last_n) { qs_set_error("ring capacity"); return QS_EINVAL; }
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
    g.capw = any_sample ? (kmax + 512 + 63) / 64 * 64 : 0;
    g.bm_words = g.slice_len / 32;
    RowState st{b->d_prm, b->d_rng, b->d_ring, b->d_hlen, b->d_hhead,
                b->max_last_n > 0 ? b->max_last_n : 1};
    const bool vec = ((uintptr_t)d_logits % 16 == 0) && (row_stride % 4 == 0);
    const dim3 grid(g.slices, n_rows);
    const size_t lds_scan = sizeof(uint32_t) * ((size_t)g.bm_words + (size_t)NW * 2 * g.capw);
    const size_t lds_exp = sizeof(uint32_t) * (size_t)g.bm_words;
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
    FinArgs fa{g, st, b->sc, d_out, d_diag, 0};
    int gcap = g.slices * NW * (g.capw > 0 ? g.capw : 1);
    if (gcap > FIN_CAP) gcap = FIN_CAP;
    fa.gcap = gcap;
    const int nlist = g.slices * NW;
    const size_t lds_fin = sizeof(uint32_t) * (2 * (size_t)gcap + ((nlist + 1) & ~1)) +
                           sizeof(uint64_t) * SORT_CAP;
    hipLaunchKernelGGL(k_finalize, dim3(n_rows), dim3(WG), any_sample ? lds_fin : 0, b->stream, fa);
    HIP_TRY(hipGetLastError(), "k_finalize launch");
    if (any_sample) {
        FullArgs ua{g, st, b->sc, d_out, d_diag};
        const int grid_full = n_rows < b->slots ? n_rows : b->slots;
        hipLaunchKernelGGL(k_full, dim3(grid_full), dim3(WG), 0, b->stream, ua);
        HIP_TRY(hipGetLastError(), "k_full launch");
    }
    return 0;
}

int qs_batch_synchronize(qs_batch *b) {
    if (!b) return QS_EINVAL;
    HIP_TRY(hipStreamSynchronize(b->stream), "qs_batch_synchronize");
    return 0;
}

void *qs_batch_stream(qs_batch *b) { return b ? (void *)b->stream : nullptr; }

int qs_batch_time_picks(qs_batch *b, const float *d_logits, int64_t row_stride, int n_rows,
                        int n_vocab, int32_t *d_out, int iters, float *ms) {
    if (!b || iters < 1 || !ms) return QS_EINVAL;
    HIP_TRY(hipEventRecord(b->ev0, b->stream), "event");
    for (int i = 0; i < iters; ++i) {
        const int rc = qs_batch_pick(b, d_logits, row_stride, n_rows, n_vocab, d_out, nullptr);
        if (rc) return rc;
    }
    HIP_TRY(hipEventRecord(b->ev1, b->stream), "event");
    HIP_TRY(hipEventSynchronize(b->ev1), "event sync");
    HIP_TRY(hipEventElapsedTime(ms, b->ev0, b->ev1), "elapsed");
    return 0;
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

int qs_expf_device(const float *d_x, float *d_y, int64_t n) {
    if (!d_x || !d_y || n < 1) { qs_set_error("qs_expf_device: bad arguments"); return QS_EINVAL; }
    const int64_t blocks = (n + WG - 1) / WG;
    hipLaunchKernelGGL(k_expf, dim3((unsigned)blocks), dim3(WG), 0, 0, d_x, d_y, n);
    HIP_TRY(hipGetLastError(), "k_expf launch");
    HIP_TRY(hipDeviceSynchronize(), "k_expf");
    return 0;
}

}  // extern "C"
