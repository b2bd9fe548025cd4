// qs_row.hip - the row pick: one workgroup per row streams the row's logits once and decides
// the row from LDS (sample.c:111-179), for batches of at least one row per CU.
//
// k_row<NW>, one workgroup of NW wavefronts per row (16: one workgroup per CU; 8: two per
// CU, one row deciding while the other streams).  The row is cut into chunks of 64 lanes x
// RU float4; each wavefront holds two chunks in registers (buffer loads; past the row they
// read nothing) and takes the next from the workgroup's LDS counter, so the row's
// wavefronts finish together.  At launch each wavefront requests its first chunk together
// with the history ring's first slots; the second goes out once the history bitmap is
// built.  No wavefront waits for another until the row is done:
//   1. the repeat penalty from the row's history bitmap in LDS and each chunk's mask of the
//      float4 groups holding a history id (sample.c:118-128); each lane's max and min
//      (NaN-propagating);
//   2. sampling rows: per logit sc = w * inv_t, t = fl(sc * L - c), e = 2^t (v_exp_f32),
//      summed in float quads then binary64, and e * t, against the wavefront's integer
//      exponent base c >= its running max * L; when a chunk raises the base the sums are
//      scaled by 2^-(rise), exactly.  At the end each wavefront's sums are one certified
//      part of the row's softmax denominator (qs_cert.h);
//   3. the candidates: every logit at or above the row's running bound, appended to the
//      wavefront's LDS list.  The bound is a ratchet shared through LDS: raised only when at
//      least K + 2 published running maxima (16-lane maxima, or every lane's for top-k
//      above 64) lie strictly above the new value, so at least K + 2 logits of the row do;
//      rows with other K take the smaller of each wavefront's m-th largest lane maximum and
//      the others' published ones.
// After one barrier the workgroup gathers the candidates above the row's rejected bound
// with their exact numerators, one wavefront totals the segments into the denominator
// interval, and the first four wavefronts take the row's decision: the certified decision
// (qs_cert.h) proved for every normaliser of the interval, with the exact path
// (qs_decide.h) for rows it does not cover.

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <algorithm>
#include <cstring>
#include <type_traits>

#include "../../include/quasar_sampler.h"
#include "qs_cert.h"
#include "qs_decide.h"
#include "qs_device.h"
#include "qs_launch.h"

using namespace qs;
using namespace qs::dec;

namespace {

// float4 per lane per chunk: 5 with 16 wavefronts a row (one row a CU), 6 with 8 (two rows a
// CU, where larger chunks, so fewer per-chunk steps, measured faster; both fit 128 VGPRs)
template <int NW>
constexpr int row_ru() { return NW == 8 ? 6 : 5; }
constexpr int RU = row_ru<16>();         // the 16-wavefront chunk (the read ceiling's too)
constexpr int RCH = 64 * RU;             // float4 per chunk
constexpr int ROW_VMAX = QS_ROW_MAX_VOCAB;   // longest row (its history bitmap is in LDS)
constexpr int RBM = ROW_VMAX / 32 + 4;   // bitmap words
constexpr uint32_t RATCHET_STEP = 1u << 17;   // the threshold ratchet's first step (keys)
constexpr int LIST_CAP = 2048;           // candidates all of a row's lists hold (16
                                         // wavefronts; 8 wavefronts: twice that, two
                                         // workgroups sharing a CU's 160 KB of LDS)
constexpr float C_INIT = -0x1p24f;       // a lane's exponent base before its first finite max
constexpr int BUF_WORD3 = 0x00020000;    // raw buffer, 32-bit data format
constexpr int BUF_NT = 2;                // nontemporal: each logit is read once

__constant__ uint64_t c_tab_row[QS_EXPF_TAB_N] = QS_EXPF_TABLE_INIT;

// The timeline build (make timeline: -DQS_TIMELINE) records the 100 MHz clock at the phase
// boundaries of each wavefront of rows below TLR_ROWS, for quasar_amd/timeline.py:
// 0 start, 1 bitmap built, 2 first chunk's data in, 3 segment done, 4 every segment done,
// 5 candidates gathered, 6 decided (wavefront 0).
#ifdef QS_TIMELINE
constexpr int TLR_ROWS = 4096, TLR_W = 16;
__device__ uint64_t g_tl_row[TLR_ROWS * TLR_W * 8];
#define TL_ROW(e)                                                                             \
    do {                                                                                      \
        if ((threadIdx.x & 63) == 0 && blockIdx.x < TLR_ROWS)                                 \
            g_tl_row[(blockIdx.x * TLR_W + (threadIdx.x >> 6)) * 8 + (e)] =                   \
                __builtin_amdgcn_s_memrealtime();                                             \
    } while (0)
#else
#define TL_ROW(e) ((void)0)
#endif

// One wavefront's chunks (its segment): one certified part, and what the window count and
// the candidate gather need.
struct SegRec {
    double sum;                          // sum of e^ against base c
    double term;                         // sum of e^ * (-t) against base c
    float c;                             // the base (integer-valued)
    uint32_t maxk;                       // largest penalised logit (key)
    uint32_t mink;                       // least non-NaN penalised logit (key; ~0u: none)
    int nan;                             // NaNs
    int len;                             // logits
    uint32_t rej;                        // bound on every logit not in the list (key)
    int cnt;                             // candidates found (above the capacity: overflowed)
};

template <int NW>
struct RowLds {
    static constexpr int WCAP = (NW == 8 ? 2 : 1) * LIST_CAP / NW;   // candidates per
                                                                     // wavefront list
    union {
        uint32_t bm[RBM];                // streaming: the row's history ids (bit per logit)
        DecLds dl;                       // decision (the bitmap is dead by then)
    };
    static constexpr int NCH = (ROW_VMAX / 4 + 64 * row_ru<NW>() - 1) / (64 * row_ru<NW>());
    uint32_t hitu[NCH];                  // chunk j: bit u set when its float4 group u holds a
                                         // history id
    int next;                            // the row's next chunk to take
    uint32_t theta[NW];                  // published running thresholds (keys)
    uint32_t pub[NW * 64];               // ratchet rows: the 16-lane maxima of the running
                                         // lane maxima, 4 per wavefront, or (top K above
                                         // 64) every lane's running maximum (0: not yet)
    uint32_t rth, rstep;                 // the ratchet's threshold (0: not seeded) and step
    SegRec seg[NW];
    uint32_t ckey[NW][WCAP];
    int32_t cid[NW][WCAP];
    uint64_t tab[QS_EXPF_TAB_N];         // the expf table (the decision's copy is in dl)
    uint64_t gk[WAVE_CAND];              // gathered candidates' (e, ~id) keys (0: outside the
                                         // window), e the exact numerator
    int gcount, gwin;                    // gathered candidates; those in the window
    float e64;                           // numerator ranked 64th (rows with more in the window)
    float e_rej;                         // numerator bound of every logit not gathered
    CertTotals ct;
    float gbv[NW];                       // greedy rows: each list's first maximum
    int gbi[NW];
};

// A workgroup barrier over LDS only: __syncthreads() also waits for every global load in
// flight (the next chunks'); the wavefronts share nothing but LDS here.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 bload(__amdgpu_buffer_rsrc_t rs, int off) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, BUF_NT);
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z),
                       __uint_as_float(v.w));
}
// Chunk j of a segment into registers (lane l, float4 u of U: segment float4
// j*64*U + u*64 + l).
template <int U>
__device__ __forceinline__ void load_chunk(float4 (&X)[U], __amdgpu_buffer_rsrc_t rs, int j,
                                           int lane) {
#pragma unroll
    for (int u = 0; u < U; ++u) X[u] = bload(rs, (j * 64 * U + u * 64 + lane) * 16);
}

template <typename T>
__device__ __forceinline__ T lds_ld(const T *p) {
    return __hip_atomic_load(const_cast<T *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
template <typename T>
__device__ __forceinline__ void lds_st(T *p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Candidates wanted above the row's bound: the threshold rule keeps about 2 NW m logits
// above it; m0 for a wavefront's first chunk (nothing published yet).
__device__ __forceinline__ int row_m(const qs_row_param &P, int nw) {
    if (row_greedy(P)) return 1;
    const int m = (row_ksel(P) + 8 + nw - 1) / nw;
    return m < 64 ? m : 64;
}

// At least 4 wavefronts per SIMD (at most 128 VGPRs): one 16-wavefront or two 8-wavefront
// workgroups per CU.
template <int NW>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(4))) k_row(PartArgs a) {
    static_assert(NW <= 16, "the segment records are reduced over lanes 0-15");
    constexpr int RU = row_ru<NW>(), RCH = 64 * RU;   // this kernel's chunk
    __shared__ RowLds<NW> rl;
    constexpr int WCAP = RowLds<NW>::WCAP;
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    TL_ROW(0);
    const qs_row_param P = row_param(a.st, row);
#ifdef QS_TIMELINE
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    QS_TL_HOOK(12);
#endif
    const bool greedy = row_greedy(P);
    const float inv_t = P.inv_t, rp = P.repeat_penalty;
    const int V = a.vocab, n4 = V >> 2;
    const int nch = (n4 + RCH - 1) / RCH;           // chunks of the row
    const float *rowp = a.logits + (int64_t)row * a.stride;
    // the loads the bitmap and the decision need go out before any chunk load: a load
    // issued behind the first chunks of every workgroup waits for them.  The ring's first
    // slots are read over the batch's ring stride (not the row's capacity, which is in the
    // parameters still on their way), so that they and the first chunks need nothing loaded
    const int32_t *ring = a.st.ring + (int64_t)row * a.st.ring_stride;
    const __amdgpu_buffer_rsrc_t rr =
        __builtin_amdgcn_make_buffer_rsrc((void *)ring, 0, a.st.ring_stride * 4, BUF_WORD3);
    const int slot0 = (int)__builtin_amdgcn_raw_buffer_load_b32(rr, tid * 4, 0, 0);
    // this wavefront's first chunk (chunk wv; the last wavefront's also the row's partial
    // last chunk) goes out now and arrives while the bitmap is built; its second after the
    // bitmap (a wavefront whose loads wait for room in the CU's memory queue then holds up
    // no other wavefront at the barriers)
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)rowp, 0, n4 * 16, BUF_WORD3);
    float4 A[RU], B[RU], T[RU];
    const int nr = n4 / RCH;                        // whole chunks
    int jA = wv, jB = NW + wv;
    if (nr < nch && wv == NW - 1) load_chunk(T, rs, nr, lane);
    load_chunk(A, rs, jA, lane);
    const int cap = P.repeat_penalty > 1.0f ? P.ring_cap : 0;   // sample.c:119 (clamped: row_param)
    const uint64_t tabv = tid < QS_EXPF_TAB_N ? c_tab_row[tid] : 0ull;
    RowHist hist{0ull, 0, 0};
    if (wv == 0 && !greedy) hist = row_hist(a.st, row);
    int hlen, hhead;
    ring_pos(a.st, row, cap, hlen, hhead);
    const float x0 = rowp[0];
    // the history bitmap and each chunk's hit bit
    const int bw = ((n4 + 7) / 8 + 3) / 4;       // uint4s of bitmap words in use
    for (int i = tid; i < bw; i += NW * 64) ((uint4 *)rl.bm)[i] = make_uint4(0u, 0u, 0u, 0u);
    for (int i = tid; i < nch; i += NW * 64) rl.hitu[i] = 0u;
    if (tid < NW) rl.theta[tid] = 0xFFFFFFFFu;
    rl.pub[tid] = 0u;
    if (tid == 0) {
        rl.rth = 0u;
        rl.rstep = RATCHET_STEP;
        rl.next = 2 * NW;
        rl.gcount = 0;
        rl.gwin = 0;
    }
    if (tid < QS_EXPF_TAB_N) rl.tab[tid] = tabv;
#ifdef QS_TIMELINE
    asm volatile("" ::"v"(slot0) : "memory");
    QS_TL_HOOK(13);
#endif
    lds_barrier();
    QS_TL_HOOK(14);
    auto mark = [&](int p, int id) {
        if (qs_ring_live(cap, hlen, hhead, p) && id >= 0 && id < V) {   // each id once (a bit)
            atomicOr(&rl.bm[id >> 5], 1u << (id & 31));
            const int f = id >> 2, ch = f / RCH, r = f - ch * RCH;
            atomicOr(&rl.hitu[ch], 1u << (r >> 6));
        }
    };
    mark(tid, slot0);
    for (int p = NW * 64 + tid; p < cap; p += NW * 64) mark(p, ring[p]);
    asm volatile("" ::: "memory");                  // the chunk loads go out after the ring's
    QS_TL_HOOK(15);
    lds_barrier();
    TL_ROW(1);
    // the second chunk of this wavefront (chunk NW + wv; later ones are taken from the
    // workgroup's counter, so the wavefronts of a row finish together)
    load_chunk(B, rs, jB, lane);
    TL_ROW(7);
    const bool pen = cap > 0;
    const double rinv = 1.0 / (double)rp;           // penalise_r's reciprocal
    // the threshold rule: rows with a small top K take the smaller of the two 32-lane maxima
    // of the running lane maxima (at least 2 logits per wavefront reach it); others the m-th
    // largest running lane maximum
    const int m = row_m(P, NW), m0 = m <= 8 ? 2 * m : m;
    const bool halves = row_greedy(P) || row_ksel(P) + 8 <= 4 * NW;
    // rows with top K up to 48 (16 wavefronts): the ratchet rule over 16-lane maxima,
    // kp = K + 2 published maxima strictly above the bound (about K + 20 candidates end
    // above it); rows with top K above 64: the ratchet over every lane's maximum.  A
    // candidate only counts in the decision's proven prefix when its numerator clears the
    // bound's, so the ones equal to the bound do not; the two spare ones cover numerators
    // within rounding of it.
    const int kp = row_ksel(P) + 2;
    const bool rat_lane = !row_greedy(P) && row_ksel(P) > 64 && kp <= NW * 64;
    const bool ratchet = rat_lane || (!row_greedy(P) && row_ksel(P) <= 48 && 4 * NW >= 64);
    const int m_first = min(64, max(6, (row_ksel(P) + 7) / 8));
    auto take = [&]() {                             // the next chunk of the row (uniform)
        int j = 0;
        if (lane == 0) j = atomicAdd(&rl.next, 1);
        return __builtin_amdgcn_readfirstlane(j);
    };

    // per lane: sums against the wavefront's base cw, running max key, least key, NaNs
    double accS = 0.0, accT = 0.0;
    uint32_t run = 0u, mink = 0xFFFFFFFFu;
    int nan = 0;
    float cw = C_INIT;                              // the wavefront's exponent base (uniform)
    uint32_t rej_w = 0u;
    int wn = 0, len = 0, first = 1;
    uint32_t th0 = 0u;                              // the ratchet's bound before it is seeded
    uint32_t thw_r = 0u, stp_r = RATCHET_STEP;      // other rows: this wavefront's statistic
                                                    // after its first chunk, and its step
    uint32_t wmx_base = 0xFFFFFFFFu;                // the max key the base was last set from
    auto chunk = [&](auto tail_c, float4 (&X)[RU], int j) {
        constexpr bool tail = decltype(tail_c)::value;   // the row's partial last chunk
        const int f0 = j * RCH;
        len += 4 * min(RCH, n4 - f0);
        // sample.c:124 on this chunk's history ids, float4 group by group from the bitmap
        // (the groups of the chunk that hold one; their bitmap words read together), without
        // a branch per id
        if (pen) {
            const uint32_t um = (uint32_t)__builtin_amdgcn_readfirstlane((int)rl.hitu[j]);
            if (um) {
                uint32_t wd[RU];
#pragma unroll
                for (int u = 0; u < RU; ++u) {
                    const int f = f0 + u * 64 + lane;
                    wd[u] = (um >> u) & 1u ? rl.bm[min(f >> 3, RBM - 1)] : 0u;
                }
#pragma unroll
                for (int u = 0; u < RU; ++u) {
                    if (!((um >> u) & 1u)) continue;
                    const int f = f0 + u * 64 + lane;
                    const uint32_t nib = (wd[u] >> ((f & 7) * 4)) & 0xFu;
                    float w[4] = {X[u].x, X[u].y, X[u].z, X[u].w};
                    if (__ballot((nib & (nib - 1u)) != 0u)) {
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const float v = penalise_r(w[k], rp, rinv);
                            w[k] = (nib >> k) & 1u ? v : w[k];
                        }
                    } else {
                        // at most one history id per lane in this group: penalise that one
                        const bool h1 = nib == 2u, h2 = nib == 4u, h3 = nib == 8u;
                        const float x = h1 ? w[1] : h2 ? w[2] : h3 ? w[3] : w[0];
                        const float v = penalise_r(x, rp, rinv);
                        w[0] = nib == 1u ? v : w[0];
                        w[1] = h1 ? v : w[1];
                        w[2] = h2 ? v : w[2];
                        w[3] = h3 ? v : w[3];
                    }
                    X[u] = make_float4(w[0], w[1], w[2], w[3]);
                }
            }
        }
        // each lane's max and min (positions past the row: -inf, not in the min)
        float mx = -INFINITY, mn = INFINITY;
        if constexpr (!tail) {
#pragma unroll
            for (int u = 0; u < RU; ++u) {
                mn = min3n(min3n(mn, X[u].x, X[u].y), X[u].z, X[u].w);
                mx = max3n(max3n(mx, X[u].x, X[u].y), X[u].z, X[u].w);
            }
        } else {
#pragma unroll
            for (int u = 0; u < RU; ++u) {
                if (f0 + u * 64 + lane >= n4) {
                    X[u] = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
                } else {
                    mn = min3n(min3n(mn, X[u].x, X[u].y), X[u].z, X[u].w);
                    mx = max3n(mx, max3n(X[u].x, X[u].y, X[u].z), X[u].w);
                }
            }
        }
#ifdef QS_TIMELINE
        if (first) {
            asm volatile("" ::"v"(mx), "v"(mn) : "memory");   // the chunk's data is in
            TL_ROW(2);
        }
#endif
        int nanc = 0;
        if (__ballot(mx != mx || mn != mn)) {    // a NaN: not a max, not in the min, counted
            mx = -INFINITY;
            mn = INFINITY;
#pragma unroll
            for (int u = 0; u < RU; ++u) {
                const bool past = tail && f0 + u * 64 + lane >= n4;
                const float w[4] = {X[u].x, X[u].y, X[u].z, X[u].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    nanc += w[k] != w[k];
                    mx = w[k] > mx ? w[k] : mx;
                    mn = (w[k] < mn && !past) ? w[k] : mn;
                }
            }
        }
        nan += nanc;
        if (mn != INFINITY) mink = min(mink, f2key(mn));
        const uint32_t tmk = f2key(mx);
        run = max(run, tmk);
        // the four 16-lane maxima of the running maxima (lanes 15, 31, 47, 63), in DPP moves
        uint32_t h = run;
        h = max(h, dpp_move<0xB1, 0xF>(h));
        h = max(h, dpp_move<0x4E, 0xF>(h));
        h = max(h, dpp_move<0x141, 0xF>(h));
        h = max(h, dpp_move<0x140, 0xF>(h));
        const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)h, 15);
        const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)h, 31);
        const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)h, 47);
        const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)h, 63);
        const uint32_t h0 = max(r0, r1), h1 = max(r2, r3);
        const uint32_t wmx = max(h0, h1);
        if (!greedy) {
            // the base: raised to the wavefront's running max (an exact rescale of its sums)
            if (wmx != wmx_base) {
                wmx_base = wmx;
                const float Mw = key2f(wmx) * inv_t;
                float cn = (Mw > -INFINITY && Mw < INFINITY) ? cert_cbase(Mw) : cw;
                cn = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(cn)));
                if (cn > cw) {
                    const float d = cn - cw;
                    const int sh = -(int)fminf(d, 4096.0f);
                    accT = ldexp(accT - (double)d * accS, sh);
                    accS = ldexp(accS, sh);
                    cw = cn;
                }
            }
            const bool dirty = tail || __ballot(!(mn * inv_t >= SC_SANE) || nanc != 0) != 0ull;
            float Tn = 0.0f;
            if (dirty) {
#pragma unroll
                for (int u = 0; u < RU; ++u) sum4<true>(X[u], inv_t, cw, accS, Tn);
            } else {
#pragma unroll
                for (int u = 0; u < RU; ++u) sum4<false>(X[u], inv_t, cw, accS, Tn);
            }
            accT += (double)Tn;
        }
        uint32_t th;
        if (ratchet) {
            // the row's threshold: a ratchet over the published maxima (the 4 NW 16-lane
            // maxima, each a distinct logit, or with rat_lane every lane's running maximum),
            // raised only when at least kp of them lie strictly above the new value (so at
            // least kp logits of the row do).  It starts at the largest first-chunk bound a
            // wavefront has entered (below), or, before any has, at a seed once kp are
            // published: one key below the least 16-lane maximum or below the kp-th largest
            // lane maximum.
            uint32_t pv = 0u;
            if (rat_lane) {
                rl.pub[wv * 64 + lane] = run;
            } else {
                if ((lane & 15) == 15) rl.pub[wv * 4 + (lane >> 4)] = h;
                pv = rl.pub[lane];
            }
            // published values above x (x = 0: published at all), over the wavefront
            auto count_above = [&](uint32_t x) -> int {
                if (!rat_lane) return (int)__popcll(__ballot(pv > x));
                int c = 0;
#pragma unroll
                for (int v = 0; v < NW; ++v) c += (int)__popcll(__ballot(rl.pub[v * 64 + lane] > x));
                return c;
            };
            uint32_t rt = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_ld(&rl.rth));
            const uint32_t st = (uint32_t)__builtin_amdgcn_readfirstlane((int)lds_ld(&rl.rstep));
            if (rt == 0u) {
                if (count_above(0u) >= kp) {
                    // kp published: one key below their least (16-lane maxima), or below the
                    // kp-th largest published lane maximum (a bitwise search: the largest x
                    // with at least kp published values at or above it)
                    if (rat_lane) {
                        uint32_t x = 0u;
                        for (int b = 31; b >= 0; --b) {
                            const uint32_t y = x | (1u << b);
                            if (count_above(y - 1u) >= kp) x = y;
                        }
                        rt = x - 1u;
                    } else {
                        rt = wave_min_u(pv != 0u ? pv : 0xFFFFFFFFu) - 1u;
                    }
                    if (lane == 0 && rt) atomicMax(&rl.rth, rt);
                }
            } else {
                const uint32_t cand = rt + st > rt ? rt + st : 0xFFFFFFFFu;
                if (count_above(cand) >= kp) {
                    if (lane == 0) {
                        atomicMax(&rl.rth, cand);
                        lds_st(&rl.rstep, st < 0x40000000u ? 2u * st : st);
                    }
                    rt = cand;
                } else if (lane == 0) {
                    lds_st(&rl.rstep, st > 1u ? st >> 1 : 1u);
                }
            }
            // a wavefront's first chunk takes at least th0, the m_first-th largest lane
            // maximum of that chunk, m_first = 6 or ceil(K / 8) (of one chunk only: the
            // running maxima of several chunks hold more of the row's largest logits, and a
            // bound that high leaves fewer than K logits above the row's bound; a chunk's 6th
            // largest lies above a row's 200th largest logit in a few rows in a hundred).
            // Its rejections put th0 - 1 into the row's rejected bound, so every later chunk
            // of the row may take at least th0 too: a logit below it would only be gathered
            // to be dropped.  th0 enters the shared threshold (the ratchet then climbs from
            // it, each raise still proved by kp published maxima, and needs no seed).
            if (first) {
                th0 = wave_mth(run, wmx, m_first);
                if (lane == 0 && th0 > rt) atomicMax(&rl.rth, th0);
            }
            th = max(rt, th0);
            first = 0;
        } else {
            // this wavefront's statistic, capped by the others' published ones
            uint32_t oth = lane < NW ? lds_ld(&rl.theta[lane]) : 0xFFFFFFFFu;
            oth = min(oth, dpp_move<0xB1, 0xF>(oth));
            oth = min(oth, dpp_move<0x4E, 0xF>(oth));
            oth = min(oth, dpp_move<0x141, 0xF>(oth));
            oth = min(oth, dpp_move<0x140, 0xF>(oth));
            const uint32_t othm = (uint32_t)__builtin_amdgcn_readlane((int)oth, 15);
            // (a wavefront's first chunk, before the others have published: its m0-th
            // largest).  Without halves, later chunks raise the first chunk's statistic as a
            // ratchet (a step up taken when at least m running lane maxima lie strictly
            // above it, doubled on success and halved on failure): every value it takes
            // still has m lane maxima at or above it, without a selection every chunk
            uint32_t thw;
            if (halves && !first) {
                thw = min(h0, h1);
            } else if (first) {
                thw = wave_mth(run, wmx, halves ? 6 : m0);
                thw_r = thw;
            } else {
                const uint32_t c = thw_r + stp_r > thw_r ? thw_r + stp_r : 0xFFFFFFFFu;
                if ((int)__popcll(__ballot(run > c)) >= m) {
                    thw_r = c;
                    stp_r = stp_r < 0x40000000u ? 2u * stp_r : stp_r;
                } else {
                    stp_r = stp_r > 1u ? stp_r >> 1 : 1u;
                }
                thw = thw_r;
            }
            first = 0;
            if (lane == 0) lds_st(&rl.theta[wv], thw);
            th = min(thw, othm);
        }
        if (th <= KEY_NEG_INF) th = KEY_NEG_INF + 1u;
        rej_w = max(rej_w, th - 1u);
        const float thf = key2f(th);
        if (__ballot(tmk >= th)) {
#pragma unroll
            for (int u = 0; u < RU; ++u) {
                if (!__ballot(!(max4(X[u]) < thf))) continue;   // (a NaN: not skipped)
                const int c4 = f0 + u * 64 + lane;
                const float w[4] = {X[u].x, X[u].y, X[u].z, X[u].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const bool hit = w[k] >= thf;
                    const uint64_t mk = __ballot(hit);
                    if (mk == 0ull) continue;
                    const int pos = wn + lane_prefix(mk);
                    if (hit && pos < WCAP) {
                        rl.ckey[wv][pos] = f2key(w[k]);
                        rl.cid[wv][pos] = 4 * c4 + k;
                    }
                    wn += __popcll(mk);
                }
            }
        }
    };
    // whole chunks are taken in increasing order, so a wavefront's first index past them ends
    // its walk; a chunk's buffer is refilled right after the chunk is processed (a load that
    // waits for room in the CU's memory queue then holds up no data that is in).  A partial
    // last chunk is the last wavefront's, before its walk.
    if (nr < nch && wv == NW - 1) chunk(std::true_type{}, T, nr);
    for (;;) {
        if (jA >= nr) break;
        chunk(std::false_type{}, A, jA);
        jA = take();
        load_chunk(A, rs, jA, lane);
        if (jB >= nr) break;
        chunk(std::false_type{}, B, jB);
        jB = take();
        load_chunk(B, rs, jB, lane);
    }
    TL_ROW(3);
    // the segment's record (every lane's sums are against the wavefront's base)
    {
        const double Sw = greedy ? 0.0 : wave_sum_d(accS);
        const double Tw = greedy ? 0.0 : wave_sum_d(accT);
        const uint32_t maxk = wave_max_u(run);
        const uint32_t mnk = wave_min_u(mink);
        const int nanw = __ballot(nan != 0) ? wave_sum_i(nan) : 0;
        if (lane == 0) {
            SegRec r;
            r.sum = Sw;
            r.term = -Tw;
            r.c = cw;
            r.maxk = maxk > KEY_NEG_INF ? maxk : KEY_NEG_INF;
            r.mink = mnk;
            r.nan = nanw;
            r.len = len;
            r.rej = rej_w;
            r.cnt = wn;
            rl.seg[wv] = r;
        }
    }
    lds_barrier();
    TL_ROW(4);
    QS_TL_HOOK(8);
    // every wavefront: the row's max, window threshold, rejected bound and list overflow
    auto umax = [](uint32_t x, uint32_t y) { return x > y ? x : y; };
    const uint32_t rmx = lane16_reduce(lane < NW ? rl.seg[lane].maxk : 0u, umax);
    const float maxl = key2f(rmx > KEY_NEG_INF ? rmx : KEY_NEG_INF);
    const float msc = maxl * inv_t, thr = msc - 30.0f;
    const uint32_t rej_row = lane16_reduce(lane < NW ? rl.seg[lane].rej : 0u, umax);
    const bool cflag = __ballot(lane < NW && rl.seg[lane].cnt > WCAP) != 0ull;
    const bool cert_ok = !greedy && isfinite(msc) && fabsf(msc) < CERT_MSC_MAX && !cflag;
    const int nl = min(rl.seg[wv].cnt, WCAP);
    if (greedy) {
        float bv = -INFINITY;
        int bi = -1;
        for (int i = lane; i < nl; i += 64) best_combine(bv, bi, key2f(rl.ckey[wv][i]), rl.cid[wv][i]);
        wave_best(bv, bi);
        if (lane == 0) {
            rl.gbv[wv] = bv;
            rl.gbi[wv] = bi;
        }
    } else if (wv != NW - 1) {
        // the candidates above the row's bound (below it every list is incomplete and
        // counts as rejected) appended to the gathered arrays with their exact numerators
        // (any order: every decision selects and sorts): each wavefront but the last takes
        // its own list, and the last one's list (that wavefront takes the row's totals) is
        // dealt out to them in slices of 64
        auto gather = [&](int w, int i, int n) {    // entry i of list w, which holds n
            const bool valid = i < n;
            const uint32_t kv = valid ? rl.ckey[w][i] : 0u;
            const bool hit = valid && kv > rej_row;
            const uint64_t mk = __ballot(hit);
            if (mk == 0ull) return;
            const int idv = hit ? rl.cid[w][i] : 0;
            const float e = hit && cert_ok ? cert_e(kv, inv_t, msc, thr, rl.tab) : 0.0f;
            const uint64_t mw = __ballot(e > 0.0f);
            int base = 0;
            if (lane == 0) {
                base = atomicAdd(&rl.gcount, __popcll(mk));
                if (mw) atomicAdd(&rl.gwin, __popcll(mw));
            }
            base = __builtin_amdgcn_readfirstlane(base);
            const int pos = base + lane_prefix(mk);
            if (hit && pos < FCAP) {
                rl.dl.keys[pos] = kv;
                rl.dl.ids[pos] = idv;
                if (pos < WAVE_CAND) rl.gk[pos] = e > 0.0f ? eid_key(e, idv) : 0ull;
            }
        };
        const int own = __builtin_amdgcn_readfirstlane(min(rl.seg[wv].cnt, WCAP));
        const int last = __builtin_amdgcn_readfirstlane(min(rl.seg[NW - 1].cnt, WCAP));
        for (int i0 = 0; i0 < own; i0 += 64) gather(wv, i0 + lane, own);
        for (int i0 = wv * 64; i0 < last; i0 += (NW - 1) * 64) gather(NW - 1, i0 + lane, last);
    }
    QS_TL_HOOK(9);
    if (wv == NW - 2 && lane == 0)                  // the rejected logits' numerator bound
        rl.e_rej = cert_ok && rej_row > KEY_NEG_INF ? cert_e(rej_row, inv_t, msc, thr, rl.tab)
                                                    : 0.0f;
    if (wv == NW - 1) {
        // the row's totals from the segments' records: one certified part (every segment's
        // sums moved exactly to the row's base, the largest), the denominator interval and
        // the window size when every segment lies wholly in or out of the window
        const bool have = lane < NW;
        const SegRec r = rl.seg[have ? lane : 0];
        const float maxw = have ? key2f(r.maxk) : -INFINITY;
        const float cr = lane16_reduce(have ? r.c : C_INIT, [](float x, float y) { return fmaxf(x, y); });
        // the part's scale needs neither sum: every lane computes it while the sums reduce
        const double s_row = cert_scale_c(maxl, cr, inv_t, msc);
        const float d = have ? cr - r.c : 0.0f;
        const int sh = -(int)fminf(d, 4096.0f);
        const double Sx = have ? ldexp(r.sum, sh) : 0.0;
        const double Tx = have ? ldexp(r.term + (double)d * r.sum, sh) : 0.0;
        auto dsum = [](double x, double y) { return x + y; };
        const double S_row = lane16_reduce(Sx, dsum), T_row = lane16_reduce(Tx, dsum);
        const bool out_j = !(maxw * inv_t >= thr);
        const bool in_j = have && r.mink != 0xFFFFFFFFu && key2f(r.mink) * inv_t >= thr;
        const bool known = __ballot(have && !out_j && !in_j) == 0ull;
        const int nin = lane16_reduce(have && !out_j && in_j ? r.len - r.nan : 0,
                                      [](int x, int y) { return x + y; });
        if (lane == 0) {
            CertTotals t;
            t.maxl = maxl;
            t.msc = msc;
            double S_lo = 1.0, S_hi = 1.0;
            if (!greedy) {
                const CertPart cp = cert_part_cs(maxl, cr, S_row, T_row, inv_t, msc, thr, s_row);
                cert_interval(cp.lo, cp.hi, msc, thr, V, S_lo, S_hi);
            }
            t.S_lo = S_lo;
            t.S_hi = S_hi;
            t.v_lo = (float)(1.0 / S_hi);
            t.v_hi = (float)(1.0 / S_lo);
            t.nwin = known ? nin : -1;
            t.cflag = cflag;
            t.rej = rej_row;
            t.total = 0;
            rl.ct = t;
        }
    }
    QS_TL_HOOK(10);
    lds_barrier();
    QS_TL_HOOK(11);
    // rows with top K at most 64: the gathered candidates in the window ranked in (e desc,
    // id asc) order by counting, G threads per candidate, the first 64 placed by rank
    const int total = rl.gcount, nwin_c = rl.gwin;
    const bool rank = cert_ok && total >= 1 && total <= WAVE_CAND && row_ksel(P) <= 64;
#ifdef QS_TIMELINE
    if (tid == 0 && row < 4096) {
        qs::g_tl_hook[row * 16 + 5] = (uint64_t)total;
        qs::g_tl_hook[row * 16 + 7] = (uint64_t)nwin_c;
    }
#endif
    const bool small = rank && total <= 64;         // sorted by one wavefront instead
    if (rank && !small) {
        int np = 64;
        while (np < total) np <<= 1;
        const int G = min(16, NW * 64 / np);            // a power of two, lanes of one row
        const int c = tid / G, g = tid - c * G;
        const uint64_t kc = c < total ? rl.gk[c] : 0ull;
        int cnt = 0;
        if (kc != 0ull) {
            int q = g;
            for (; q + 3 * G < total; q += 4 * G) {
                const uint64_t k0 = rl.gk[q], k1 = rl.gk[q + G], k2 = rl.gk[q + 2 * G],
                               k3 = rl.gk[q + 3 * G];
                cnt += (k0 > kc) + (k1 > kc) + (k2 > kc) + (k3 > kc);
            }
            for (; q < total; q += G) cnt += rl.gk[q] > kc;
        }
        QS_TL_HOOK(6);
        // the G lanes of a candidate (consecutive, G a power of two up to 16) add up
        if (G > 1) cnt += dpp_move<0xB1, 0xF>(cnt);     // lane ^ 1
        if (G > 2) cnt += dpp_move<0x4E, 0xF>(cnt);     // lane ^ 2: quads
        if (G > 4) cnt += dpp_move<0x141, 0xF>(cnt);    // half-row mirror: eights
        if (G > 8) cnt += dpp_move<0x140, 0xF>(cnt);    // row mirror: sixteens
        if (g == 0 && kc != 0ull) {
            if (cnt < 64) rl.dl.srt[cnt] = kc;
            else if (cnt == 64) rl.e64 = key_p(kc);
        }
    }
    if (tid < QS_EXPF_TAB_N) rl.dl.dl.tab[tid] = tabv;
    lds_barrier();
    TL_ROW(5);
    // the decision: the first ND threads (the other wavefronts end here; a barrier waits only
    // for the wavefronts still running)
    if (tid >= ND) return;
    DecLds &dl = rl.dl;
    if (greedy) {
        float bv = -INFINITY;
        int bi = -1;
        for (int v = 0; v < NW; ++v) best_combine(bv, bi, rl.gbv[v], rl.gbi[v]);
        if (cflag) {                              // a list overflowed: scan the row
            bv = -INFINITY;
            bi = -1;
            row_visit(a, row, P, dl, [&](float w, int id) {
                if (w == w) best_combine(bv, bi, w, id);
            });
            block_best(bv, bi, dl);
        }
        if (tid == 0) record_greedy(row, P, bv, bi, maxl, x0, a.st, a.out, a.diag);
        return;
    }
    CertTotals t = rl.ct;
    t.total = total;
    int status = isfinite(msc) ? CF_MSC : CF_INPUT;
    if (rank) {
        if (tid < 64) {
            const int m = min(nwin_c, 64);
            uint64_t ek;
            if (small) {
                ek = lane < total ? rl.gk[lane] : 0ull;
                ek = wave_sort_desc(ek);
            } else {
                ek = lane < m ? dl.srt[lane] : 0ull;
            }
            float e_rej = rl.e_rej;
            if (nwin_c > 64) e_rej = fmaxf(e_rej, rl.e64);
            const int s2 = cert_finish_wave(row, P, t, ek, e_rej, a.st, a.out, a.diag, hist);
            if (tid == 0) dl.dl.sh[7] = s2;
        }
        __syncthreads();
        status = dl.dl.sh[7];
        __syncthreads();
        TL_ROW(6);
    } else if (cert_ok && total >= 1 && total <= FCAP) {
        status = cert_row_block<ND>(row, P, t, dl.keys, dl.ids, dl.srt, dl.dl, a.st, a.out,
                                    a.diag, hist);
    } else if (cflag || total > FCAP) {
        status = CF_INPUT;
    }
    if (status == 0) return;
    // hist was loaded by wavefront 0 only; the exact path's decision reads it there
    exact_row(a, row, P, t, dl, hist, status);
}

// The row pick's loads alone, for the read ceiling its streaming is measured against: the
// row kernel's launch shape at one row per CU (one workgroup of 16 wavefronts per row), its
// chunks, load instruction and order (two chunks in flight a wavefront, the next taken from
// the row's LDS counter, the partial last chunk by the last wavefront), each lane's floats
// added up and nothing else.  sink[row] is written only for a sum no row of finite logits
// reaches, so the loads stay and the kernel writes nothing.
__global__ void __launch_bounds__(1024) k_row_read(const float *logits, int64_t stride,
                                                    int vocab, float *sink) {
    constexpr int NW = 16;
    __shared__ int next;
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n4 = vocab >> 2, nch = (n4 + RCH - 1) / RCH, nr = n4 / RCH;
    const float *rowp = logits + (int64_t)row * stride;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)rowp, 0, n4 * 16, BUF_WORD3);
    float4 A[RU], B[RU], T[RU];
    int jA = wv, jB = NW + wv;
    if (nr < nch && wv == NW - 1) load_chunk(T, rs, nr, lane);
    load_chunk(A, rs, jA, lane);
    load_chunk(B, rs, jB, lane);
    if (tid == 0) next = 2 * NW;
    lds_barrier();
    float s = 0.0f;
    auto add = [&](float4 (&X)[RU]) {
#pragma unroll
        for (int u = 0; u < RU; ++u) s += (X[u].x + X[u].y) + (X[u].z + X[u].w);
    };
    auto take = [&]() {
        int j = 0;
        if (lane == 0) j = atomicAdd(&next, 1);
        return __builtin_amdgcn_readfirstlane(j);
    };
    if (nr < nch && wv == NW - 1) add(T);             // (past the row the loads read 0)
    for (;;) {
        if (jA >= nr) break;
        add(A);
        jA = take();
        load_chunk(A, rs, jA, lane);
        if (jB >= nr) break;
        add(B);
        jB = take();
        load_chunk(B, rs, jB, lane);
    }
    if (s == -0x1.234p120f) sink[row] = s;
}

}  // namespace

int qs_time_row_reads(const float *const *d_logits, int n_buffers, int64_t row_stride,
                      int n_rows, int n_vocab, float *d_sink, int iters, float *ms) {
    if (!d_logits || n_buffers < 1 || !d_sink || iters < 1 || !ms || n_rows < 1 ||
        row_stride < n_vocab) {
        qs_set_error("qs_time_row_reads: bad arguments");
        return QS_EINVAL;
    }
    for (int i = 0; i < n_buffers; ++i)
        if (!d_logits[i] || !qs_row_supported(n_rows, n_vocab, row_stride, d_logits[i])) {
            qs_set_error("qs_time_row_reads: buffer %d is not a row kernel input", i);
            return QS_EINVAL;
        }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = 0;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) rc = QS_EDEVICE;
    if (!rc && hipEventRecord(e0, 0) != hipSuccess) rc = QS_EDEVICE;
    for (int i = 0; i < iters && !rc; ++i) {
        hipLaunchKernelGGL(k_row_read, dim3((unsigned)n_rows), dim3(1024), 0, 0,
                           d_logits[i % n_buffers], row_stride, n_vocab, d_sink);
        if (hipGetLastError() != hipSuccess) rc = QS_EDEVICE;
    }
    if (!rc && (hipEventRecord(e1, 0) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                hipEventElapsedTime(ms, e0, e1) != hipSuccess))
        rc = QS_EDEVICE;
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (rc) qs_set_error("qs_time_row_reads: device error");
    return rc;
}

int qs_row_resident(int waves) {
    int nb = 0;
    const hipError_t e =
        waves == 16 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_row<16>, 1024, 0)
                    : hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_row<8>, 512, 0);
    return e == hipSuccess ? nb : 0;
}

int qs_row_timeline_read(uint64_t *dst, int n) {
#ifdef QS_TIMELINE
    // rows x wavefronts x 8 phase stamps, then rows x 16 decision steps
    constexpr size_t n0 = sizeof(g_tl_row) / 8, n1 = sizeof(qs::g_tl_hook) / 8;
    if (!dst || n < 0 || (size_t)n > n0 + n1) return QS_EINVAL;
    if (hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_tl_row), 8 * std::min((size_t)n, n0)) != hipSuccess)
        return QS_EDEVICE;
    if ((size_t)n > n0 &&
        hipMemcpyFromSymbol(dst + n0, HIP_SYMBOL(qs::g_tl_hook), 8 * ((size_t)n - n0)) != hipSuccess)
        return QS_EDEVICE;
    return 0;
#else
    (void)dst;
    (void)n;
    return QS_EINVAL;
#endif
}

int qs_row_supported(int n_rows, int n_vocab, int64_t row_stride, const void *logits) {
    return n_rows >= 1 && n_vocab >= 4 && n_vocab % 4 == 0 && n_vocab <= ROW_VMAX &&
           row_stride % 4 == 0 && ((uintptr_t)logits % 16) == 0;
}

int qs_row_launch(const float *logits, int64_t row_stride, int n_rows, int n_vocab,
                  const RowState &st, const Scratch &sc, int32_t *out, qs_pick_diag *diag,
                  int waves, hipStream_t stream) {
    PartArgs a;
    a.logits = logits;
    a.stride = row_stride;
    a.vocab = n_vocab;
    a.n_rows = n_rows;
    a.parts = 1;
    a.part_len = n_vocab;
    a.xcd_map = 0;
    a.st = st;
    a.sc = sc;
    a.out = out;
    a.diag = diag;
    if (waves == 16)
        hipLaunchKernelGGL(k_row<16>, dim3((unsigned)n_rows), dim3(1024), 0, stream, a);
    else
        hipLaunchKernelGGL(k_row<8>, dim3((unsigned)n_rows), dim3(512), 0, stream, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        qs_set_error("row pick launch: %s", hipGetErrorString(e));
        return e == hipErrorOutOfMemory ? QS_ENOMEM : QS_EDEVICE;
    }
    return 0;
}
