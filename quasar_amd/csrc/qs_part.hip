// qs_part.hip - the streaming pick: one workgroup per part of a row, every logit read once,
// then one workgroup per row for the decision.
//
// A pick of B rows of V logits (sample.c:111-179 per row) is two kernels:
//
// k_part, B x P workgroups of 512 threads, P = ceil(V / 10240) parts per row (15 at
// V = 151,936).  A workgroup holds its part in registers (five float4 per thread, the
// 16-byte loads issued at once) and never waits for another workgroup:
//   1. the repeat penalty from an LDS bitmap of the row's history (sample.c:118-128),
//      each thread's max and min (NaN-propagating), greedy rows: the first argmax;
//   2. the part's max M and (wavefront 0) the candidate threshold, the kw-th largest
//      thread maximum, so the part's top kw logits are kept;
//   3. sampling rows: per logit sc = w * inv_t, t = fl(sc * L - c), e = 2^t (v_exp_f32),
//      summed in float quads then binary64, and e * t summed in float: with M these bound
//      the part's share of the reference's softmax denominator (qs_cert.h);
//   4. the logits at or above the threshold as (key, id) candidates, stored with the
//      part's sums.
// When every row is greedy, k_part alone: each part joins its first argmax into the row's
// by device-wide atomic maxima, and the row's last part records it (greedy_part_done).
// k_decide, B workgroups of 256 threads: the row's denominator interval, the candidates'
// exact numerators (the host-libm-equal expf) and the cuts and draw proved for every
// normaliser of the interval (cert_row_wave / cert_row_block).  A row the proof does not
// cover (a cut on the edge of the interval, neighbours that may swap, a large nucleus,
// non-finite or huge maxima) has its exact denominator recomputed from the logits and goes
// through the exact decision (decide_row_fast, with its whole-window fallback, whose
// scratch-slot lock is the only wait: its holders are running workgroups).

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>

#include "../../include/quasar_sampler.h"
#include "qs_cert.h"
#include "qs_decide.h"
#include "qs_device.h"
#include "qs_launch.h"

using namespace qs;
using namespace qs::dec;

namespace {

constexpr int NT = 512;              // threads per streaming workgroup
constexpr int NWV = NT / 64;         // its wavefronts
constexpr int UP = 5;                // float4 per thread per part
constexpr int STAGES = 1;            // parts whose loads are in flight during one part
constexpr int PART_MAX = NT * UP * 4;    // longest part (elements)
constexpr int WCAP = 32;             // candidates per wavefront list
constexpr int PCAP = NWV * WCAP;     // candidates per part
static_assert(NWV == QS_PART_WAVES && PCAP == QS_PART_CANDS, "scratch layout");
constexpr int RING_W = NT;           // ring slots the workgroup loads at once (one per thread)


__constant__ uint64_t c_tab_part[QS_EXPF_TAB_N] = QS_EXPF_TABLE_INIT;

// The timeline build (make timeline: -DQS_TIMELINE) records the 100 MHz clock at the phase
// boundaries of each streaming wavefront's first TL_STEPS parts (workgroups below TL_WG),
// for quasar_amd/timeline.py; the decision's clocks are QS_DEC_MARK (qs_decide.h).
#ifdef QS_TIMELINE
constexpr int TL_WG = 1024, TL_STEPS = 8;
__device__ uint64_t g_tl_part[TL_WG * TL_STEPS * QS_PART_WAVES * 8];
#define TL_PART(k, e)                                                                         \
    do {                                                                                      \
        if ((tix() & 63) == 0 && blockIdx.x < TL_WG && (k) < TL_STEPS)                        \
            g_tl_part[((blockIdx.x * TL_STEPS + (k)) * QS_PART_WAVES + (tix() >> 6)) * 8 + (e)] = \
                __builtin_amdgcn_s_memrealtime();                                             \
    } while (0)
#else
#define TL_PART(k, e) ((void)(k))
#endif


// What the streaming kernel reads and writes (kept small: it stays in scalar registers
// across the workgroup's loop over its parts).
// tix() behind an opaque copy: values derived from it are recomputed where they are
// used instead of being held in registers across the streaming loop (which would cost the
// kernel its third resident workgroup per CU).
__device__ __forceinline__ int tix() {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

struct StreamArgs {
    const float *logits;
    int64_t stride;
    int vocab, n_rows, parts, part_len, xcd_map, ring_stride;
    const qs_row_param *prm;
    const int32_t *ring, *hlen, *hhead;
    WaveRec *rec;
    uint2 *cand;
    // greedy rows decided by their last part (gbest null: by k_decide), and what that
    // decision writes: the rows' rings, lengths and heads, ids and diagnostics
    uint64_t *gbest;
    uint32_t *gmaxk, *gcnt;
    int32_t *ring_w, *hlen_w, *hhead_w, *out;
    qs_pick_diag *diag;
};

constexpr int PART_BM = bitmap_words(PART_MAX);

struct PartLds {
    uint32_t bm[3][PART_BM];         // history bitmaps: part i uses slot i mod 3
    uint32_t hitw[3][NWV];           // bit u: the wavefront's float4s u hold history ids
    uint32_t wmax[2][NWV];           // per-wave max key, by part parity
    uint32_t wth[2][NWV];            // per-wave threshold key (0xFFFFFFFF: not counted)
    uint32_t lmax[NT];               // a short part's thread maxima (keys)
    uint32_t theta;                  // a short part's threshold key
    WaveRec rec[NWV];                // each wavefront's record of the last part, and
    uint2 cand[NWV][WCAP];           // its candidates, stored out during the next part
    uint64_t gbw[2][NWV];            // greedy rows: per-wave (key, ~id) best, by parity
};

struct Loc {                          // a part of a row
    int row, part, lo, hi, c_lo, c_hi;
};
__device__ __forceinline__ Loc part_loc(int part_len, int vocab, int row, int part) {
    Loc l;
    l.row = row;
    l.part = part;
    l.lo = part * part_len;
    l.hi = min(l.lo + part_len, vocab);
    l.c_lo = l.lo >> 2;
    l.c_hi = l.hi >> 2;
    return l;
}

// The parts of the pick are dealt to the grid's workgroups in contiguous runs.  With
// rows >= 8 the dispatcher's round-robin over the 8 XCDs is followed: workgroup w runs on
// XCD w mod 8, so it takes parts of the rows r = w (mod 8) only (a row's parts, its history
// ring and its results stay in one L2).
struct Run {
    int begin, end;                  // part indexes of this workgroup
    int xcd;                         // rows xcd, xcd + 8, ... (xcd_map) or all rows (-1)
};
__device__ __forceinline__ Run my_run(const StreamArgs &a) {
    const int G = gridDim.x, w = blockIdx.x;
    Run r;
    if (a.xcd_map) {
        const int x = w & 7, S = G >> 3, sl = w >> 3;
        const int rows_x = (a.n_rows - x + 7) >> 3;
        const int64_t n = (int64_t)rows_x * a.parts;
        r.begin = (int)(n * sl / S);
        r.end = (int)(n * (sl + 1) / S);
        r.xcd = x;
    } else {
        const int64_t n = (int64_t)a.n_rows * a.parts;
        r.begin = (int)(n * w / G);
        r.end = (int)(n * (w + 1) / G);
        r.xcd = -1;
    }
    return r;
}
__device__ __forceinline__ Loc part_at(const StreamArgs &a, const Run &r, int idx) {
    const int q = idx / a.parts, j = idx - q * a.parts;
    return part_loc(a.part_len, a.vocab, r.xcd >= 0 ? q * 8 + r.xcd : q, j);
}
// The part after l in a run (no division).
__device__ __forceinline__ Loc loc_next(const StreamArgs &a, const Run &r, const Loc &l) {
    return l.part + 1 < a.parts ? part_loc(a.part_len, a.vocab, l.row, l.part + 1)
                                : part_loc(a.part_len, a.vocab, l.row + (r.xcd >= 0 ? 8 : 1), 0);
}

// The part's logits into the LDS staging buffer: a buffer resource over its float4s; float4
// u of thread tid (byte offset (u*NT + tid)*16 in the part) lands at stage[u*NT + tid]
// (the direct-to-LDS form writes a wavefront's 64 lanes to 64 consecutive float4s), so each
// thread later reads back exactly what it loaded.  Loads past the part read no memory.
constexpr int BUF_WORD3 = 0x00020000;    // raw buffer, 32-bit data format
constexpr int BUF_NT = 2;                // nontemporal: each logit is read once
typedef __attribute__((address_space(3))) void lds_void;
__device__ __forceinline__ void issue_stage(float4 *stage, const StreamArgs &a, const Loc &l) {
    const float *base = a.logits + (int64_t)l.row * a.stride + 4 * (int64_t)l.c_lo;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)base, 0, (l.c_hi - l.c_lo) * 16, BUF_WORD3);
    const int tid = tix();
    float4 *dst = stage + (tid & ~63);
#pragma unroll
    for (int u = 0; u < UP; ++u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void *)(dst + u * NT), 16, tid * 16,
                                                 u * NT * 16, 0, BUF_NT);
}

// One float4 of LDS read by an instruction the compiler does not track: its own waits would
// hold a staging buffer read until every staging load in flight lands, where the kernel
// waits for exactly the loads it reads (by count).
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 lds_read4(const float4 *p) {
    const uint32_t off = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const float4 *)p;
    f32x4 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(off) : "memory");
    return make_float4(v.x, v.y, v.z, v.w);
}

// Ring slot `tid` of a row (0 past the ring's storage, without a memory access): each
// thread holds one, so a workgroup covers RING_W slots with one load each.
__device__ __forceinline__ int ring_slot(const StreamArgs &a, int row) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a.ring + (int64_t)row * a.ring_stride), 0, a.ring_stride * 4, BUF_WORD3);
    return (int)__builtin_amdgcn_raw_buffer_load_b32(rs, tix() * 4, 0, 0);
}

// An LDS atomic OR issued as an instruction the compiler does not track: its own waits
// treat any LDS write as possibly overlapping the staging loads in flight and would hold it
// until they land.  It completes before the next LDS barrier (which waits for all of this
// wavefront's LDS operations); nothing reads the word before that barrier.
__device__ __forceinline__ void lds_or(uint32_t *p, uint32_t v) {
    const uint32_t off = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t *)p;
    asm volatile("ds_or_b32 %0, %1" ::"v"(off), "v"(v) : "memory");
}

// All threads: mark the history ids of [l.lo, l.hi) in a zeroed bitmap and its hit masks.
// `slot` is this thread's ring slot of the row (slots RING_W and up are read directly: rings
// longer than the workgroup).  A ring slot p holds a history id iff p < cap and
// (p - head) mod cap < len (sample.c:118: duplicates set the same bit, so each id is
// penalised once).
__device__ __forceinline__ void bitmap_mark(uint32_t *bm, uint32_t *hitw, const StreamArgs &a,
                                            const Loc &l, int slot, int cap) {
    int len = a.hlen[l.row], head = a.hhead[l.row];
    qs_ring_clamp(cap, &len, &head);
    auto mark = [&](int p, int id) {
        if (qs_ring_live(cap, len, head, p) && id >= l.lo && id < l.hi) {
            const int q = id - l.lo, c = q >> 2, u = c / NT;   // float4 c: thread c - u*NT
            lds_or(&bm[q >> 5], 1u << (q & 31));
            lds_or(&hitw[(c - u * NT) >> 6], 1u << u);
        }
    };
    mark(tix(), slot);
    for (int p = RING_W + tix(); p < cap; p += NT)
        mark(p, a.ring[(int64_t)l.row * a.ring_stride + p]);
}
// A workgroup barrier over LDS traffic only.  __syncthreads() also orders global memory,
// which on this chip waits for every load in flight, the staging buffer's included; the
// streaming kernel shares nothing but LDS between its wavefronts, so it waits for its own
// LDS operations and meets the others (the memory clobber keeps the compiler from moving
// LDS accesses across it).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// A row's parameters with its ring capacity clamped to the ring's storage (qs_ring_cap).
__device__ __forceinline__ qs_row_param stream_param(const StreamArgs &a, int row) {
    qs_row_param P = a.prm[row];
    P.ring_cap = qs_ring_cap(P.ring_cap, a.ring, a.ring_stride);
    return P;
}
// The ring capacity whose ids a row's bitmap marks: none without a penalty (sample.c:119).
__device__ __forceinline__ int mark_cap(const StreamArgs &a, int row) {
    const qs_row_param P = stream_param(a, row);
    return P.repeat_penalty > 1.0f ? P.ring_cap : 0;
}
// All threads: zero a bitmap slot and its hit masks.
__device__ __forceinline__ void bitmap_zero(uint32_t *bm, uint32_t *hitw) {
    static_assert(PART_BM / 4 <= NT, "one store per thread");
    uint4 *b4 = (uint4 *)bm;
    if (tix() < PART_BM / 4) b4[tix()] = make_uint4(0u, 0u, 0u, 0u);
    if (tix() < NWV) hitw[tix()] = 0u;
}

// Whether float4 group u of wavefront wv reaches past the part (a uniform test).
__device__ __forceinline__ bool wave_tail(const Loc &l, int u, int wv) {
    return l.c_lo + u * NT + wv * 64 + 63 >= l.c_hi;
}

// Pass 1: penalty, each thread's max and min over non-NaN logits, its NaN count.  Positions
// past the part become -inf in the registers; NaNs stay (no >= test passes them and the
// sums of a wavefront holding one floor t, which sends e to 0).
struct Pass1 {
    float mx, mn;                    // max / min over the thread's logits (min: non-NaN)
    int nan;                         // NaNs among them
};
template <bool TAIL>
__device__ __forceinline__ Pass1 pass1(float4 (&buf)[UP], const Loc &l, const uint32_t *bm,
                                       const uint32_t *hitw, bool pen, float rp, int wv) {
    const int tid = tix();
    const uint32_t *bw = bm + (tid >> 3);             // word (u*NT + tid)/8, NT % 8 == 0
    const uint32_t bsh = (uint32_t)(tid & 7) * 4u;
    const uint32_t hm = pen ? (uint32_t)__builtin_amdgcn_readfirstlane((int)hitw[wv]) : 0u;
    Pass1 r{-INFINITY, INFINITY, 0};
#pragma unroll
    for (int u = 0; u < UP; ++u) {
        float w[4] = {buf[u].x, buf[u].y, buf[u].z, buf[u].w};
        if ((hm >> u) & 1u) {                        // positions past the part are unmarked
            const uint32_t nib = __builtin_amdgcn_ubfe(bw[u * (NT / 8)], bsh, 4);
            if (__ballot(nib != 0u)) {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if ((nib >> k) & 1u) w[k] = penalise(w[k], rp);
            }
        }
        if (TAIL && wave_tail(l, u, wv)) {           // a scalar branch: tail waves only
            if (l.c_lo + u * NT + tid >= l.c_hi) w[0] = w[1] = w[2] = w[3] = -INFINITY;
            else r.mn = min3n(min3n(r.mn, w[0], w[1]), w[2], w[3]);
        } else {
            r.mn = min3n(min3n(r.mn, w[0], w[1]), w[2], w[3]);
        }
        r.mx = max3n(max3n(r.mx, w[0], w[1]), w[2], w[3]);
        buf[u] = make_float4(w[0], w[1], w[2], w[3]);
    }
    if (__ballot(r.mx != r.mx || r.mn != r.mn)) {   // a NaN in the wavefront: not a max,
        r.mx = -INFINITY;                             // not in the min, counted (a NaN
        r.mn = INFINITY;                              // never passes a >= test, and the
#pragma unroll                                        // sums' t floor drops it)
        for (int u = 0; u < UP; ++u) {
            const bool tail = TAIL && l.c_lo + u * NT + tid >= l.c_hi;
            const float w[4] = {buf[u].x, buf[u].y, buf[u].z, buf[u].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                r.nan += w[k] != w[k];
                r.mx = w[k] > r.mx ? w[k] : r.mx;
                r.mn = (w[k] < r.mn && !tail) ? w[k] : r.mn;
            }
        }
    }
    return r;
}

// A greedy row's part is done (one thread): its best (key, ~id) and max key join the
// row's by device-wide atomic maxima, each performed before the part is counted; the part
// that counts last reads the row's best and records it (sample.c:130-134) and resets the
// three for the next pick.  No part waits for another.
__device__ __forceinline__ void greedy_part_done(const StreamArgs &a, int row, const qs_row_param &P,
                                              uint32_t pmk, const uint64_t *gbw) {
    uint64_t pb = 0ull;
    for (int j = 0; j < NWV; ++j) pb = gbw[j] > pb ? gbw[j] : pb;
    const uint64_t ob = atomicMax((unsigned long long *)&a.gbest[row], (unsigned long long)pb);
    const uint32_t om = atomicMax(&a.gmaxk[row], pmk);
    asm volatile("s_waitcnt vmcnt(0)" ::"v"(ob), "v"(om) : "memory");   // both performed
    if (atomicAdd(&a.gcnt[row], 1u) != (uint32_t)a.parts - 1u) return;
    const uint64_t best = atomicExch((unsigned long long *)&a.gbest[row], 0ull);
    const uint32_t mk = atomicExch(&a.gmaxk[row], 0u);
    atomicExch(&a.gcnt[row], 0u);
    const int bi = best != 0ull ? (int)~(uint32_t)best : -1;
    const float bv = best != 0ull ? key2f((uint32_t)(best >> 32)) : -INFINITY;
    const RowState st{a.prm, nullptr, a.ring_w, a.hlen_w, a.hhead_w, a.ring_stride};
    record_greedy(row, P, bv, bi, key2f(mk > KEY_NEG_INF ? mk : KEY_NEG_INF),
                  a.logits[(int64_t)row * a.stride], st, a.out, a.diag);
}

// The candidate rule.  Wavefront w of a part offers th_w, the m-th largest of its 64 lane
// maxima (so at least m of its logits reach th_w); the part keeps every logit at or above
// min_w th_w, at least NWV*m logits and in practice about twice that.  m follows the part's
// share of the row's top K (greedy rows only need the part's maxima); the decision proves
// whatever it gets.  A row's short last part uses the kw-th largest thread maximum instead.
__device__ __forceinline__ int part_m(const qs_row_param &P, int parts) {
    if (row_greedy(P)) return 1;
    const int kw = 2 * ((row_ksel(P) + parts - 1) / parts) + 8;
    const int m = (kw + 2 * NWV - 1) / (2 * NWV);    // the minimum over NWV offers keeps
                                                       // about twice NWV*m
    return m < 64 ? m : 64;
}
// One part, all threads: pass 1, the wavefront's statistics into LDS, the part's one
// barrier, then `mid` (the caller's bitmap upkeep), the part's max and threshold, the sums
// (sampling rows), the candidates and the wavefront's record.  Nothing here waits for
// another wavefront after the barrier.
template <bool GF, typename Mid>
__device__ __forceinline__ void part_step(float4 (&buf)[UP], const StreamArgs &a, const Loc &l,
                                          const qs_row_param &P, const uint32_t *bm,
                                          const uint32_t *hitw, int par, PartLds &pl, Mid &&mid,
                                          int tl) {
    const int tid = tix(), lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const float rp = P.repeat_penalty;
    const bool pen = rp > 1.0f && P.ring_cap > 0;
    // only a row's last part can be short of the float4 rows its threads cover (a part is
    // NT*UP float4 long): its positions past the row hold -inf after pass 1, and the sums
    // of the wavefronts with such positions floor t
    TL_PART(tl, 1);
    const bool tailp = l.c_hi - l.c_lo < NT * UP;
    const Pass1 r = tailp ? pass1<true>(buf, l, bm, hitw, pen, rp, wv)
                          : pass1<false>(buf, l, bm, hitw, pen, rp, wv);
    const float inv_t = P.inv_t;
    const bool greedy = row_greedy(P);
    const bool dirty = (tailp && wave_tail(l, UP - 1, wv)) ||
                       __ballot(!(r.mn * inv_t >= SC_SANE) || r.nan != 0) != 0ull;
    const uint32_t tmk = f2key(r.mx);
    const uint32_t wmx = wave_max_u(tmk);
    if (tailp) {
        pl.lmax[tid] = tmk;
        if (lane == 0) pl.wmax[par][wv] = wmx;
    } else {
        const uint32_t th = wave_mth(tmk, wmx, part_m(P, a.parts));
        if (lane == 0) {
            pl.wmax[par][wv] = wmx;
            pl.wth[par][wv] = th;
        }
    }
    const uint32_t wmn = wave_min_u(r.mn == INFINITY ? 0xFFFFFFFFu : f2key(r.mn));
    const int wnan = __ballot(r.nan != 0) ? wave_sum_i(r.nan) : 0;
    const bool gfuse = GF && greedy;               // (GF: every row of the pick is greedy)
    if (gfuse) {
        // sample.c:130-132 over this wavefront's share: the largest penalised logit, the
        // first id among equals (NaNs never; -0 equals +0, so both take +0's key), as the
        // largest (key, ~id)
        uint64_t g = 0ull;
#pragma unroll
        for (int u = 0; u < UP; ++u) {
            const int c = l.c_lo + u * NT + tid;
            const float w[4] = {buf[u].x, buf[u].y, buf[u].z, buf[u].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t wk = f2key(w[k] == 0.0f ? 0.0f : w[k]);
                const uint64_t gk = ((uint64_t)wk << 32) | (uint32_t)~(uint32_t)(4 * c + k);
                if (c < l.c_hi && w[k] == w[k] && gk > g) g = gk;
            }
        }
        g = wave_reduce(g, [](uint64_t x, uint64_t y) { return x > y ? x : y; });
        if (lane == 0) pl.gbw[par][wv] = g;
    }
    TL_PART(tl, 2);
    lds_barrier();
    TL_PART(tl, 3);
    mid();
    TL_PART(tl, 4);
    // the part's max and threshold (every lane reads the NWV entries; never -inf)
    uint32_t pmk = 0u, th = 0xFFFFFFFFu;
#pragma unroll
    for (int j = 0; j < NWV; ++j) pmk = max(pmk, pl.wmax[par][j]);
    if (!tailp) {
#pragma unroll
        for (int j = 0; j < NWV; ++j) th = min(th, pl.wth[par][j]);
    } else {
        // a row's short last part (its wavefronts hold unequal shares): wavefront 0 takes
        // the kw-th largest thread maximum, so at least kw logits of the part reach it
        if (wv == 0) {
            const int kw = min(2 * NWV * part_m(P, a.parts), NT);   // what the rule
                                                                  // above keeps
            uint32_t k[NWV];
#pragma unroll
            for (int j = 0; j < NWV; ++j) k[j] = pl.lmax[j * 64 + lane];
            const uint32_t t = wave_kth(k, kw, NT);
            if (lane == 0) pl.theta = t;
        }
        lds_barrier();
        th = pl.theta;
    }
    if (th <= KEY_NEG_INF) th = KEY_NEG_INF + 1u;
    if (gfuse && tid == 0) greedy_part_done(a, l.row, P, pmk, pl.gbw[par]);
    const float M = key2f(pmk) * inv_t;
    // the sums: approximate numerators and e * t, float4 by float4
    double S = 0.0;
    float Tn = 0.0f;
    if (!greedy && isfinite(M)) {
        const float c = cert_c(M);
        if (dirty) {
#pragma unroll
            for (int u = 0; u < UP; ++u) sum4<true>(buf[u], inv_t, c, S, Tn);
        } else {
#pragma unroll
            for (int u = 0; u < UP; ++u) sum4<false>(buf[u], inv_t, c, S, Tn);
        }
    }
    TL_PART(tl, 5);
    // the candidates: every logit at or above the threshold, by ballot prefix into this
    // wavefront's LDS list (stored out, with the record, during the next part: stores
    // issued after the staging loads would hold up the wait for them)
    const float thf = key2f(th);
    int wn = 0;
    if (__ballot(tmk >= th)) {
        uint2 *lc = pl.cand[wv];
#pragma unroll
        for (int u = 0; u < UP; ++u) {
            if (!__ballot(!(max4(buf[u]) < thf))) continue;   // (a NaN: not skipped)
            const int c = l.c_lo + u * NT + tid;
            const float w[4] = {buf[u].x, buf[u].y, buf[u].z, buf[u].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const bool hit = w[k] >= thf;
                const uint64_t m = __ballot(hit);
                if (m == 0ull) continue;
                const int pos = wn + lane_prefix(m);
                if (hit && pos < WCAP) lc[pos] = make_uint2(f2key(w[k]), (uint32_t)(4 * c + k));
                wn += __popcll(m);
            }
        }
    }
    const double ws = wave_sum_d(S);
    const float wt = wave_reduce(Tn, [](float x, float y) { return x + y; });
    if (lane == 0) {
        WaveRec rec;
        rec.sum = ws;
        rec.term = -wt;
        rec.mink = wmn;
        rec.nan = wnan;
        rec.maxk = pmk;
        rec.rej = th - 1u;
        rec.cnt = wn;
        pl.rec[wv] = rec;
    }
    TL_PART(tl, 6);
}

// Store out a wavefront's record and candidates of part li (what part_step left in LDS).
__device__ __forceinline__ void flush_part(const StreamArgs &a, PartLds &pl, int li) {
    const int tid = tix(), lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t at = (int64_t)li * NWV + wv;
    const int n = min(pl.rec[wv].cnt, WCAP);
    if (lane < n) a.cand[at * WCAP + lane] = pl.cand[wv][lane];
    if (lane == 0) a.rec[at] = pl.rec[wv];
}

// The streaming kernel: a persistent grid (about as many workgroups as are resident), each
// walking its run of parts with the next two parts' loads in flight (straight into LDS)
// while it processes the current one (read out of LDS into registers).  Part i's history bitmap sits in slot i mod 3: it is
// marked two parts ahead, after part i-2's barrier (the ring slots of its row are loaded
// ahead of the logit loads issued with them), and its slot is cleared after part i's
// barrier, so one barrier per part orders every bitmap access.
//
// The pointers come as separate restrict arguments: with them the row parameters, history
// lengths and heads (uniform addresses) are scalar loads, which the wavefront waits for
// without waiting for the logit loads in flight.  They are written only by a greedy row's
// last part (GF), through other pointers, once every part of the row has read them.
template <bool GF>
__global__ void __launch_bounds__(NT, 6)
k_part(StreamArgs sa, const float *__restrict__ logits, const qs_row_param *__restrict__ prm,
       const int32_t *__restrict__ ring, const int32_t *__restrict__ hlen,
       const int32_t *__restrict__ hhead, WaveRec *__restrict__ rec, uint2 *__restrict__ cand) {
    __shared__ float4 stage0[UP * NT];                // the next STAGES parts' logits, in
    __shared__ float4 stage1[STAGES > 1 ? UP * NT : 1];  // flight (part i: stage i mod 2)
    __shared__ PartLds pl;
    StreamArgs a = sa;
    a.logits = logits;
    a.prm = prm;
    a.ring = ring;
    a.hlen = hlen;
    a.hhead = hhead;
    a.rec = rec;
    a.cand = cand;
    const Run run = my_run(a);
    if (run.begin >= run.end) return;
    // Every staging load batch of a part after the first goes out right behind that part's
    // ring slot load: six vector memory operations, so a wavefront waiting for the batch
    // before them waits with vmcnt(6) while they stay in flight.
    Loc cur = part_at(a, run, run.begin);
    const int ring0 = ring_slot(a, cur.row);
    issue_stage(stage0, a, cur);
    for (int s = 0; s < 3; ++s) bitmap_zero(pl.bm[s], pl.hitw[s]);
    lds_barrier();
    bitmap_mark(pl.bm[0], pl.hitw[0], a, cur, ring0, mark_cap(a, cur.row));
    if (run.begin + 1 < run.end) {
        const Loc n1 = loc_next(a, run, cur);
        const int ring1 = ring_slot(a, n1.row);
        if constexpr (STAGES > 1) issue_stage(stage1, a, n1);
        bitmap_mark(pl.bm[1], pl.hitw[1], a, n1, ring1, mark_cap(a, n1.row));
    }
    lds_barrier();
    const int tid = tix();
    int idx = run.begin, s0 = 0;                      // part idx: bitmap slot s0
    Loc prev = cur;                                   // the part whose results are in LDS
    // one part: out of its staging buffer (each thread reads what it loaded), whose loads
    // for part idx + 2 then go out (after the ring slots that part needs)
    auto step = [&](float4 *stage) {
        const bool more = idx + 1 < run.end, more2 = idx + 2 < run.end;
        const int tl = idx - run.begin;
        TL_PART(tl, 0);
        // this part's staging loads: with two stages and a next part, its ring slot load and
        // staging loads (six operations) were issued after them; with one, nothing was
        if (STAGES > 1 && more) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        float4 X[UP];
#pragma unroll
        for (int u = 0; u < UP; ++u) X[u] = lds_read4(stage + u * NT + tid);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // read before overwritten
        if (idx > run.begin) flush_part(a, pl, prev.row * a.parts + prev.part);
        Loc n1 = cur, n2 = cur;
        int ring_val;                                 // set (and only read) with more2; no
        if (more) {                                   // initial value, which would have to
                                                      // wait for last part's ring load
            n1 = loc_next(a, run, cur);
            if (more2) {
                n2 = loc_next(a, run, n1);
                ring_val = ring_slot(a, n2.row);
                if constexpr (STAGES > 1) issue_stage(stage, a, n2);
            }
            if constexpr (STAGES == 1) issue_stage(stage, a, n1);
        }
        const qs_row_param P = stream_param(a, cur.row);
        const int s2 = s0 == 0 ? 2 : s0 - 1;          // (s0 + 2) mod 3
        part_step<GF>(X, a, cur, P, pl.bm[s0], pl.hitw[s0], (idx - run.begin) & 1, pl, [&] {
            // slot s0 was read by this part's pass 1 (done): cleared for part idx + 3;
            // slot s2 (cleared a part ago) gets part idx + 2's ids
            bitmap_zero(pl.bm[s0], pl.hitw[s0]);
            if (more2) bitmap_mark(pl.bm[s2], pl.hitw[s2], a, n2, ring_val,
                                   mark_cap(a, n2.row));
        }, tl);
        prev = cur;
        cur = n1;
        s0 = s0 == 2 ? 0 : s0 + 1;
        ++idx;
        return more;
    };
    if constexpr (STAGES > 1) {
        while (step(stage0) && step(stage1)) {
        }
    } else {
        while (step(stage0)) {
        }
    }
    flush_part(a, pl, prev.row * a.parts + prev.part);
}

// Row totals from the parts' aggregates held by lanes 0..NP-1 (one wavefront): the row's
// max, the certified denominator interval, the window size when every part lies wholly in or
// out of the window, the largest rejected key.
__device__ __forceinline__ CertTotals row_totals(const PartArgs &a, const qs_row_param &P,
                                                 bool greedy, bool have, uint32_t mk,
                                                 double psum, float pterm, uint32_t pmn,
                                                 int pnan, uint32_t prej) {
    const int lane = threadIdx.x & 63;
    const uint32_t rmx = wave_max_u(have ? mk : 0u);
    const float maxl = key2f(rmx > KEY_NEG_INF ? rmx : KEY_NEG_INF);
    const float inv_t = P.inv_t;
    const float msc = maxl * inv_t, thr = msc - 30.0f;
    CertPart cp{0.0, 0.0};
    const float maxw = have ? key2f(mk > KEY_NEG_INF ? mk : KEY_NEG_INF) : -INFINITY;
    if (!greedy && have) cp = cert_part(maxw, psum, pterm, inv_t, msc, thr);
    const double lo = wave_sum_d(cp.lo), hi = wave_sum_d(cp.hi);
    const int plen = have ? min(a.part_len, a.vocab - lane * a.part_len) : 0;
    const bool out_j = !(maxw * inv_t >= thr);
    const bool in_j = have && pmn != 0xFFFFFFFFu && key2f(pmn) * inv_t >= thr;
    const bool known = __ballot(have && !out_j && !in_j) == 0ull;
    const int nin = wave_sum_i(have && !out_j && in_j ? plen - pnan : 0);
    CertTotals t;
    t.maxl = maxl;
    t.msc = msc;
    double S_lo = 1.0, S_hi = 1.0;
    if (!greedy) cert_interval(lo, hi, msc, thr, a.vocab, S_lo, S_hi);
    t.S_lo = S_lo;
    t.S_hi = S_hi;
    t.v_lo = (float)(1.0 / S_hi);
    t.v_hi = (float)(1.0 / S_lo);
    t.nwin = known ? nin : -1;
    t.cflag = 0;
    t.rej = wave_max_u(have ? prej : 0u);
    t.total = 0;
    return t;
}

// Reductions over groups of 8 consecutive lanes in DPP moves: f(move) is called three times
// with the partner-lane moves quad_perm [1,0,3,2], quad_perm [2,3,0,1] and the half-row
// mirror; afterwards every lane of a group holds the group's result (a fixed order).
template <typename F>
__device__ __forceinline__ void group8(F &&f) {
    f([](auto v) { return dpp_move<0xB1, 0xF>(v); });
    f([](auto v) { return dpp_move<0x4E, 0xF>(v); });
    f([](auto v) { return dpp_move<0x141, 0xF>(v); });
}

// Decision statuses handed from the gathering wavefront to the whole workgroup.
enum { DS_DONE = 0, DS_BLOCK = 100, DS_SCAN = 101 };

// The row's gather and certified decision by wavefront 0 alone (rows of at most 16 parts:
// lanes hold wavefront records and lists L = lane and 64 + lane), with no workgroup barrier:
// the records and the first SPEC candidates of each list in one round trip, each part's
// totals over its 8 consecutive lanes, the row totals, the candidates above the row's bound
// compacted into LDS by a wavefront scan, then greedy rows' first maximum or cert_row_wave.
// Returns DS_DONE, DS_BLOCK (the block decision or the exact path must run: dl.ct and the
// gathered candidates are in place), DS_SCAN (a greedy row whose lists overflowed), or a
// CF_* reason (dl.ct and the candidates in place).
__device__ __forceinline__ int decide_wave0(const PartArgs &a, int row, const qs_row_param &P,
                                            DecLds &dl, const RowHist &hist) {
    constexpr int SPEC = 8;
    const int lane = threadIdx.x & 63;
    const Scratch &sc = a.sc;
    const int NP = a.parts, NL = NP * NWV;
    const int64_t l0 = (int64_t)row * NP * NWV;
    const bool greedy = row_greedy(P);
    WaveRec r[2];
    uint4 sp[2][SPEC / 2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int L = h * 64 + lane;
        if (L < NL) {
            r[h] = sc.wrec[l0 + L];
            const uint4 *src = (const uint4 *)(sc.pcand + (l0 + L) * WCAP);
#pragma unroll
            for (int i = 0; i < SPEC / 2; ++i) sp[h][i] = src[i];
        } else {
            r[h].sum = 0.0;
            r[h].term = 0.0f;
            r[h].mink = 0xFFFFFFFFu;
            r[h].nan = 0;
            r[h].maxk = 0u;
            r[h].rej = 0u;
            r[h].cnt = 0;
        }
    }
#ifdef QS_TIMELINE
    if (lane == 0) {
        volatile int sink = r[0].cnt + (int)sp[0][0].x;   // the loads have landed
        (void)sink;
    }
#endif
    QS_DEC_MARK(1);
    // each part's totals over its NWV consecutive lanes (a fixed order)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        double ps = r[h].sum;
        float pt = r[h].term;
        uint32_t pmn = r[h].mink;
        int pn = r[h].nan;
        static_assert(NWV == 8, "groups of 8 lanes");
        group8([&](auto &&mv) {
            ps += mv(ps);
            pt += mv(pt);
            pmn = min(pmn, mv(pmn));
            pn += mv(pn);
        });
        const int L = h * 64 + lane;
        if ((lane & (NWV - 1)) == 0 && L < NL) {
            const int j = L / NWV;
            dl.pmaxk[j] = r[h].maxk;
            dl.prej[j] = r[h].rej;
            dl.psum[j] = ps;
            dl.pterm[j] = pt;
            dl.pmin[j] = pmn;
            dl.pnan[j] = pn;
        }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    const bool have = lane < NP;
    CertTotals t = row_totals(a, P, greedy, have, have ? dl.pmaxk[lane] : 0u,
                              have ? dl.psum[lane] : 0.0, have ? dl.pterm[lane] : 0.0f,
                              have ? dl.pmin[lane] : 0xFFFFFFFFu, have ? dl.pnan[lane] : 0,
                              have ? dl.prej[lane] : 0u);
    QS_DEC_MARK(2);
    const int c[2] = {min(r[0].cnt, WCAP), min(r[1].cnt, WCAP)};
    t.cflag = __ballot(r[0].cnt > WCAP || r[1].cnt > WCAP) != 0ull;
    // f(entry) over the entries of this lane's lists
    auto each_entry = [&](auto &&f) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < SPEC; ++i)
                if (i < c[h]) {
                    const uint4 q = sp[h][i >> 1];
                    f((i & 1) ? make_uint2(q.z, q.w) : make_uint2(q.x, q.y));
                }
            const uint2 *src = sc.pcand + (l0 + h * 64 + lane) * WCAP;
            for (int i = SPEC; i < c[h]; ++i) f(src[i]);
        }
    };
    if (greedy) {
        // the first largest penalised logit (sample.c:130-132): every part's maxima are
        // among its candidates unless a list overflowed
        float bv = -INFINITY;
        int bi = -1;
        each_entry([&](uint2 e) { best_combine(bv, bi, key2f(e.x), (int)e.y); });
        if (t.cflag) {
            if (lane == 0) dl.ct = t;
            return DS_SCAN;
        }
        wave_best(bv, bi);
        if (lane == 0)
            record_greedy(row, P, bv, bi, t.maxl, a.logits[(int64_t)row * a.stride], a.st,
                          a.out, a.diag);
        return DS_DONE;
    }
    // the candidates above the row's bound (below it the lists are incomplete and everything
    // there counts as rejected), compacted in list order
    const uint32_t rej = t.rej;
    int k = 0;
    each_entry([&](uint2 e) { k += e.x > rej; });
    const int incl = wave_scan(k);
    t.total = __builtin_amdgcn_readlane(incl, 63);
    const bool finite = isfinite(t.msc);
    if (t.total <= FCAP && finite) {
        int at = incl - k;
        each_entry([&](uint2 e) {
            if (e.x > rej) {
                dl.keys[at] = e.x;
                dl.ids[at] = (int32_t)e.y;
                ++at;
            }
        });
    }
    if (lane == 0) dl.ct = t;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_wave_barrier();
    QS_DEC_MARK(3);
    if (!finite) return CF_INPUT;
    if (!(fabsf(t.msc) < CERT_MSC_MAX) || t.total > FCAP) return CF_MSC;
    if (row_ksel(P) > 64 || t.total > WAVE_CAND) return DS_BLOCK;
    return cert_row_wave(row, P, t, dl.keys, dl.ids, dl.srt, dl.dl.tab, a.st, a.out, a.diag,
                         hist);
}

// The decision of a sampling row of at most 16 parts by the whole workgroup: wavefront 0
// totals the parts' records into the denominator interval while wavefronts 1-3 gather the
// candidates above the row's bound into LDS, each from a third of every list's entries;
// then wavefront 0 takes the certified decision (cert_row_wave).  All threads call it;
// returns (in wavefront 0) DS_DONE, DS_BLOCK (the block decision or the exact path must
// run), or a CF_* reason, with dl.ct and the gathered candidates in place.
__device__ __forceinline__ int decide_par(const PartArgs &a, int row, const qs_row_param &P,
                                          DecLds &dl, const RowHist &hist) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    static_assert(ND == 256 && WCAP == 32, "three gathering wavefronts, 16 uint4 a list");
    const Scratch &sc = a.sc;
    const int NP = a.parts, NL = NP * NWV;
    const int64_t l0 = (int64_t)row * NP * NWV;
    // uint4s (two entries) of a list taken by wavefronts 1, 2, 3: [0, 5), [5, 10), [10, 16)
    const int u0 = wv == 0 ? 0 : 5 * (wv - 1), u1 = wv == 3 ? WCAP / 2 : 5 * wv;
    WaveRec r[2];
    uint4 q[2][6];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int L = h * 64 + lane;
        if (L < NL) {
            r[h] = sc.wrec[l0 + L];
            if (wv > 0) {
                const uint4 *src = (const uint4 *)(sc.pcand + (l0 + L) * WCAP);
#pragma unroll
                for (int i = 0; i < 6; ++i)
                    if (u0 + i < u1) q[h][i] = src[u0 + i];
            }
        } else {
            r[h].sum = 0.0;
            r[h].term = 0.0f;
            r[h].mink = 0xFFFFFFFFu;
            r[h].nan = 0;
            r[h].maxk = 0u;
            r[h].rej = 0u;
            r[h].cnt = 0;
        }
    }
    if (tid == 0) dl.gcount = 0;
    lds_barrier();                                // the counter (the loads stay in flight)
    QS_DEC_MARK(1);
    const bool ovf = __ballot(r[0].cnt > WCAP || r[1].cnt > WCAP) != 0ull;
    if (wv == 0) {
        // each part's totals over its NWV consecutive lanes (a fixed order), then the row's
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            double ps = r[h].sum;
            float pt = r[h].term;
            uint32_t pmn = r[h].mink;
            int pn = r[h].nan;
            group8([&](auto &&mv) {
                ps += mv(ps);
                pt += mv(pt);
                pmn = min(pmn, mv(pmn));
                pn += mv(pn);
            });
            const int L = h * 64 + lane;
            if ((lane & (NWV - 1)) == 0 && L < NL) {
                const int j = L / NWV;
                dl.pmaxk[j] = r[h].maxk;
                dl.prej[j] = r[h].rej;
                dl.psum[j] = ps;
                dl.pterm[j] = pt;
                dl.pmin[j] = pmn;
                dl.pnan[j] = pn;
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_wave_barrier();
        const bool have = lane < NP;
        CertTotals t = row_totals(a, P, false, have, have ? dl.pmaxk[lane] : 0u,
                                  have ? dl.psum[lane] : 0.0, have ? dl.pterm[lane] : 0.0f,
                                  have ? dl.pmin[lane] : 0xFFFFFFFFu, have ? dl.pnan[lane] : 0,
                                  have ? dl.prej[lane] : 0u);
        t.cflag = ovf;
        if (lane == 0) dl.ct = t;
    } else {
        // this wavefront's entries above the row's bound (the largest part bound: below it
        // the lists are incomplete and everything there counts as rejected), counted, placed
        // by one atomic and stored
        const uint32_t rj = wave_max_u(max(r[0].rej, r[1].rej));
        const int c[2] = {min(r[0].cnt, WCAP), min(r[1].cnt, WCAP)};
        auto each = [&](auto &&f) {
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 6; ++i) {
                    if (u0 + i >= u1) continue;
                    const int j = 2 * (u0 + i);
                    if (j < c[h] && q[h][i].x > rj) f(q[h][i].x, (int)q[h][i].y);
                    if (j + 1 < c[h] && q[h][i].z > rj) f(q[h][i].z, (int)q[h][i].w);
                }
        };
        int k = 0;
        each([&](uint32_t, int) { ++k; });
        const int incl = wave_scan(k);
        const int tot = __builtin_amdgcn_readlane(incl, 63);
        int base = 0;
        if (lane == 0 && tot > 0) base = atomicAdd(&dl.gcount, tot);
        base = __builtin_amdgcn_readfirstlane(base);
        int at = base + incl - k;
        each([&](uint32_t kv, int id) {
            if (at < FCAP) {
                dl.keys[at] = kv;
                dl.ids[at] = id;
            }
            ++at;
        });
    }
    lds_barrier();
    QS_DEC_MARK(2);
    const int total = dl.gcount;
    if (wv != 0) return 0;                        // (the caller reads wavefront 0's status)
    CertTotals t = dl.ct;
    t.total = total;
    if (lane == 0) dl.ct.total = total;
    QS_DEC_MARK(3);
    if (!isfinite(t.msc)) return CF_INPUT;
    if (!(fabsf(t.msc) < CERT_MSC_MAX) || total > FCAP) return CF_MSC;
    if (row_ksel(P) > 64 || total > WAVE_CAND) return DS_BLOCK;
    return cert_row_wave(row, P, t, dl.keys, dl.ids, dl.srt, dl.dl.tab, a.st, a.out, a.diag,
                         hist);
}

__global__ void __launch_bounds__(ND) k_decide(PartArgs a) {
    __shared__ DecLds dl;
    QS_DEC_MARK(0);
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const Scratch &sc = a.sc;
    const RowState &st = a.st;
    const int NP = a.parts;
    const int NL = NP * NWV;                          // candidate lists: NWV per part
    const int l0 = row * NP;
    const qs_row_param P = row_param(st, row);
    const bool greedy = row_greedy(P);
    const float *x = a.logits + (int64_t)row * a.stride;
    if (tid < QS_EXPF_TAB_N) dl.dl.tab[tid] = c_tab_part[tid];
    RowHist hist{0ull, 0, 0};
    if (tid < 64 && !greedy) hist = row_hist(st, row);
    if (NL <= 128) {
        // rows of up to 16 parts: greedy rows by wavefront 0 alone, sampling rows by the
        // workgroup (decide_par); the whole workgroup then takes the block decision, a
        // greedy row's scan or the exact path
        if (greedy) {
            if (wv == 0) {
                const int s0 = decide_wave0(a, row, P, dl, hist);
                if (lane == 0) dl.dl.sh[7] = s0;
            }
        } else {
            const int s0 = decide_par(a, row, P, dl, hist);
            if (tid == 0) dl.dl.sh[7] = s0;
        }
        __syncthreads();
        const int s0 = dl.dl.sh[7];
        QS_DEC_MARK(4);
        if (s0 == DS_DONE) return;
        if (s0 == DS_SCAN) {
            float bv = -INFINITY;
            int bi = -1;
            row_visit(a, row, P, dl, [&](float w, int id) {
                if (w == w) best_combine(bv, bi, w, id);
            });
            block_best(bv, bi, dl);
            if (tid == 0) record_greedy(row, P, bv, bi, dl.ct.maxl, x[0], st, a.out, a.diag);
            return;
        }
        const CertTotals t = dl.ct;
        int status = s0;
        if (s0 == DS_BLOCK) {
            status = cert_row_block<ND>(row, P, t, dl.keys, dl.ids, dl.srt, dl.dl, st, a.out,
                                        a.diag, hist);
            if (status == 0) return;
        }
        exact_row(a, row, P, t, dl, hist, status);
        return;
    }
    // records and lists tid and ND + tid (number L: wavefront L mod 8 of part L / 8, its
    // candidates at (l0*8 + L)*WCAP), with the first SPEC candidates: one round trip
    constexpr int SPEC = 8;
    WaveRec rec[2];
    uint4 spec[2][SPEC / 2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int L = h * ND + tid;
        if (L < NL) {
            rec[h] = sc.wrec[(int64_t)l0 * NWV + L];
            const uint4 *src = (const uint4 *)(sc.pcand + ((int64_t)l0 * NWV + L) * WCAP);
#pragma unroll
            for (int i = 0; i < SPEC / 2; ++i) spec[h][i] = src[i];
        } else {
            rec[h].sum = 0.0;
            rec[h].term = 0.0f;
            rec[h].mink = 0xFFFFFFFFu;
            rec[h].nan = 0;
            rec[h].maxk = 0u;
            rec[h].rej = 0u;
            rec[h].cnt = 0;
        }
    }
    // each part's totals from its NWV wavefront records (consecutive lanes, a fixed order)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        double ps = rec[h].sum;
        float pt = rec[h].term;
        uint32_t pmn = rec[h].mink;
        int pn = rec[h].nan;
#pragma unroll
        for (int o = 1; o < NWV; o <<= 1) {
            ps += __shfl_xor(ps, o, 64);
            pt += __shfl_xor(pt, o, 64);
            pmn = min(pmn, (uint32_t)__shfl_xor((int)pmn, o, 64));
            pn += __shfl_xor(pn, o, 64);
        }
        const int L = h * ND + tid;
        if ((tid & (NWV - 1)) == 0 && L < NL) {
            const int j = L / NWV;
            dl.pmaxk[j] = rec[h].maxk;
            dl.prej[j] = rec[h].rej;
            dl.psum[j] = ps;
            dl.pterm[j] = pt;
            dl.pmin[j] = pmn;
            dl.pnan[j] = pn;
        }
    }
    __syncthreads();
    if (tid < 64) {
        const bool have = lane < NP;
        const uint32_t mk = have ? dl.pmaxk[lane] : 0u;
        const uint32_t rmx = wave_max_u(mk);
        const float maxl = key2f(rmx > KEY_NEG_INF ? rmx : KEY_NEG_INF);
        const float inv_t = P.inv_t;
        const float msc = maxl * inv_t, thr = msc - 30.0f;
        CertPart cp{0.0, 0.0};
        const float maxw = have ? key2f(mk > KEY_NEG_INF ? mk : KEY_NEG_INF) : -INFINITY;
        if (!greedy && have) cp = cert_part(maxw, dl.psum[lane], dl.pterm[lane], inv_t, msc, thr);
        const double lo = wave_sum_d(cp.lo), hi = wave_sum_d(cp.hi);
        // window size: exact when every part lies wholly in or wholly out of it
        const int plen = have ? min(a.part_len, a.vocab - lane * a.part_len) : 0;
        const uint32_t pmn = have ? dl.pmin[lane] : 0xFFFFFFFFu;
        const bool out_j = !(maxw * inv_t >= thr);
        const bool in_j = have && pmn != 0xFFFFFFFFu && key2f(pmn) * inv_t >= thr;
        const bool known = __ballot(have && !out_j && !in_j) == 0ull;
        const int nin = wave_sum_i(have && !out_j && in_j ? plen - dl.pnan[lane] : 0);
        const uint32_t rj = wave_max_u(have ? dl.prej[lane] : 0u);
        if (lane == 0) {
            CertTotals t;
            t.maxl = maxl;
            t.msc = msc;
            double S_lo = 1.0, S_hi = 1.0;
            if (!greedy) cert_interval(lo, hi, msc, thr, a.vocab, S_lo, S_hi);
            t.S_lo = S_lo;
            t.S_hi = S_hi;
            t.v_lo = (float)(1.0 / S_hi);
            t.v_hi = (float)(1.0 / S_lo);
            t.nwin = known ? nin : -1;
            t.cflag = 0;
            t.rej = rj;
            t.total = 0;
            dl.ct = t;
        }
    }
    const int cnt0 = rec[0].cnt, cnt1 = rec[1].cnt;
    const int c0 = min(cnt0, WCAP), c1 = min(cnt1, WCAP);
    const int ovf = __ballot(cnt0 > WCAP || cnt1 > WCAP) != 0ull;
    // f(entry, list h, position) over the entries of lists tid and ND + tid
    auto each_entry = [&](auto &&f) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int n = h ? c1 : c0;
#pragma unroll
            for (int i = 0; i < SPEC; ++i)
                if (i < n) {
                    const uint4 q = spec[h][i >> 1];
                    f((i & 1) ? make_uint2(q.z, q.w) : make_uint2(q.x, q.y), h, i);
                }
            const uint2 *src = sc.pcand + ((int64_t)l0 * NWV + h * ND + tid) * WCAP;
            for (int i = SPEC; i < n; ++i) f(src[i], h, i);
        }
    };
    if (greedy) {
        // the first largest penalised logit (sample.c:130-132): every part's maxima are
        // among its candidates unless a list overflowed; then the row is scanned
        float bv = -INFINITY;
        int bi = -1;
        each_entry([&](uint2 e, int, int) { best_combine(bv, bi, key2f(e.x), (int)e.y); });
        if (lane == 0) dl.offs[wv] = ovf;
        __syncthreads();
        int anyovf = 0;
        for (int j = 0; j < ND / 64; ++j) anyovf |= dl.offs[j];
        if (anyovf) {
            bv = -INFINITY;
            bi = -1;
            row_visit(a, row, P, dl, [&](float w, int id) {
                if (w == w) best_combine(bv, bi, w, id);
            });
        }
        block_best(bv, bi, dl);
        if (tid == 0) record_greedy(row, P, bv, bi, dl.ct.maxl, x[0], st, a.out, a.diag);
        return;
    }
    // only candidates above the row's bound are gathered: below it a list is incomplete
    // (other parts may hold larger logits they did not keep), and the decision treats
    // everything there as rejected
    __syncthreads();
    const uint32_t rej_row = dl.ct.rej;
    int k0 = 0, k1 = 0;
    each_entry([&](uint2 e, int h, int) {
        if (e.x > rej_row) (h ? k1 : k0) += 1;
    });
    const int wincl = wave_scan(k0 + k1);
    if (lane == 63) dl.exc[wv] = wincl;
    if (lane == 0) dl.offs[wv] = ovf;
    __syncthreads();
    int wbase = 0, total = 0, anyovf = 0;
    for (int j = 0; j < ND / 64; ++j) {
        if (j < wv) wbase += dl.exc[j];
        total += dl.exc[j];
        anyovf |= dl.offs[j];
    }
    CertTotals t = dl.ct;
    t.total = total;
    t.cflag = anyovf;
    const bool finite = isfinite(t.msc);
    if (t.total <= FCAP && finite) {
        int at = wbase + wincl - (k0 + k1);
        each_entry([&](uint2 e, int, int) {
            if (e.x > rej_row) {
                dl.keys[at] = e.x;
                dl.ids[at] = (int32_t)e.y;
                ++at;
            }
        });
    }
    __syncthreads();
    int status = finite ? CF_MSC : CF_INPUT;
    if (finite && fabsf(t.msc) < CERT_MSC_MAX && t.total <= FCAP) {
        if (row_ksel(P) <= 64 && t.total <= WAVE_CAND) {
            if (tid < 64) {
                const int s = cert_row_wave(row, P, t, dl.keys, dl.ids, dl.srt, dl.dl.tab, st,
                                            a.out, a.diag, hist);
                if (tid == 0) dl.dl.sh[7] = s;
            }
            __syncthreads();
            status = dl.dl.sh[7];
            __syncthreads();
        } else {
            status = cert_row_block<ND>(row, P, t, dl.keys, dl.ids, dl.srt, dl.dl, st, a.out,
                                        a.diag, hist);
        }
    }
    if (status == 0) return;
    exact_row(a, row, P, t, dl, hist, status);
}

}  // namespace

int qs_part_parts(int n_vocab) { return (n_vocab + PART_MAX - 1) / PART_MAX; }

int qs_part_supported(int n_rows, int n_vocab, int64_t row_stride, const void *logits) {
    if (n_rows < 1 || n_vocab < 4 || n_vocab % 4 != 0 || row_stride % 4 != 0 ||
        ((uintptr_t)logits % 16) != 0)
        return 0;
    return qs_part_parts(n_vocab) <= QS_PART_MAX_PARTS;
}

int qs_part_resident(void) {
    int dev = 0, ncu = 0, nb = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_part<false>, NT, 0) != hipSuccess ||
        nb < 1)
        return 0;
    return ncu * nb;
}

int qs_part_launch(const float *logits, int64_t row_stride, int n_rows, int n_vocab,
                   const RowState &st, const Scratch &sc, int32_t *out, qs_pick_diag *diag,
                   int resident, hipStream_t stream, hipEvent_t mid, bool all_greedy) {
    PartArgs a;
    a.logits = logits;
    a.stride = row_stride;
    a.vocab = n_vocab;
    a.n_rows = n_rows;
    a.parts = qs_part_parts(n_vocab);
    a.part_len = PART_MAX;              // whole float4 rows: only a row's last part is short
    a.xcd_map = n_rows >= 8 ? 1 : 0;
    a.st = st;
    a.sc = sc;
    a.out = out;
    a.diag = diag;
    StreamArgs sa;
    sa.logits = logits;
    sa.stride = row_stride;
    sa.vocab = n_vocab;
    sa.n_rows = n_rows;
    sa.parts = a.parts;
    sa.part_len = a.part_len;
    sa.xcd_map = a.xcd_map;
    sa.ring_stride = st.ring_stride;
    sa.prm = st.prm;
    sa.ring = st.ring;
    sa.hlen = st.hlen;
    sa.hhead = st.hhead;
    sa.rec = sc.wrec;
    sa.cand = sc.pcand;
    sa.gbest = sc.gbest;
    sa.gmaxk = sc.gmaxk;
    sa.gcnt = sc.gcnt;
    sa.ring_w = st.ring;
    sa.hlen_w = st.hlen;
    sa.hhead_w = st.hhead;
    sa.out = out;
    sa.diag = diag;
    // a persistent grid: the resident workgroups (a multiple of 8 for the XCD mapping), or
    // one per part when there are fewer parts
    const int64_t total = (int64_t)n_rows * a.parts;
    int64_t grid = (int64_t)resident;
    if (a.xcd_map) grid = grid / 8 * 8;
    if (grid > total) grid = a.xcd_map ? (total + 7) / 8 * 8 : total;
    if (grid < 1) grid = 1;
    // every row greedy, with the scratch for it: each row decided by its last part
    const bool gf = all_greedy && sc.gbest != nullptr;
    if (gf)
        hipLaunchKernelGGL(k_part<true>, dim3((unsigned)grid), dim3(NT), 0, stream, sa,
                           sa.logits, sa.prm, sa.ring, sa.hlen, sa.hhead, sa.rec, sa.cand);
    else
        hipLaunchKernelGGL(k_part<false>, dim3((unsigned)grid), dim3(NT), 0, stream, sa,
                           sa.logits, sa.prm, sa.ring, sa.hlen, sa.hhead, sa.rec, sa.cand);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && mid) e = hipEventRecord(mid, stream);
    if (e == hipSuccess && !gf) {
        hipLaunchKernelGGL(k_decide, dim3((unsigned)n_rows), dim3(ND), 0, stream, a);
        e = hipGetLastError();
    }
    if (e != hipSuccess) {
        qs_set_error("streaming pick launch: %s", hipGetErrorString(e));
        return e == hipErrorOutOfMemory ? QS_ENOMEM : QS_EDEVICE;
    }
    return 0;
}

int qs_timeline_read(int which, uint64_t *dst, int n) {
    if (which == 2) {
        const int rc = qs_row_timeline_read(dst, n);
        if (rc) qs_set_error("qs_timeline_read: bad arguments, or not a timeline build");
        return rc;
    }
#ifdef QS_TIMELINE
    const size_t cap = which == 0 ? sizeof(g_tl_part) / 8 : sizeof(g_tl_dec) / 8;
    if (!dst || n < 0 || (size_t)n > cap || (which != 0 && which != 1)) {
        qs_set_error("qs_timeline_read: bad arguments");
        return QS_EINVAL;
    }
    const hipError_t e = which == 0
        ? hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_tl_part), 8 * (size_t)n)
        : hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_tl_dec), 8 * (size_t)n);
    if (e != hipSuccess) {
        qs_set_error("qs_timeline_read: %s", hipGetErrorString(e));
        return QS_EDEVICE;
    }
    return 0;
#else
    (void)which; (void)dst; (void)n;
    qs_set_error("qs_timeline_read: not a timeline build (make -C quasar_amd/csrc timeline)");
    return QS_EINVAL;
#endif
}
