// qs_pipe.hip - the pipelined pick for batches large enough to fill the GPU.
//
// One persistent workgroup of 1024 threads per CU (grid G <= CUs, checked against the
// device's occupancy for this kernel, so the whole grid is resident at once).  Every row
// is cut into PARTS = 8 parts; at stage s the grid works on G/PARTS rows, part j of
// row-in-stage q going to workgroup q + j*G/PARTS (with G a multiple of 64 the eight
// workgroups of a row are congruent mod 8, i.e. on one XCD when workgroups are dealt to
// XCDs round-robin).  A part is read from HBM once, straight into registers, and stays
// there until its softmax terms are summed.
//
// Wave 0 is the control wave and never loads logits; waves 1-15 (960 threads, UP float4
// each) hold data.  Three register buffers rotate: the part being summed (s), the next
// part, already penalised and published (s+1), and the part after that (s+2), loaded as
// part s-1 was summed.  Per stage, between two barriers:
//
//   data waves                                control wave
//   sum(s): w*inv_t, window, libm-equal       publish the max of part s+1 (completed last
//   expf, double partial sums, candidates     stage); store part s-1's sums and
//   at or above threshold(s); loads of part   candidates; part s+1's candidate threshold;
//   s+3 into the summed registers             history bitmap of part s+3; read the row
//   complete(s+2): penalty, thread max and    max of part s+1 (all eight partners
//   min                                       published it about the same time)
//
// so the row-max exchange overlaps the control wave's other work, the stores overlap the
// data waves' and a wave's memory counter never covers another wave's loads.  After the last
// stage each workgroup finishes rows r = w (mod G) with decide_row_fast, using its own
// full-window scratch slot.
//
// Every wait is bounded (SPIN_LIMIT polls): one that gives up sets the sticky error flag
// and the pick reports an error instead of hanging.  A workgroup only waits for
// publications that its partners make before they wait on anything later, and every
// workgroup of the grid is resident, so the waits end.

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>

#include "../../include/quasar_sampler.h"
#include "qs_device.h"
#include "qs_launch.h"

using namespace qs;

namespace {

constexpr int NT = 1024;             // threads per workgroup
constexpr int NWV = NT / 64;         // wavefronts
constexpr int DT = NT - 64;          // data threads (waves 1..15)
constexpr int PARTS = 8;             // parts per row
constexpr int UP = 5;                // float4 per data thread per part
constexpr int PCAP = 512;            // candidates per part (<= Scratch::ccap)
constexpr int WCAP = 32;             // candidates per data wave in LDS (NDW * WCAP <= PCAP)
constexpr int FCAP = 4096;           // candidates gathered per row in the epilogue
constexpr int NDW = NWV - 1;         // data waves
// Thread max keys of data wave j start at j*LM_STRIDE: an odd stride puts the 16 keys
// that lanes 4j..4j+3 of the control wave read at once (j + 16q + i mod 64) in distinct
// LDS banks.
constexpr int LM_STRIDE = 65;

__constant__ uint64_t c_exp_tab_p[QS_EXPF_TAB_N] = QS_EXPF_TABLE_INIT;

struct PipeArgs {
    const float *logits;
    int64_t stride;
    int vocab;
    int n_rows;
    int part_len;                    // elements per part (multiple of 4)
    int stages;
    RowState st;
    Scratch sc;
    int32_t *out;
    qs_pick_diag *diag;
};

// What the data waves need of a part's row, copied to LDS by the control wave: the data
// waves then issue no global reads besides the logits (a read of anything else would make
// their waits also cover the logit loads issued before it).
struct PartCfg {
    float inv_t;
    float rp;                        // repeat penalty
    int flags;                       // CFG_GREEDY | CFG_PEN
    int kw;                          // candidates the part keeps at least (part_k)
};
constexpr int CFG_GREEDY = 1, CFG_PEN = 2;

// Shared state of one workgroup besides the dynamic region.
struct PipeLds {
    DecideLds<NT> dl;
    uint64_t xtab[QS_EXPF_XTAB_N];   // qs_expf_window's extended table (the sums)
    // hand-offs between the data waves and the control wave, double-buffered by part
    // parity: written for one part while the other part's copy is read
    float wbv[2][NWV];               // greedy: per-wave best value / index
    int wbi[2][NWV];
    double wsum[2][NWV];             // per-wave partial sums of a summed part
    int wcnt[2][NWV];                // per-wave window counts
    int wcand[2][NWV];               // candidates each data wave found (its LDS list holds
                                     // the first WCAP of them)
    uint32_t maxkey[3];              // row max keys (by part index mod 3)
    uint32_t theta[4];               // candidate threshold keys (by part index mod 4)
    PartCfg cfg[4];                  // by part index mod 4
    uint32_t hitw[3][NDW];           // per bitmap slot and data wave: bit u set when the
                                     // wave's float4s u hold a history position
    uint32_t lmax[2][NDW * LM_STRIDE];   // each data thread's max key of a completed part
                                         // (data wave j at j*LM_STRIDE: see LM_STRIDE)
    RowTotals tot;
    int offs[PARTS + 1];
    float gbv;
    int gbi;
};

// History bitmap words of a part (one bit per logit, rounded up to whole 16-byte groups so
// that each of the three slots starts 16-byte aligned and is cleared with 16-byte stores).
__host__ __device__ constexpr int bitmap_words(int part_len) { return (part_len / 32 + 1 + 3) / 4 * 4; }

struct Geo {                         // this workgroup's part of every row
    int part, c_lo, c_hi, lo, rps, bm_words;
};

__device__ __forceinline__ int task_row(int s, int w, int rps) { return s * rps + (w % rps); }

// The data thread index, opaque to the compiler: each stage recomputes its few per-float4
// indices instead of the compiler keeping all of them (for all three buffer roles) live
// across the stage loop, which does not fit beside the three part buffers.
__device__ __forceinline__ int data_tid() {
    int dt = (int)threadIdx.x - 64;
    asm volatile("" : "+v"(dt));
    return dt;
}

// Candidates a part keeps: about twice its share of the row's top K plus a margin (the
// decision proves whatever it gets; a row whose top K crowd into one part takes the
// full-window path).
__device__ __forceinline__ int part_k(const qs_row_param &P) {
    const int k = 2 * ((row_ksel(P) + PARTS - 1) / PARTS) + 8;
    return k < DT ? k : DT;
}

__device__ __forceinline__ bool task_valid(const PipeArgs &a, int s, const Geo &g, int w) {
    return s < a.stages && task_row(s, w, g.rps) < a.n_rows;
}

// Control wave: the settings of a row for the data waves (from its fetched parameters).
__device__ __forceinline__ void set_cfg(PartCfg &c, const qs_row_param &P, bool pen) {
    if ((threadIdx.x & 63) != 0) return;
    c.inv_t = P.inv_t;
    c.rp = P.repeat_penalty;
    c.flags = (row_greedy(P) ? CFG_GREEDY : 0) | (pen ? CFG_PEN : 0);
    c.kw = part_k(P);
}

// Data waves: loads of one part into registers, through a buffer resource over the part
// (base: its first float4; size: its length), float4 u of data thread dt at byte offset
// (u*DT + dt)*16.  Loads past the part's end, and all loads of a stage without a part
// (size 0), return zeros without a memory access.  Every stage issues the same UP loads,
// so each wave's memory counter names exactly the loads a use waits for.
constexpr int BUF_WORD3 = 0x00020000;    // raw buffer, 32-bit data format
struct PartLoad {                        // the loads of one part (see issue_loads)
    __amdgpu_buffer_rsrc_t rs;
    int off;
    __device__ PartLoad(const PipeArgs &a, int row, bool live, const Geo &g) {
        const float *base = a.logits + (live ? (int64_t)row * a.stride + 4 * (int64_t)g.c_lo : 0);
        const int bytes = live ? (g.c_hi - g.c_lo) * 16 : 0;
        rs = __builtin_amdgcn_make_buffer_rsrc((void *)base, 0, bytes, BUF_WORD3);
        off = data_tid() * 16;
    }
    __device__ float4 load(int u) const {        // u's offset in the scalar offset
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, u * DT * 16, 0);
        return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                           __uint_as_float(v[3]));
    }
};
__device__ __forceinline__ void issue_loads(float4 (&buf)[UP], const PipeArgs &a, int row,
                                            bool live, const Geo &g) {
    const PartLoad nl(a, row, live, g);
#pragma unroll
    for (int u = 0; u < UP; ++u) buf[u] = nl.load(u);
}

// Data waves: penalty (sample.c:118-128) and each thread's max key (the control wave takes
// the part's max and candidate threshold from them); greedy rows: the wave's first argmax.
// `mn` receives the least of the thread's logits, NaN if one is NaN (positions past the part
// take part as the zeros their loads return, which the window test then passes).
// The max and min propagate NaN (one v_maximum3 / v_minimum3 per pair of logits, where
// fmaxf would first quiet each operand); a thread whose max comes out NaN takes the max of
// its other logits, as sample.c:125-127 does (NaN never wins).  Positions past the part
// read as -inf: never a max, a candidate or in the window.
__device__ __forceinline__ float max3n(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
__device__ __forceinline__ float min3n(float a, float b, float c) {
    return __builtin_elementwise_minimum(__builtin_elementwise_minimum(a, b), c);
}
__device__ __forceinline__ void complete_part(float4 (&buf)[UP], float &mn, const Geo &g,
                                              const uint32_t *bm, const uint32_t *hitw,
                                              const PartCfg &cf, PipeLds &pl, int par) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float rp = cf.rp;
    const bool pen = (cf.flags & CFG_PEN) != 0;
    const bool greedy = (cf.flags & CFG_GREEDY) != 0;
    const int dt = data_tid();
    // history bits of float4 u: word (u*DT + dt)/8 = u*DT/8 + dt/8, bits 4*(dt%8).. (DT is a
    // multiple of 8, so the shift is the same for every u)
    const uint32_t *bw = bm + (dt >> 3);
    const uint32_t bsh = (uint32_t)(dt & 7) * 4u;
    float mx = -INFINITY, bv = -INFINITY;
    mn = INFINITY;
    int bi = -1;
    // the float4s of this wavefront that hold history positions (a scalar mask), and
    // their history words, read at once
    const uint32_t hm = pen ? (uint32_t)__builtin_amdgcn_readfirstlane((int)hitw[wv - 1]) : 0u;
    uint32_t hw[UP];
#pragma unroll
    for (int u = 0; u < UP; ++u) hw[u] = ((hm >> u) & 1u) ? bw[u * (DT / 8)] : 0u;
#pragma unroll
    for (int u = 0; u < UP; ++u) {
        const int c = g.c_lo + u * DT + dt;
        float w[4] = {buf[u].x, buf[u].y, buf[u].z, buf[u].w};
        if ((hm >> u) & 1u) {                        // positions past the part are unmarked
            const uint32_t nib = __builtin_amdgcn_ubfe(hw[u], bsh, 4);
            if (__ballot(nib != 0u)) {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if ((nib >> k) & 1u) w[k] = penalise(w[k], rp);
            }
        }
        mn = min3n(min3n(mn, w[0], w[1]), w[2], w[3]);
        if (u == UP - 1 && c >= g.c_hi)             // past the part: only the last group
            w[0] = w[1] = w[2] = w[3] = -INFINITY;
        mx = max3n(max3n(mx, w[0], w[1]), w[2], w[3]);
        if (greedy) {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (w[k] > bv) { bv = w[k]; bi = 4 * c + k; }
        }
        buf[u] = make_float4(w[0], w[1], w[2], w[3]);
    }
    if (mx != mx) {                                  // a NaN among them: the others' max
        mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < UP; ++u)
            mx = fmaxf(mx, fmaxf(fmaxf(buf[u].x, buf[u].y), fmaxf(buf[u].z, buf[u].w)));
    }
    if (greedy) {
        wave_best(bv, bi);
        if (lane == 0) {
            pl.wbv[par][wv] = bv;
            pl.wbi[par][wv] = bi;
        }
    } else {
        pl.lmax[par][(wv - 1) * LM_STRIDE + lane] = f2key(mx);
    }
}

// Data waves: exact softmax numerators, partial sums, window count and candidates of one
// part, from registers (sample.c:136-149 per element).  When the thread minima (`mn`, from
// complete_part) of the whole wavefront are in the window, its float4s skip the per-logit
// window tests (the last one only in wavefronts without positions past the part);
// otherwise out-of-window lanes evaluate the exp at X_OUT (inside qs_expf_window's range)
// and their result is discarded.  A float4 holding no logit at or
// above the threshold skips the candidate test.
constexpr float X_OUT = -32.0f;

// The largest of four products w * inv_t (never signalling NaNs: the product quiets them)
// with quiet NaNs ignored, as v_max3_f32 does without the operand canonicalisation that
// fmaxf implies: a float4 holding a candidate always passes the test below.
__device__ __forceinline__ float max4q(const float (&v)[4]) {
    float m;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(m) : "v"(v[0]), "v"(v[1]), "v"(v[2]));
    asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(m), "v"(v[3]));
    return m;
}

__device__ __forceinline__ void sum_part(float4 (&buf)[UP], float mn, const PartLoad &nl,
                                         bool live, const Geo &g, const PartCfg &cf,
                                         uint32_t *ckey, int32_t *cid, uint32_t maxkey,
                                         uint32_t th, PipeLds &pl, int par) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const float inv_t = cf.inv_t;
    const float msc = key2f(maxkey) * inv_t;
    const float thr = msc - 30.0f;
    static_assert(NDW * WCAP <= PCAP, "every wave's list fits the part's");
    // greedy rows and rows without a finite maximum are decided in the epilogue: only the
    // next part's loads
    const bool work = live && !(cf.flags & CFG_GREEDY) && isfinite(msc);
    // candidates: every w >= key2f(th), tested as w*inv_t >= key2f(th)*inv_t (monotone in
    // w, so a superset; rejected logits stay below th)
    const float ths = key2f(th) * inv_t;
    const uint64_t *xtab = pl.xtab;
    const bool wave_in = __ballot(!(mn * inv_t >= thr)) == 0ull;   // NaN is not in
    // every lane's last float4 inside the part (only the part's last wavefront has lanes
    // past it)
    const bool full_last = g.c_lo + (UP - 1) * DT + (wv - 1) * 64 + 63 < g.c_hi;
    // no lane whose max key (complete_part's, still in its slot) reaches th: no candidate
    // (a logit below th that the scaled test would also take is not needed: the part's
    // rejected bound is th - 1)
    const bool wave_cand =
        work && __ballot(pl.lmax[par][(wv - 1) * LM_STRIDE + lane] >= th) != 0ull;
    float xo = X_OUT;
    asm volatile("" : "+v"(xo));                    // a register, selected before the exp
    double kshift = QS_EXPF_XSHIFT, c1 = QS_EXPF_C1;
    asm volatile("" : "+v"(kshift), "+v"(c1));      // in registers for the whole loop
    double acc = 0.0;
    int cnt = 0, wn = 0;                            // window count; candidates found
    uint32_t *wk = ckey + (wv - 1) * WCAP;         // this wave's candidate list
    int32_t *wi = cid + (wv - 1) * WCAP;
    const int dt = data_tid();
#pragma unroll
    for (int u = 0; u < UP; ++u) {
        if (u == 3) __builtin_amdgcn_s_setprio(1);   // the stage's priority steps (data_stage)
        if (u == 4) __builtin_amdgcn_s_setprio(0);
        float sc[4];
        if (work) {
            const int c = g.c_lo + u * DT + dt;
            const float w[4] = {buf[u].x, buf[u].y, buf[u].z, buf[u].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) sc[k] = w[k] * inv_t;
            if (wave_cand && __ballot(max4q(sc) >= ths)) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {            // positions by ballot prefix: no
                    const bool hit = sc[k] >= ths;       // atomics, nothing waited for
                    const uint64_t m = __ballot(hit);
                    if (m == 0ull) continue;
                    const int pos = wn + lane_prefix(m);
                    if (hit && pos < WCAP) {
                        wk[pos] = f2key(w[k]);
                        wi[pos] = 4 * c + k;
                    }
                    wn += __popcll(m);
                }
            }
        }
        // the next part's float4 u as soon as this one's logits are no longer needed (the
        // exp below works on sc); kept here: hoisted, the load would need registers of its
        // own
        asm volatile("" ::: "memory");
        buf[u] = nl.load(u);
        if (!work) continue;
        uint64_t in[4];
        bool all;
        if ((u < UP - 1 || full_last) && wave_in) { // every lane's four in the window
            in[0] = in[1] = in[2] = in[3] = ~0ull;
            cnt += 4 * 64;
            all = true;
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                in[k] = __ballot(sc[k] >= thr);     // NaN (or past the part) is out
                cnt += __popcll(in[k]);
            }
            all = (in[0] & in[1] & in[2] & in[3]) == __ballot(true);
        }
        if (all) {
            float xa[4], e[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) xa[k] = sc[k] - msc;
            qs_expf4_window(xa, e, xtab, kshift, c1);
            acc += (double)e[0];
            acc += (double)e[1];
            acc += (double)e[2];
            acc += (double)e[3];
        } else if (in[0] | in[1] | in[2] | in[3]) {
            float xa[4], e[4];
            bool ok[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                ok[k] = sc[k] >= thr;
                xa[k] = ok[k] ? sc[k] - msc : xo;
            }
            qs_expf4_window(xa, e, xtab, kshift, c1);
#pragma unroll
            for (int k = 0; k < 4; ++k) e[k] = ok[k] ? e[k] : 0.0f;
            acc += (double)e[0];
            acc += (double)e[1];
            acc += (double)e[2];
            acc += (double)e[3];
        }
    }
    if (!work) return;
    const double sa = wave_sum_d(acc);
    if (lane == 0) {
        pl.wsum[par][wv] = sa;
        pl.wcnt[par][wv] = cnt;        // the wave's count (sum of ballot popcounts)
        pl.wcand[par][wv] = wn;
    }
}

// Control wave: wait (bounded) until all parts of `row` published their max key (one slot
// per part, 0 until published: keys of part maxima are never 0); the row max key.  `k`
// holds lane i's first read of part i's slot (rowmax_slots), taken ahead by the caller so
// that its latency passes during other work.
__device__ __forceinline__ uint32_t poll_rowmax(const PipeArgs &a, int row, uint32_t k) {
    const int lane = threadIdx.x & 63;
    const uint32_t *slot = a.sc.rowmax + (int64_t)row * PARTS;
    int it = 0;
    while (__ballot(k == 0u) != 0ull) {
        if (++it >= SPIN_LIMIT) {
            if (lane == 0) atomicOr(a.sc.err, 2);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        k = lane < PARTS ? ld_dev(&slot[lane]) : 1u;
    }
    return wave_max_u(lane < PARTS ? k : 0u);
}
// The first read of those slots (lane i: part i's), issued ahead of the poll.
__device__ __forceinline__ uint32_t rowmax_slots(const PipeArgs &a, int row) {
    const int lane = threadIdx.x & 63;
    return lane < PARTS ? ld_dev(&a.sc.rowmax[(int64_t)row * PARTS + lane]) : 1u;
}

// Control wave: a row's parameters, history ring position and the first RING_PF*64 ring
// slots, all loaded at once (the slots do not wait for the position: a slot p holds a
// history id iff (p - head) mod cap < len, the positions sample.c:118 marks).  Fetched a
// stage before the row's part is completed, so the loads complete during other work.
constexpr int RING_PF = 8;
struct RowFetch {
    int pw;                          // lane i < 8: word i of the row's qs_row_param
    int lw, hw;                      // history length and ring head (every lane)
    int slot[RING_PF];
    __device__ qs_row_param param() const {   // read out of the lanes when used
        qs_row_param P;
        P.temperature = __int_as_float(__builtin_amdgcn_readlane(pw, 0));
        P.top_p = __int_as_float(__builtin_amdgcn_readlane(pw, 1));
        P.min_p = __int_as_float(__builtin_amdgcn_readlane(pw, 2));
        P.repeat_penalty = __int_as_float(__builtin_amdgcn_readlane(pw, 3));
        P.top_k = __builtin_amdgcn_readlane(pw, 4);
        P.ring_cap = __builtin_amdgcn_readlane(pw, 5);
        P.inv_t = __int_as_float(__builtin_amdgcn_readlane(pw, 6));
        P.pad = 0;
        return P;
    }
    __device__ int len() const { return __builtin_amdgcn_readfirstlane(lw); }
    __device__ int head() const { return __builtin_amdgcn_readfirstlane(hw); }
};
// Buffer loads at offsets the compiler treats as per-lane, so it moves nothing out of
// them into scalar registers (which would wait for them) before they are used.
__device__ __forceinline__ int lane_load(const void *base, int bytes, int off) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, BUF_WORD3);
    return (int)__builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
}
__device__ __forceinline__ RowFetch fetch_row(const PipeArgs &a, int row) {
    const int lane = threadIdx.x & 63;
    int vz;
    asm volatile("v_mov_b32 %0, 0" : "=v"(vz));     // zero, as a per-lane value
    RowFetch f;
    static_assert(sizeof(qs_row_param) == 32, "eight words of parameters");
    const int nb = a.n_rows * 4;
    f.pw = lane_load(a.st.prm, a.n_rows * 32, row * 32 + (lane & 7) * 4);
    f.lw = lane_load(a.st.hlen, nb, row * 4 + vz);
    f.hw = lane_load(a.st.hhead, nb, row * 4 + vz);
    // the ring slots: slots past the row's ring read as 0 without a memory access (and are
    // never marked, p >= ring_stride >= cap)
    const int32_t *ring = a.st.ring + (int64_t)row * a.st.ring_stride;
#pragma unroll
    for (int q = 0; q < RING_PF; ++q)
        f.slot[q] = lane_load(ring, a.st.ring_stride * 4, (q * 64 + lane) * 4);
    return f;
}
__device__ __forceinline__ bool row_pen(const RowFetch &f) {
    const qs_row_param P = f.param();
    return P.repeat_penalty > 1.0f && f.len() > 0 && P.ring_cap > 0;
}

// Control wave: the history bitmap of this workgroup's part of a row.
__device__ __forceinline__ void bitmap_build(uint32_t *bm, uint32_t *hitw, const RowFetch &f,
                                             const PipeArgs &a, int row, const Geo &g) {
    const int lane = threadIdx.x & 63;
    if (!row_pen(f)) return;
    uint4 *b4 = (uint4 *)bm;                        // bm_words is a multiple of 4
    for (int j = lane; j < g.bm_words / 4; j += 64) b4[j] = make_uint4(0u, 0u, 0u, 0u);
    if (lane < NDW) hitw[lane] = 0u;
    const int hi = g.c_hi * 4, cap = f.param().ring_cap, head = f.head(), len = f.len();
    auto mark = [&](int p, int id) {
        int d = p - head;
        if (d < 0) d += cap;
        if (p < cap && d < len && id >= g.lo && id < hi) {
            const int q = id - g.lo, c = q >> 2, u = c / DT;   // float4 c: thread c - u*DT
            atomicOr(&bm[q >> 5], 1u << (q & 31));
            atomicOr(&hitw[(c - u * DT) >> 6], 1u << u);
        }
    };
#pragma unroll
    for (int q = 0; q < RING_PF; ++q) mark(q * 64 + lane, f.slot[q]);
    if (cap > RING_PF * 64) {                       // longer rings: the rest directly
        const int32_t *ring = a.st.ring + (int64_t)row * a.st.ring_stride;
        for (int p = RING_PF * 64 + lane; p < cap; p += 64) mark(p, ring[p]);
    }
}

// Control wave: the largest of a part's thread max keys.
__device__ __forceinline__ uint32_t part_max(const uint32_t *lm) {
    const int lane = threadIdx.x & 63;
    uint32_t m = 0u;
#pragma unroll
    for (int j = 0; j < NDW; ++j) m = max(m, lm[j * LM_STRIDE + lane]);
    return wave_max_u(m);
}

__device__ __forceinline__ uint32_t umed3(uint32_t a, uint32_t b, uint32_t c) {
    return max(min(a, b), min(max(a, b), c));
}
// (t1 >= t2 >= t3) keeps the three largest of itself and v.
__device__ __forceinline__ void top3_insert(uint32_t &t1, uint32_t &t2, uint32_t &t3, uint32_t v) {
    const uint32_t n1 = max(t1, v), n2 = umed3(t1, t2, v), n3 = umed3(t2, t3, v);
    t1 = n1;
    t2 = n2;
    t3 = n3;
}

// Control wave: the three largest thread max keys of each data wave, lanes 4j..4j+3 holding
// data wave j's (each scans 16 of its 64 keys, then the quad merges); zeros past the data
// waves.  Their lane maximum is the part's max key.
struct Top3 {
    uint32_t t1, t2, t3;
};
__device__ __forceinline__ Top3 quad_top3(const uint32_t *lm) {
    const int lane = threadIdx.x & 63, j = lane >> 2;
    uint32_t t1 = 0u, t2 = 0u, t3 = 0u;              // thread max keys are never 0
    if (j < NDW) {
        const uint32_t *src = lm + j * LM_STRIDE + (lane & 3) * 16;
#pragma unroll
        for (int i = 0; i < 16; ++i) top3_insert(t1, t2, t3, src[i]);
    }
    {
        const uint32_t o1 = xor_lane<1>(t1), o2 = xor_lane<1>(t2), o3 = xor_lane<1>(t3);
        top3_insert(t1, t2, t3, o1);
        top3_insert(t1, t2, t3, o2);
        top3_insert(t1, t2, t3, o3);
    }
    {
        const uint32_t o1 = xor_lane<2>(t1), o2 = xor_lane<2>(t2), o3 = xor_lane<2>(t3);
        top3_insert(t1, t2, t3, o1);
        top3_insert(t1, t2, t3, o2);
        top3_insert(t1, t2, t3, o3);
    }
    return Top3{t1, t2, t3};
}

// The four largest thread max keys of each data wave, as quad_top3 (lanes 4j..4j+3 hold
// data wave j's); for parts whose kw exceeds what the top three give.
struct Top4 {
    uint32_t t1, t2, t3, t4;
};
__device__ __forceinline__ void top4_insert(Top4 &t, uint32_t v) {
    const uint32_t n1 = max(t.t1, v), n2 = umed3(t.t1, t.t2, v), n3 = umed3(t.t2, t.t3, v),
                   n4 = umed3(t.t3, t.t4, v);
    t = Top4{n1, n2, n3, n4};
}
__device__ __forceinline__ Top4 quad_top4(const uint32_t *lm) {
    const int lane = threadIdx.x & 63, j = lane >> 2;
    Top4 t{0u, 0u, 0u, 0u};                          // thread max keys are never 0
    if (j < NDW) {
        const uint32_t *src = lm + j * LM_STRIDE + (lane & 3) * 16;
#pragma unroll
        for (int i = 0; i < 16; ++i) top4_insert(t, src[i]);
    }
    {
        const Top4 o{xor_lane<1>(t.t1), xor_lane<1>(t.t2), xor_lane<1>(t.t3), xor_lane<1>(t.t4)};
        top4_insert(t, o.t1);
        top4_insert(t, o.t2);
        top4_insert(t, o.t3);
        top4_insert(t, o.t4);
    }
    {
        const Top4 o{xor_lane<2>(t.t1), xor_lane<2>(t.t2), xor_lane<2>(t.t3), xor_lane<2>(t.t4)};
        top4_insert(t, o.t1);
        top4_insert(t, o.t2);
        top4_insert(t, o.t3);
        top4_insert(t, o.t4);
    }
    return t;
}

// Control wave: the part's candidate threshold, the kw-th largest of a set of thread max
// keys (kw distinct logits of the part reach it; the part keeps every logit at or above
// it, and every other one lies below it).  The set is each data wave's three largest
// (from quad_top3), or four largest (quad_top4) when kw exceeds those, or all of them.
__device__ __forceinline__ uint32_t part_theta(const Top3 &tp, const uint32_t *lm,
                                               const PartCfg &cf) {
    const int lane = threadIdx.x & 63;
    uint32_t th;
    if (cf.kw <= 3 * NDW) {
        // the 45 values one per lane (lane 4j+q: wave j's (q+1)-th), sorted: the kw-th
        const int q = lane & 3;
        uint32_t v = ((lane >> 2) < NDW && q < 3) ? (q == 0 ? tp.t1 : q == 1 ? tp.t2 : tp.t3) : 0u;
        v = wave_sort_desc_u32(v);
        th = (uint32_t)__builtin_amdgcn_readlane((int)v, cf.kw - 1);
    } else if (cf.kw <= 4 * NDW) {
        // the 60 values one per lane (lane 4j+q: wave j's (q+1)-th), sorted: the kw-th
        const Top4 t4 = quad_top4(lm);
        const int q = lane & 3;
        uint32_t v = (lane >> 2) < NDW ? (q == 0 ? t4.t1 : q == 1 ? t4.t2 : q == 2 ? t4.t3 : t4.t4)
                                       : 0u;
        v = wave_sort_desc_u32(v);
        th = (uint32_t)__builtin_amdgcn_readlane((int)v, cf.kw - 1);
    } else {
        uint32_t k[NDW];
#pragma unroll
        for (int j = 0; j < NDW; ++j) k[j] = lm[j * LM_STRIDE + lane];
        th = wave_kth(k, cf.kw, DT);
    }
    return th <= KEY_NEG_INF ? KEY_NEG_INF + 1u : th;   // -inf and NaN never qualify
}

// Control wave: publish the completed part's max (sampling; returns the per-wave top three
// for the part's threshold) or best (greedy).
__device__ __forceinline__ Top3 control_publish(const PipeArgs &a, int row, const Geo &g,
                                                PipeLds &pl, int par, int cfg_slot) {
    const int lane = threadIdx.x & 63;
    const PartCfg &cf = pl.cfg[cfg_slot];
    const int li = row * PARTS + g.part;
    Top3 tp{0u, 0u, 0u};
    if (cf.flags & CFG_GREEDY) {
        if (lane == 0) {
            float v0 = pl.wbv[par][1];
            int i0 = pl.wbi[par][1];
            for (int k = 2; k < NWV; ++k) best_combine(v0, i0, pl.wbv[par][k], pl.wbi[par][k]);
            st_dev(&a.sc.bestv[li], v0);
            st_dev(&a.sc.besti[li], i0);
            stores_done();
            add_dev(&a.sc.done[row], 1);
        }
        return tp;
    }
    uint32_t mk;
    if (cf.kw <= 3 * NDW) {
        tp = quad_top3(pl.lmax[par]);
        mk = wave_max_u(tp.t1);
    } else {
        mk = part_max(pl.lmax[par]);
    }
    if (lane == 0) st_dev(&a.sc.rowmax[li], mk);  // seen by the partners' polls
    return tp;
}

// Control wave: store a summed part's results; control_release announces them once every
// store has completed.  Returns whether there is anything to announce.
__device__ __forceinline__ bool control_store(const PipeArgs &a, int row, const Geo &g,
                                              uint32_t maxkey, uint32_t th,
                                              const uint32_t *ckey, const int32_t *cid,
                                              const PartCfg &cf, PipeLds &pl, int par) {
    const int lane = threadIdx.x & 63;
    if (cf.flags & CFG_GREEDY) return false;      // published with its best already
    const int li = row * PARTS + g.part;
    const bool live = isfinite(key2f(maxkey) * cf.inv_t);
    // the data waves' lists, one count per lane, concatenated in wave order: lane 4j+q
    // copies entries q, q+4, ... of data wave j's list
    const int cw = (live && lane < NDW) ? pl.wcand[par][lane + 1] : 0;
    const int cwc = min(cw, WCAP);
    const int incl = wave_scan(cwc);
    const int n = __builtin_amdgcn_readlane(incl, NDW - 1);
    const int ovf = __ballot(cw > WCAP) != 0ull;   // a list overflowed: incomplete
    uint32_t *gk = a.sc.ckey + (int64_t)li * PCAP;
    int32_t *gi = a.sc.cid + (int64_t)li * PCAP;
    {
        const int j = (lane >> 2) & 15;            // lanes 60-63: lane 15's count, 0
        const int cnt_j = __shfl(cwc, j, 64), off_j = __shfl(incl - cwc, j, 64);
        for (int i = lane & 3; i < cnt_j; i += 4) {
            st_dev(&gk[off_j + i], ckey[j * WCAP + i]);
            st_dev(&gi[off_j + i], cid[j * WCAP + i]);
        }
    }
    // the data waves' partial sums and window counts, one per lane (every data wave wrote
    // its own when the part is live)
    const bool mine = live && lane < NDW;
    const double t = wave_sum_d(mine ? pl.wsum[par][lane + 1] : 0.0);
    const int ct = wave_sum_i(mine ? pl.wcnt[par][lane + 1] : 0);
    if (lane == 0) {
        st_dev(&a.sc.psum[li], t);
        st_dev(&a.sc.pcnt[li], ct);
        st_dev(&a.sc.ccnt[li], n);
        st_dev(&a.sc.cflag[li], ovf);
        st_dev(&a.sc.crej[li], (live && th > KEY_NEG_INF) ? th - 1u : 0u);
    }
    return true;
}
__device__ __forceinline__ void control_release(const PipeArgs &a, int row) {
    stores_done();                                // the whole wave's stores, then the count
    if ((threadIdx.x & 63) == 0) add_dev(&a.sc.done[row], 1);
}

// Finish row r: gather its PARTS partial results and decide (all threads).
template <bool PAR>
__device__ __forceinline__ void finish_row(const PipeArgs &a, int row, uint32_t *dyn, PipeLds &pl, int slot) {
    const int tid = threadIdx.x, lane = tid & 63;
    const RowState &st = a.st;
    const Scratch &sc = a.sc;
    const qs_row_param P = st.prm[row];
    RowHist hist{0ull, 0, 0};                        // the decision's, in flight meanwhile
    if (tid < 64) hist = row_hist(st, row);
    if (tid == 0) {
        int it = 0;
        while (ld_dev(&sc.done[row]) < PARTS) {
            if (++it >= SPIN_LIMIT) {
                atomicOr(sc.err, 4);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
    const int l0 = row * PARTS;
    // The first SPEC candidates of every part, loaded with the totals (one round trip;
    // a part with more is completed below).
    constexpr int SPEC = NT / PARTS;
    const int sp = tid / SPEC, si = tid % SPEC;
    uint32_t skey = 0u;
    int32_t sid = 0;
    if (!row_greedy(P)) {
        const int64_t src = (int64_t)(l0 + sp) * PCAP + si;
        skey = ld_dev(&sc.ckey[src]);
        sid = ld_dev(&sc.cid[src]);
    }
    if (tid < 64) {
        const bool have = lane < PARTS;
        if (row_greedy(P)) {
            float bv = have ? ld_dev(&sc.bestv[l0 + lane]) : -INFINITY;
            int bi = have ? ld_dev(&sc.besti[l0 + lane]) : -1;
            const float mx = wave_max_f(bv);
            wave_best(bv, bi);
            if (lane == 0) { pl.gbv = bv; pl.gbi = bi; pl.tot.maxl = mx; }
        } else {
            // one value per part in lanes 0-7: eight-lane reductions and scan
            static_assert(PARTS == 8, "lanes 0-7 hold the parts");
            double ps = have ? ld_dev(&sc.psum[l0 + lane]) : 0.0;
            int pc = have ? ld_dev(&sc.pcnt[l0 + lane]) : 0;
            int cc = have ? ld_dev(&sc.ccnt[l0 + lane]) : 0;
            int cf = have ? ld_dev(&sc.cflag[l0 + lane]) : 0;
            uint32_t cr = have ? ld_dev(&sc.crej[l0 + lane]) : 0u;
            uint32_t rk = have ? ld_dev(&sc.rowmax[(int64_t)row * PARTS + lane]) : 0u;
            ps = lane8_reduce(ps, [](double x, double y) { return x + y; });
            pc = lane8_reduce(pc, [](int x, int y) { return x + y; });
            cf = lane8_reduce(cf, [](int x, int y) { return x | y; });
            cr = lane8_reduce(cr, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
            const uint32_t rmx = lane8_reduce(rk, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
            const int incl = wave_scan(cc);
            if (have) pl.offs[lane] = incl - cc;
            if (lane == PARTS - 1) pl.offs[PARTS] = incl;
            if (lane == 0) {
                pl.tot.maxl = key2f(rmx);
                pl.tot.sum = ps;
                pl.tot.nwin = pc;
                pl.tot.cflag = cf;
                pl.tot.rej = cr;
            }
        }
    }
    __syncthreads();
    const float *x = a.logits + (int64_t)row * a.stride;
    if (row_greedy(P)) {
        if (tid == 0) record_greedy(row, P, pl.gbv, pl.gbi, pl.tot.maxl, x[0], st, a.out, a.diag);
    } else {
        uint32_t *keys = dyn;
        int32_t *ids = (int32_t *)(dyn + FCAP);
        uint64_t *srt = (uint64_t *)(dyn + 2 * FCAP);
        FullLds<NT> &fl = *(FullLds<NT> *)dyn;       // aliases keys/ids (dead by then)
        RowTotals t = pl.tot;
        t.total = pl.offs[PARTS];
        if (t.total <= FCAP && isfinite(t.maxl * P.inv_t)) {
            const int n_sp = pl.offs[sp + 1] - pl.offs[sp];
            if (si < n_sp) {
                keys[pl.offs[sp] + si] = skey;
                ids[pl.offs[sp] + si] = sid;
            }
            for (int p = 0; p < PARTS; ++p) {            // parts with more than SPEC
                const int n = pl.offs[p + 1] - pl.offs[p];
                for (int j = SPEC + tid; j < n; j += NT) {
                    const int64_t src = (int64_t)(l0 + p) * PCAP + j;
                    keys[pl.offs[p] + j] = ld_dev(&sc.ckey[src]);
                    ids[pl.offs[p] + j] = ld_dev(&sc.cid[src]);
                }
            }
        }
        __syncthreads();
        decide_row_fast<NT, SORT_CAP, PAR>(row, P, t, FCAP, keys, ids, srt, pl.dl, fl, x, a.vocab, st, sc,
                            a.out, a.diag, slot, &hist);
    }
    __syncthreads();
    if (tid < PARTS) st_dev(&sc.rowmax[(int64_t)row * PARTS + tid], 0u);   // ready for the
    if (tid == 0) st_dev(&sc.done[row], 0);                                 // next pick
}

// One stage, data waves: sum part s (in `cur`), issue the loads of part s+3 into `cur`,
// complete part s+2 (in `ld`, loaded during the previous stage).
__device__ __forceinline__ void data_stage(float4 (&cur)[UP], float mcur, float4 (&ld)[UP],
                                           float &mld, int s,
                                           const PipeArgs &a, const Geo &g, int w,
                                           const uint32_t *bm, uint32_t *ckey, int32_t *cid,
                                           PipeLds &pl) {
    const bool v0 = task_valid(a, s, g, w), v2 = task_valid(a, s + 2, g, w),
               v3 = task_valid(a, s + 3, g, w);
    const int r3 = task_row(s + 3, w, g.rps);
    const int p0 = s & 1;
    __syncthreads();
    // The SIMD issues for the wavefront of highest priority first (then the oldest): each
    // data wavefront lowers its priority as it gets through the stage (2 for float4s 0-2
    // of the sum, 1 for float4 3, 0 from float4 4 on, set in sum_part), so the ones behind
    // catch up and the SIMD keeps several wavefronts to switch between until the end.
    __builtin_amdgcn_s_setprio(2);
    const PartLoad nl(a, r3, v3, g);              // part s+3, into `cur` as it is summed
    sum_part(cur, mcur, nl, v0, g, pl.cfg[s & 3], ckey + p0 * PCAP, cid + p0 * PCAP,
             pl.maxkey[s % 3], pl.theta[s & 3], pl, p0);
    __builtin_amdgcn_s_setprio(0);
    if (v2)
        complete_part(ld, mld, g, bm + ((s + 2) % 3) * g.bm_words, pl.hitw[(s + 2) % 3],
                      pl.cfg[(s + 2) & 3], pl, p0);
}

// One stage, control wave: publish part s+1's max (completed during the previous stage),
// store part s-1's sums and candidates, build part s+3's history bitmap, read part s+1's
// row max.  Every hand-off crosses the barrier at the top of a stage into a slot the other
// side does not use in that stage (part parity for thread maxima, wave results and
// candidate lists; part index mod 3 for bitmaps and row maxima, mod 4 for thresholds and
// settings).
__device__ __forceinline__ void control_stage(int s, RowFetch &rp, const PipeArgs &a,
                                              const Geo &g, int w,
                                              uint32_t *bm, const uint32_t *ckey,
                                              const int32_t *cid, PipeLds &pl) {
    const int lane = threadIdx.x & 63;
    const bool v1 = task_valid(a, s + 1, g, w), v3 = task_valid(a, s + 3, g, w);
    const int r1 = task_row(s + 1, w, g.rps), r3 = task_row(s + 3, w, g.rps);
    const int p1 = (s & 1) ^ 1;
    __syncthreads();
    const RowFetch f3 = rp;                      // part s+3's row, fetched last stage
    if (task_valid(a, s + 4, g, w)) rp = fetch_row(a, task_row(s + 4, w, g.rps));
    Top3 tp{0u, 0u, 0u};
    if (v1) tp = control_publish(a, r1, g, pl, p1, (s + 1) & 3);
    const bool sv = s >= 1 && task_valid(a, s - 1, g, w);
    const int rs = task_row(s - 1, w, g.rps);
    bool rel = false;
    if (sv)
        rel = control_store(a, rs, g, pl.maxkey[(s + 2) % 3], pl.theta[(s + 3) & 3],
                            ckey + p1 * PCAP, cid + p1 * PCAP, pl.cfg[(s + 3) & 3], pl, p1);
    // the row max: the partners' slots read now (after the stores, which the wait for this
    // read then covers), looked at after the threshold and bitmap
    const bool sampled = v1 && !(pl.cfg[(s + 1) & 3].flags & CFG_GREEDY);
    const uint32_t k0 = sampled ? rowmax_slots(a, r1) : 1u;
    if (sampled) {
        const uint32_t th = part_theta(tp, pl.lmax[p1], pl.cfg[(s + 1) & 3]);
        if (lane == 0) pl.theta[(s + 1) & 3] = th;
    }
    if (v3) {
        bitmap_build(bm + (s % 3) * g.bm_words, pl.hitw[s % 3], f3, a, r3, g);   // s+3's slot
        set_cfg(pl.cfg[(s + 3) & 3], f3.param(), row_pen(f3));   // part s-1's settings are used
    }
    if (sampled) {
        const uint32_t key = poll_rowmax(a, r1, k0);
        if (lane == 0) pl.maxkey[(s + 1) % 3] = key;
    }
    if (rel) control_release(a, rs);              // the stores completed before the poll
}

// PAR: the block decision takes the wavefront prefix sums where they are exact (rows with
// top K above 64).  Without it that code stays out of the kernel, whose register
// allocation the stages feel; both give the same results.
template <bool PAR>
__global__ void __launch_bounds__(NT) k_pipe(PipeArgs a) {
    extern __shared__ __align__(16) uint32_t dyn[];
    __shared__ PipeLds pl;
    const int w = blockIdx.x, tid = threadIdx.x;
    const bool data = tid >= 64;
    Geo g;
    g.rps = gridDim.x / PARTS;
    g.part = w / g.rps;
    g.lo = g.part * a.part_len;
    const int p_hi = min(g.lo + a.part_len, a.vocab);
    g.c_lo = g.lo >> 2;
    g.c_hi = p_hi >> 2;
    g.bm_words = bitmap_words(a.part_len);
    uint32_t *bm = dyn;                              // [3][bm_words], part p at p mod 3
    uint32_t *ckey = dyn + 3 * g.bm_words;           // [2][PCAP]
    int32_t *cid = (int32_t *)(ckey + 2 * PCAP);     // [2][PCAP]

    // prologue: parts 0 and 1 completed, part 0's row max known (exchanged while part 1
    // is completed), part 2 loading and its bitmap built.  Data and control waves then run loops of their own (the branch is on
    // the wavefront index, uniform in each wavefront), meeting at one barrier per stage.
    const bool t0 = task_valid(a, 0, g, w), t1 = task_valid(a, 1, g, w),
               t2 = task_valid(a, 2, g, w);
    const int r0 = task_row(0, w, g.rps), r1 = task_row(1, w, g.rps), r2 = task_row(2, w, g.rps);
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (wave != 0) {
        float4 B0[UP], B1[UP], B2[UP];
        float M0 = 0.0f, M1 = 0.0f, M2 = 0.0f;  // thread minima of the parts in B0..B2
        issue_loads(B0, a, r0, t0, g);           // at once, beside the control wave's fetches
        __syncthreads();                         // every wave's part 0 ahead of part 1
        issue_loads(B1, a, r1, t1, g);
        for (int j = tid - 64; j < QS_EXPF_XTAB_N; j += DT) pl.xtab[j] = qs_expf_xtab_entry(pl.dl.tab, j);
        __syncthreads();                         // part 0's bitmap and settings
        if (t0) complete_part(B0, M0, g, bm, pl.hitw[0], pl.cfg[0], pl, 0);
        __syncthreads();                         // part 0's max is exchanged meanwhile
        issue_loads(B2, a, r2, t2, g);
        if (t1) complete_part(B1, M1, g, bm + g.bm_words, pl.hitw[1], pl.cfg[1], pl, 1);
        // buffer roles rotate with period 3: every full pass through the loop leaves the
        // same loads in flight (the next part's, in B2) and each wait covers only the
        // loads it needs; the last pass stops after the last stage
        for (int s = 0; s < a.stages; s += 3) {
            data_stage(B0, M0, B2, M2, s, a, g, w, bm, ckey, cid, pl);
            if (s + 1 >= a.stages) break;
            data_stage(B1, M1, B0, M0, s + 1, a, g, w, bm, ckey, cid, pl);
            if (s + 2 >= a.stages) break;
            data_stage(B2, M2, B1, M1, s + 2, a, g, w, bm, ckey, cid, pl);
        }
    } else {
        // the control wave's steps are on every stage's critical path: it issues ahead of
        // the data wavefronts that share its SIMD
        __builtin_amdgcn_s_setprio(3);
        // the row fetches of the prologue, issued as the data waves issue part 0's loads
        const bool t3 = task_valid(a, 3, g, w);
        RowFetch f0, f1, f2, rp;
        if (t0) f0 = fetch_row(a, r0);
        if (t1) f1 = fetch_row(a, r1);
        if (t2) f2 = fetch_row(a, r2);
        if (t3) rp = fetch_row(a, task_row(3, w, g.rps));
        if (tid < QS_EXPF_TAB_N) pl.dl.tab[tid] = c_exp_tab_p[tid];   // after the fetches
        __syncthreads();
        if (t0) {
            bitmap_build(bm, pl.hitw[0], f0, a, r0, g);
            set_cfg(pl.cfg[0], f0.param(), row_pen(f0));
        }
        __syncthreads();                             // part 0 is completed meanwhile
        if (t1) {
            bitmap_build(bm + g.bm_words, pl.hitw[1], f1, a, r1, g);
            set_cfg(pl.cfg[1], f1.param(), row_pen(f1));
        }
        if (t2) {                                    // used from stage 0 on
            bitmap_build(bm + 2 * g.bm_words, pl.hitw[2], f2, a, r2, g);
            set_cfg(pl.cfg[2], f2.param(), row_pen(f2));
        }
        __syncthreads();
        Top3 tp0{0u, 0u, 0u};
        if (t0) tp0 = control_publish(a, r0, g, pl, 0, 0);
        if (t0 && !(pl.cfg[0].flags & CFG_GREEDY)) {
            const uint32_t th = part_theta(tp0, pl.lmax[0], pl.cfg[0]);
            if ((tid & 63) == 0) pl.theta[0] = th;
        }
        if (t0 && !(pl.cfg[0].flags & CFG_GREEDY)) {
            const uint32_t key = poll_rowmax(a, r0, rowmax_slots(a, r0));
            if ((tid & 63) == 0) pl.maxkey[0] = key;
        }

        for (int s = 0; s < a.stages; ++s) control_stage(s, rp, a, g, w, bm, ckey, cid, pl);
    }
    __builtin_amdgcn_s_setprio(0);
    __syncthreads();
    if (!data) {                     // the last summed part, unless the loop stored it
        const int s = a.stages - 1;
        if (s >= 0 && task_valid(a, s, g, w))
            if (control_store(a, task_row(s, w, g.rps), g, pl.maxkey[s % 3], pl.theta[s & 3],
                              ckey + (s & 1) * PCAP, cid + (s & 1) * PCAP, pl.cfg[s & 3], pl,
                              s & 1))
                control_release(a, task_row(s, w, g.rps));
    }
    __syncthreads();
    // epilogue: rows r = w (mod G), each with this workgroup's full-window slot
    for (int r = w; r < a.n_rows; r += gridDim.x) finish_row<PAR>(a, r, dyn, pl, w);
}

}  // namespace

int qs_pipe_supported(int n_rows, int n_vocab, int64_t row_stride, const void *logits,
                      int grid) {
    if (grid < 64 || grid % 64 != 0) return 0;
    if (n_vocab % 4 != 0 || row_stride % 4 != 0 || ((uintptr_t)logits % 16) != 0) return 0;
    const int part_len = ((n_vocab + PARTS - 1) / PARTS + 3) / 4 * 4;
    if (part_len > 4 * DT * UP || part_len < 4 * DT * (UP - 1)) return 0;
    // the last part (possibly shorter) ends inside its last group of float4s too
    if (n_vocab - (PARTS - 1) * part_len <= 4 * DT * (UP - 1)) return 0;
    if ((int64_t)n_rows * PARTS < grid) return 0;     // too few rows to fill the grid
    return 1;
}

size_t qs_pipe_lds_bytes(int n_vocab) {
    const int part_len = ((n_vocab + PARTS - 1) / PARTS + 3) / 4 * 4;
    const size_t pipe = sizeof(uint32_t) * (3 * (size_t)bitmap_words(part_len) + 4 * PCAP);
    const size_t epi = sizeof(uint32_t) * 2 * FCAP + sizeof(uint64_t) * SORT_CAP;
    const size_t fl = sizeof(FullLds<NT>);
    size_t m = pipe > epi ? pipe : epi;
    return m > fl ? m : fl;
}

int qs_pipe_parts(void) { return PARTS; }

// Workgroups of the pipelined kernel: a multiple of PARTS, at most one per CU, and only if
// the device holds one workgroup per CU with the LDS the largest vocabulary needs (the
// whole grid is then resident at once, so every workgroup's partners run); 0 otherwise.
int qs_pipe_grid(int max_vocab) {
    int dev = 0, ncu = 0, nb = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_pipe<true>, NT, qs_pipe_lds_bytes(max_vocab)) !=
            hipSuccess ||
        nb < 1)
        return 0;
    return ncu / PARTS * PARTS;
}

int qs_pipe_launch(const float *logits, int64_t row_stride, int n_rows, int n_vocab,
                   const RowState &st, const Scratch &sc, int32_t *out, qs_pick_diag *diag,
                   int grid, int wide_k, hipStream_t stream) {
    PipeArgs a;
    a.logits = logits;
    a.stride = row_stride;
    a.vocab = n_vocab;
    a.n_rows = n_rows;
    a.part_len = ((n_vocab + PARTS - 1) / PARTS + 3) / 4 * 4;
    const int rps = grid / PARTS;
    a.stages = (n_rows + rps - 1) / rps;
    a.st = st;
    a.sc = sc;
    a.out = out;
    a.diag = diag;
    if (wide_k)
        hipLaunchKernelGGL(k_pipe<true>, dim3(grid), dim3(NT), qs_pipe_lds_bytes(n_vocab), stream, a);
    else
        hipLaunchKernelGGL(k_pipe<false>, dim3(grid), dim3(NT), qs_pipe_lds_bytes(n_vocab), stream, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        qs_set_error("k_pipe launch: %s", hipGetErrorString(e));
        return e == hipErrorOutOfMemory ? QS_ENOMEM : QS_EDEVICE;
    }
    return 0;
}
