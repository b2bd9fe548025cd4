// qs_head.hip - the output layer (LM head) and the sampler's streaming pass in one kernel,
// then the row decisions: forward_cpu.c:319-323 (logits = W . xn) followed by
// sample.c:111-179 per row, for batched decoding with the hidden states and the output
// matrix in HBM.
//
// k_head_prep, one workgroup per row: marks the row's history ids in a bitmap laid out by
// (row group of 32, vocabulary id), one bit per row, for k_head's epilogue.
//
// k_head64 / k_head128 / k_head256 (k_head below), one workgroup of 8 wavefronts per tile
// of 128 vocabulary columns and every row
// (at most 256): logits[r][v] = sum_k H[r][k] W[v][k] with bf16 operands and fp32
// accumulation on the matrix cores (v_mfma_f32_32x32x16_bf16), 32 embedding elements a
// stage.  Three shapes by batch size (HeadShape): up to 64, 128 or 256 rows, each
// wavefront owning 32 x 32, 64 x 32 or 64 x 64 of the output, with a six-, four- or
// three-stage LDS ring.  The hidden rows and the weights (packed by k_head_pack into the
// order they are staged) go by direct loads into the ring, read by the wavefronts as
// operands.  Two such workgroups share a CU (at most 80 KB of LDS, at most 128 registers),
// so one's epilogue runs under the other's products and loads.  Every column tile is
// computed once for all rows, so W is read from HBM once per pick.  The epilogue
// moves one 32-row block at a time through LDS and,
// per row: writes the raw logits (for the rare rows the decision recounts), applies the
// repeat penalty (sample.c:118-128), and records for the (row, tile) what the sampler's
// streaming pass takes from those logits: the penalised max and min, the NaN count and the
// certified sums of the tile against an integer exponent base (qs_cert.h), the same
// summation the row kernel uses.  It clears its columns of the history bitmap.
//
// k_head_decide, one workgroup per row: the row's max and denominator interval from its
// tile records; the tiles whose maximum is at or above a bound at or below the (K + 2)-th
// largest tile maximum hold every logit at or above that bound (at least K + 2 logits),
// so only those tiles' logits are
// read back to gather the candidates; then the certified decision (cert_row_block) and, for
// rows it does not cover, the exact path over the written logits (qs_decide.h).  A greedy
// row scans the first tile holding its max.
//
// The logits the decision reads per row are the K + 2 tiles' (at top-k 40, 42 x 512 bytes)
// instead of the whole row (4 V bytes); the write of the logits remains.

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>
#include <type_traits>
#include <cstring>

#include "../../include/quasar_sampler.h"
#include "qs_cert.h"
#include "qs_decide.h"
#include "qs_device.h"
#include "qs_launch.h"

using namespace qs;
using namespace qs::dec;

namespace {

constexpr int HT = QS_HEAD_TILE;        // vocabulary columns per tile workgroup
constexpr int HNW = 8;                  // its wavefronts
constexpr int HNT = HNW * 64;
constexpr int HK = 32;                  // embedding elements per stage
constexpr int CSP = HT + 4;             // pitch of the staged output block (floats)
constexpr int TMAX = QS_HEAD_MAX_TILES; // tiles per row at most

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__constant__ uint64_t c_tab_head[QS_EXPF_TAB_N] = QS_EXPF_TABLE_INIT;

struct HeadArgs {
    const uint16_t *h;                  // [n_rows][E] bf16 bits
    const uint16_t *w;                  // packed weights (k_head_pack), bf16 bits
    int E, n_rows, V, ntiles;
    float *logits;                      // [n_rows][V] raw logits (written)
    uint32_t *hb;                       // [QS_HEAD_MAX_ROWS / 32][V] history bits, bit r % 32 of row r
    HeadRec *rec;                       // [n_rows][ntiles]
    int records;                        // 0: logits only
    RowState st;
};

// k_head's shape for a batch of at most RB rows: each wavefront owns WRB 32-row blocks x
// WCB 32-column blocks of the RB x 128 output; NSTG stages in the LDS ring (NSTG - 1 in
// flight).  Fewer rows leave room for a deeper ring: more of the weights in flight.
template <int RB> struct HeadShape;
template <> struct HeadShape<256> { static constexpr int WRB = 2, WCB = 2, NSTG = 3; };
template <> struct HeadShape<128> { static constexpr int WRB = 2, WCB = 1, NSTG = 4; };
template <> struct HeadShape<64> { static constexpr int WRB = 1, WCB = 1, NSTG = 6; };

// One stage: 32 embedding elements of every hidden row and of the tile's 128 weight rows,
// 64 bytes a row, the row's four 16-byte segments stored in the order seg ^ ((row / 4) % 4)
// (the lanes of an operand read then hit distinct banks).
template <int RB>
struct HeadStage {
    uint16_t h[RB][HK];
    uint16_t w[HT][HK];
};
template <int RB>
struct HeadLds {
    union {
        HeadStage<RB> stg[HeadShape<RB>::NSTG];   // the K loop's ring
        float cs[32][CSP];                        // the epilogue's 32-row block
    };
    uint32_t hbits[RB / 32][HT];                  // the tile's history bits
};
// two workgroups per CU (160 KB of LDS): one's epilogue overlaps the other's products
static_assert(sizeof(HeadLds<256>) <= 80 * 1024 && sizeof(HeadLds<128>) <= 80 * 1024 &&
                  sizeof(HeadLds<64>) <= 80 * 1024,
              "two tile workgroups per CU");

// The weights in the order k_head stages them: for tile t (columns 128 t ..) and stage s
// (embedding elements 32 s ..), 128 columns x 4 segments of 8 elements, segment j of
// column c holding elements 32 s + 8 (j ^ ((c / 4) % 4)) .. + 8 of W's row 128 t + c
// (zeros past the vocabulary).  One 16-byte piece per thread.
__global__ void __launch_bounds__(256) k_head_pack(const uint16_t *w, int E, int V, int ntiles,
                                                   uint16_t *pk) {
    const int nst = E / HK;
    const int64_t n = (int64_t)ntiles * nst * HT * 4;
    for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < n;
         q += (int64_t)gridDim.x * 256) {
        const int j = (int)(q & 3), c = (int)((q >> 2) % HT);
        const int64_t ts = (q >> 2) / HT;
        const int st = (int)(ts % nst), t = (int)(ts / nst);
        const int col = t * HT + c;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (col < V)
            v = *(const uint4 *)(w + (int64_t)col * E + st * HK + ((j ^ ((c >> 2) & 3)) * 8));
        *(uint4 *)(pk + q * 8) = v;
    }
}

// Reductions over the 16 lanes of a DPP row (every lane of the row receives the result;
// the row's lanes are all active).
template <typename T, typename F>
__device__ __forceinline__ T row16_reduce(T v, F &&op) {
    v = op(v, dpp_move<0xB1, 0xF>(v));      // quad_perm [1,0,3,2]
    v = op(v, dpp_move<0x4E, 0xF>(v));      // quad_perm [2,3,0,1]
    v = op(v, dpp_move<0x141, 0xF>(v));     // row_half_mirror
    return op(v, dpp_move<0x140, 0xF>(v));  // row_mirror
}
__device__ __forceinline__ uint32_t row16_max_u(uint32_t v) {
    return row16_reduce(v, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ uint32_t row16_min_u(uint32_t v) {
    return row16_reduce(v, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ int row16_sum_i(int v) {
    return row16_reduce(v, [](int a, int b) { return a + b; });
}
__device__ __forceinline__ double row16_sum_d(double v) {
    return row16_reduce(v, [](double a, double b) { return a + b; });
}

// sample.c:119-120 for the rows of the pick: bit (r % 32) of hb[r / 32][id] for every id in
// row r's history (k_head clears the bits of its columns after reading them).
__global__ void __launch_bounds__(256) k_head_prep(HeadArgs a) {
    const int row = blockIdx.x;
    const RowState &st = a.st;
    const qs_row_param P = row_param(st, row);
    const int cap = P.ring_cap;
    int len, head;
    ring_pos(st, row, cap, len, head);
    if (!(P.repeat_penalty > 1.0f) || len <= 0 || cap <= 0) return;
    const int32_t *ring = st.ring + (int64_t)row * st.ring_stride;
    for (int j = threadIdx.x; j < len; j += 256) {
        const int id = ring[qs_ring_slot(cap, head, j)];
        if (id >= 0 && id < a.V) atomicOr(&a.hb[(int64_t)(row >> 5) * a.V + id], 1u << (row & 31));
    }
}

// Wait until at most N of this wavefront's vector memory loads are in flight.
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N <= 15, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

template <int RB>
__device__ __forceinline__ void head_tile(const HeadArgs &a) {
    using S = HeadShape<RB>;
    constexpr int NSTG = S::NSTG, WRB = S::WRB, WCB = S::WCB;
    constexpr int NRG = RB / (32 * WRB);            // row groups (NRG x column groups = 8)
    static_assert(NRG * (HT / (32 * WCB)) == HNW, "one block per wavefront");
    constexpr int HBLK = RB / 16;                   // hidden-row blocks of 16 per stage
    __shared__ __attribute__((aligned(16))) HeadLds<RB> L;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col0 = blockIdx.x * HT;
    const int B = a.n_rows, E = a.E, V = a.V;
    const int nrb = (B + 31) >> 5;

    // stage s: H[0..B)[32 s, 32 s + 32) and W[col0 .. col0 + 128)[32 s, 32 s + 32) into
    // ring slot s % NSTG by direct loads to LDS (no registers): each wavefront instruction
    // fills 1 KB of the slot, 16 rows of 64 bytes, lane i row i / 4 and stored segment i % 4
    // (global segment (i % 4) ^ ((row / 4) % 4)).  Hidden rows past the batch read row 0
    // (their results are never used); the packed weights hold each such 1 KB piece
    // contiguously, already swizzled, columns past the vocabulary as zeros.
    const int nst = E / HK;
    auto issue = [&](int st) {
        HeadStage<RB> &g = L.stg[st % NSTG];
        const int k0 = st * HK;
#pragma unroll
        for (int i = 0; i < (HBLK + HNW - 1) / HNW; ++i) {   // hidden rows: blocks of 16,
            const int blk = wv + i * HNW;                    // wavefront w takes w, w + 8
            if (blk >= HBLK) break;                          // (uniform)
            const int r = blk * 16 + (lane >> 2);
            const int sg = (lane & 3) ^ ((r >> 2) & 3);
            const uint16_t *src = a.h + (int64_t)(r < B ? r : 0) * E + k0 + sg * 8;
            __builtin_amdgcn_global_load_lds(src, &g.h[blk * 16][0], 16, 0, 0);
        }
        {                                            // weight rows (the tile's columns):
            const int blk = wv;                      // 8 blocks of 16, one per wavefront
            const uint16_t *src =
                a.w + (((int64_t)blockIdx.x * nst + st) * HT + blk * 16) * HK + lane * 8;
            __builtin_amdgcn_global_load_lds(src, &g.w[blk * 16][0], 16, 0, 0);
        }
    };

    // wavefront w computes rows 32 WRB (w % NRG) .. + 32 WRB x columns 32 WCB (w / NRG) ..
    // + 32 WCB of the tile
    const int rg = wv % NRG, cg = wv / NRG;
    f32x16 acc[WRB][WCB];
#pragma unroll
    for (int i = 0; i < WRB; ++i)
#pragma unroll
        for (int j = 0; j < WCB; ++j) acc[i][j] = f32x16{};
    // operand segment s of row r sits at segment s ^ ((r / 4) % 4)
    const int rr = lane & 31;
    const int swz = (rr >> 2) & 3;
    for (int st = 0; st < NSTG - 1 && st < nst; ++st) issue(st);
    // the tile's history bits (and clear them for the next pick), requested after the first
    // stages so that their latencies overlap
    if (a.records) {
        for (int i = tid; i < nrb * HT; i += HNT) {
            const int g = i / HT, c = i - g * HT;
            uint32_t v = 0u;
            if (col0 + c < V) {
                uint32_t *p = a.hb + (int64_t)g * V + col0 + c;
                v = *p;
                if (v) *p = 0u;
            }
            L.hbits[g][c] = v;
        }
    }

    for (int st = 0; st < nst; ++st) {
        // this stage's loads are in: at most the next NSTG - 2 stages' remain (each one
        // weight block and this wavefront's hidden blocks); near the end, none
        if (st + NSTG - 2 < nst) {
            constexpr int HL = HBLK >= HNW ? HBLK / HNW : 1;
            if (HBLK >= HNW || wv < HBLK) vm_wait<(NSTG - 2) * (HL + 1)>();
            else vm_wait<NSTG - 2>();
        } else {
            vm_wait<0>();
        }
        // a barrier without __syncthreads()'s fence, which would wait for every load in
        // flight (the later stages' too): each wavefront has just waited for its own loads
        // of this stage, and the slot refilled next was read by products already issued
        asm volatile("s_barrier" ::: "memory");
        if (st + NSTG - 1 < nst) issue(st + NSTG - 1);   // into the slot read last stage
        const HeadStage<RB> &g = L.stg[st % NSTG];
#pragma unroll
        for (int ks = 0; ks < HK / 16; ++ks) {
            // the step's operands read together, then its products
            const int sg = (ks * 2 + (lane >> 5)) ^ swz;
            u32x4 ha[WRB], wb[WCB];
#pragma unroll
            for (int i = 0; i < WRB; ++i)
                ha[i] = *(const u32x4 *)&g.h[(rg * WRB + i) * 32 + rr][sg * 8];
#pragma unroll
            for (int j = 0; j < WCB; ++j)
                wb[j] = *(const u32x4 *)&g.w[(cg * WCB + j) * 32 + rr][sg * 8];
#pragma unroll
            for (int i = 0; i < WRB; ++i)
#pragma unroll
                for (int j = 0; j < WCB; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, ha[i]), __builtin_bit_cast(bf16x8, wb[j]),
                        acc[i][j], 0, 0, 0);
        }
    }
    __syncthreads();

    // epilogue, one 32-row block at a time: lane (l, j) of accumulator (i, cb) of wavefront w
    // holds row (j / 4) * 8 + (l / 32) * 4 + j % 4 of block WRB (w % NRG) + i, column
    // 32 (WCB (w / NRG) + cb) + l % 32
    const int ncol = min(HT, V - col0);
#pragma unroll
    for (int rb = 0; rb < RB / 32; ++rb) {           // (unrolled: acc stays in registers)
        if (rb >= nrb) break;
        if (rg == rb / WRB) {                        // the wavefronts holding the block
#pragma unroll
            for (int cb = 0; cb < WCB; ++cb)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int m = (j >> 2) * 8 + (lane >> 5) * 4 + (j & 3);
                    L.cs[m][(cg * WCB + cb) * 32 + (lane & 31)] = acc[rb % WRB][cb][j];
                }
        }
        __syncthreads();
        // wavefront w: rows 4 w .. 4 w + 3 of the block, one per 16-lane DPP row; lane p of
        // a row: columns 4 p + 64 i (i < 2), so a row's lanes read 256 consecutive bytes per
        // i and its reductions stay inside the DPP row
        const int m = wv * 4 + (lane >> 4), r = rb * 32 + m, p = lane & 15;
        if (rb * 32 + wv * 4 < B) {                  // (uniform) a row of the wavefront exists
            const bool live = r < B;
            constexpr int NI = HT / 64;
            float4 v[NI];
#pragma unroll
            for (int i = 0; i < NI; ++i) v[i] = *(const float4 *)&L.cs[m][p * 4 + 64 * i];
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int c = p * 4 + 64 * i;
                if (live && c < ncol) *(float4 *)(a.logits + (int64_t)r * V + col0 + c) = v[i];
            }
            if (a.records) {
                const qs_row_param &P = a.st.prm[live ? r : B - 1];
                const float rp = P.repeat_penalty, inv_t = P.inv_t;
                const double rinv = 1.0 / (double)rp;
                float mx = -INFINITY, mn = INFINITY;
                int nan = 0;
#pragma unroll
                for (int i = 0; i < NI; ++i) {
                    const int c = p * 4 + 64 * i;
                    const uint4 hbw = *(const uint4 *)&L.hbits[rb][c];
                    const uint32_t hbit[4] = {hbw.x, hbw.y, hbw.z, hbw.w};
                    float w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {     // (ncol is a multiple of 4)
                        if (c >= ncol) { w[e] = -INFINITY; continue; }
                        if ((hbit[e] >> (r & 31)) & 1u) w[e] = penalise_r(w[e], rp, rinv);
                        if (w[e] != w[e]) { ++nan; continue; }
                        mx = fmaxf(mx, w[e]);
                        mn = fminf(mn, w[e]);
                    }
                    v[i] = make_float4(w[0], w[1], w[2], w[3]);
                }
                const uint32_t maxk = row16_max_u(f2key(mx));
                const uint32_t mink = row16_min_u(mn != INFINITY ? f2key(mn) : 0xFFFFFFFFu);
                const int nant = __ballot(nan != 0) ? row16_sum_i(nan) : 0;
                double S = 0.0, T = 0.0;
                float cbase = 0.0f;
                if (!row_greedy(P)) {                // (uniform over the DPP row)
                    const float Mw = key2f(maxk > KEY_NEG_INF ? maxk : KEY_NEG_INF) * inv_t;
                    if (Mw > -INFINITY && Mw < INFINITY) {
                        cbase = cert_cbase(Mw);
                        double s = 0.0;
                        float tn = 0.0f;
#pragma unroll
                        for (int i = 0; i < NI; ++i) sum4<true>(v[i], inv_t, cbase, s, tn);
                        S = row16_sum_d(s);
                        T = row16_sum_d((double)tn);
                    }
                }
                if (p == 0 && live) {
                    HeadRec h;
                    h.maxk = maxk > KEY_NEG_INF ? maxk : KEY_NEG_INF;
                    h.mink = mink;
                    h.nan = nant;
                    h.c = cbase;
                    h.sum = S;
                    h.term = -T;
                    a.rec[(int64_t)r * a.ntiles + blockIdx.x] = h;
                }
            }
        }
        __syncthreads();
    }
}

// One kernel per shape (a template kernel's host stub is not emitted here).
__global__ void __launch_bounds__(HNT) __attribute__((amdgpu_waves_per_eu(4)))
k_head64(HeadArgs a) { head_tile<64>(a); }
__global__ void __launch_bounds__(HNT) __attribute__((amdgpu_waves_per_eu(4)))
k_head128(HeadArgs a) { head_tile<128>(a); }
__global__ void __launch_bounds__(HNT) __attribute__((amdgpu_waves_per_eu(4)))
k_head256(HeadArgs a) { head_tile<256>(a); }

struct HeadDecLds {
    DecLds d;
    uint32_t tmax[TMAX];                // the row's tile maxima (keys)
    int sel[TMAX];                      // tile -> slot among the selected tiles (-1: not)
    int stile[TMAX];                    // slot -> tile
    uint32_t selbits[TMAX][HT / 32];    // history bits of the selected tiles' columns
    uint32_t urej;                      // largest key not gathered
    uint32_t th;                        // the tiles' threshold
    int nsel;
    double plo[ND / 64], phi[ND / 64];
    int pin[ND / 64], pkn[ND / 64];
};

__global__ void __launch_bounds__(ND) k_head_decide(HeadArgs a, PartArgs pa) {
    __shared__ HeadDecLds HL;
    DecLds &dl = HL.d;
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const RowState &st = a.st;
    const qs_row_param P = row_param(st, row);
    const bool greedy = row_greedy(P);
    const int NT_ = a.ntiles, V = a.V;
    const float *x = a.logits + (int64_t)row * V;
    const HeadRec *rr = a.rec + (int64_t)row * NT_;
    if (tid < QS_EXPF_TAB_N) dl.dl.tab[tid] = c_tab_head[tid];
    RowHist hist{0ull, 0, 0};
    if (tid < 64 && !greedy) hist = row_hist(st, row);
    // the row's tile records (each thread's RPT of them kept in registers) and its max
    constexpr int RPT = (TMAX + ND - 1) / ND;
    HeadRec hr[RPT];
    uint32_t mk = 0u;
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const int t = tid + k * ND;
        if (t < NT_) {
            hr[k] = rr[t];
            HL.tmax[t] = hr[k].maxk;
            HL.sel[t] = -1;
            mk = max(mk, hr[k].maxk);
        }
    }
    // the first ND history ids, requested with the records
    const float rp = P.repeat_penalty;
    const int cap = P.ring_cap;
    int len, head;
    ring_pos(st, row, cap, len, head);
    const bool pen = rp > 1.0f && len > 0 && cap > 0;
    const int32_t *ring = st.ring + (int64_t)row * st.ring_stride;
    const int hid0 = pen && tid < len ? ring[qs_ring_slot(cap, head, tid)] : -1;
    mk = wave_max_u(mk);
    if (lane == 0) dl.exc[wv] = (int)mk;
    __syncthreads();
    uint32_t rmx = 0u;
    for (int j = 0; j < ND / 64; ++j) rmx = max(rmx, (uint32_t)dl.exc[j]);
    const float maxl = key2f(rmx > KEY_NEG_INF ? rmx : KEY_NEG_INF);
    const float inv_t = P.inv_t, msc = maxl * inv_t, thr = msc - 30.0f;
    __syncthreads();
    // the tiles to read back: a greedy row's first tile holding its max; otherwise the tiles
    // whose maximum is at or above a bound th at or below the (K + 2)-th largest tile
    // maximum: they hold every logit at or above th, at least K + 2 of them
    const int K = row_ksel(P);
    const int kp = min(K + 2, NT_);
    uint32_t th = rmx;
    if (greedy) {
        int t0 = NT_;
        for (int t = tid; t < NT_; t += ND)
            if (HL.tmax[t] == rmx) t0 = min(t0, t);
        for (int o = 32; o > 0; o >>= 1) t0 = min(t0, __shfl_xor(t0, o, 64));
        if (lane == 0) dl.exc[wv] = t0;
        __syncthreads();
        int tb = NT_;
        for (int j = 0; j < ND / 64; ++j) tb = min(tb, dl.exc[j]);
        if (tid == 0) {
            HL.nsel = tb < NT_ ? 1 : 0;
            if (tb < NT_) {
                HL.sel[tb] = 0;
                HL.stile[0] = tb;
            }
        }
    } else {
        // the denominator interval from the tiles' sums, and the window size when every
        // tile lies wholly in or out of the window
        double lo = 0.0, hi = 0.0;
        int nin = 0, unk = 0;
#pragma unroll
        for (int k = 0; k < RPT; ++k) {
            const int t = tid + k * ND;
            if (t >= NT_) continue;
            const HeadRec &h = hr[k];
            const float maxw = key2f(h.maxk);
            const CertPart cp = cert_part_c(maxw, h.c, h.sum, h.term, inv_t, msc, thr);
            lo += cp.lo;
            hi += cp.hi;
            const int tlen = min(HT, V - t * HT);
            const bool out_j = !(maxw * inv_t >= thr);
            const bool in_j = h.mink != 0xFFFFFFFFu && key2f(h.mink) * inv_t >= thr;
            if (!out_j && in_j) nin += tlen - h.nan;
            else if (!out_j) unk = 1;
        }
        lo = wave_sum_d(lo);
        hi = wave_sum_d(hi);
        nin = wave_sum_i(nin);
        unk = __ballot(unk != 0) != 0ull;
        if (lane == 0) { HL.plo[wv] = lo; HL.phi[wv] = hi; HL.pin[wv] = nin; HL.pkn[wv] = unk; }
        if (kp <= 64) {
            // a bound at or below the kp-th largest tile maximum from one wavefront: the
            // kp-th largest of its lanes' maxima (a subset of the tile maxima), so at least
            // kp tiles lie at or above it; a few more tiles are read than with the exact
            // kp-th, without the block's radix select (the maxima were stored before the
            // last barrier)
            if (wv == 0) {
                uint32_t lm = 0u;
                for (int t = lane; t < NT_; t += 64) lm = max(lm, HL.tmax[t]);
                const uint32_t srt = wave_sort_desc_u32(lm);
                const uint32_t x = (uint32_t)__builtin_amdgcn_readlane((int)srt, kp - 1);
                if (lane == 0) HL.th = x;
            }
            __syncthreads();
            th = HL.th;
        } else {
            __syncthreads();
            th = block_kth<ND>(HL.tmax, NT_, kp, dl.dl.hist, dl.dl.sh + 4);
        }
        if (tid == 0) {
            double l2 = 0.0, h2 = 0.0;
            int n2 = 0, u2 = 0;
            for (int j = 0; j < ND / 64; ++j) { l2 += HL.plo[j]; h2 += HL.phi[j]; n2 += HL.pin[j]; u2 |= HL.pkn[j]; }
            CertTotals t;
            t.maxl = maxl;
            t.msc = msc;
            double S_lo = 1.0, S_hi = 1.0;
            cert_interval(l2, h2, msc, thr, V, S_lo, S_hi);
            t.S_lo = S_lo;
            t.S_hi = S_hi;
            t.v_lo = (float)(1.0 / S_hi);
            t.v_hi = (float)(1.0 / S_lo);
            t.nwin = u2 ? -1 : n2;
            t.cflag = 0;
            t.rej = 0u;
            t.total = 0;
            dl.ct = t;
            HL.nsel = 0;
        }
        __syncthreads();
        for (int t = tid; t < NT_; t += ND)
            if (HL.tmax[t] >= th) {
                const int sl = atomicAdd(&HL.nsel, 1);
                HL.sel[t] = sl;
                HL.stile[sl] = t;
            }
    }
    if (tid == 0) {
        HL.urej = 0u;
        dl.dl.sh[3] = 0;
    }
    __syncthreads();
    const int nsel = HL.nsel;
    // the largest maximum of the tiles not read back
    uint32_t myrej = 0u;
    for (int t = tid; t < NT_; t += ND)
        if (HL.sel[t] < 0) myrej = max(myrej, HL.tmax[t]);
    // the selected tiles' history bits (sample.c:119-120)
    for (int i = tid; i < nsel * (HT / 32); i += ND) (&HL.selbits[0][0])[i] = 0u;
    __syncthreads();
    const double rinv = 1.0 / (double)rp;
    if (pen) {
        for (int j = tid; j < len; j += ND) {
            const int id = j == tid ? hid0 : ring[qs_ring_slot(cap, head, j)];
            if (id >= 0 && id < V) {
                const int s = HL.sel[id / HT];
                if (s >= 0) atomicOr(&HL.selbits[s][(id % HT) >> 5], 1u << (id & 31));
            }
        }
        __syncthreads();
    }
    // the selected tiles' penalised logits, GR float4s a thread in flight (a flat index over
    // (slot, float4 of the tile): 32 lanes a tile, one round trip for up to ND * GR / 32
    // tiles): a greedy row's first max; a sampled row's logits at or above th as candidates
    // (NaN never), the others raising the rejected bound
    static_assert(HT == 128, "a tile is 32 lanes x 4 logits");
    constexpr int QT = HT / 4, GR = 16;
    const int nq = nsel * QT;
    const float thf = key2f(th);
    if (!greedy) myrej = max(myrej, th - 1u);            // (th > KEY_NEG_INF: a key below it)
    float bv = -INFINITY;
    int bi = -1;
    // rounds of GR float4s a thread, loaded together; a sampled row looks only at the
    // float4s reaching th (the penalty only lowers a logit, a float below thf has a key below
    // th, and with a NaN the test fails and the float4 is looked at): what it leaves is
    // bounded by th - 1, the rejected bound taken above
    auto gather = [&](auto greedy_c) {
        constexpr bool G = decltype(greedy_c)::value;
        for (int base = 0; base < nq; base += ND * GR) {
            float4 vv[GR];
            uint32_t tk[GR], kv[GR][4];                   // candidates taken, their keys
#pragma unroll
            for (int u = 0; u < GR; ++u) {
                tk[u] = 0u;
                vv[u] = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
                const int i = base + u * ND + tid;
                if (i < nq) {
                    const int c = HL.stile[i / QT] * HT + (i % QT) * 4;
                    if (c < V) vv[u] = *(const float4 *)(x + c);
                }
            }
#pragma unroll
            for (int u = 0; u < GR; ++u) {
                if (base + u * ND >= nq) break;           // (uniform)
                if (!G && !__ballot(!(max4(vv[u]) < thf))) continue;
                const int i = base + u * ND + tid, sl = i / QT, q = i % QT;
                const bool ok = i < nq;
                const int c = ok ? HL.stile[sl] * HT + q * 4 : V;
                float w[4] = {vv[u].x, vv[u].y, vv[u].z, vv[u].w};
                const uint32_t bits = ok ? (HL.selbits[sl][q >> 3] >> ((q * 4) & 31)) & 0xFu : 0u;
                if (__ballot(bits != 0u)) {               // (ids past V are never marked)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if ((bits >> e) & 1u) w[e] = penalise_r(w[e], rp, rinv);
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool live = c + e < V && w[e] == w[e];
                    if constexpr (G) {
                        if (live) best_combine(bv, bi, w[e], c + e);
                    } else {
                        kv[u][e] = f2key(w[e]);
                        tk[u] |= (live && kv[u][e] >= th ? 1u : 0u) << e;
                    }
                }
            }
            if constexpr (!G) {
                // this thread's candidates at consecutive positions: one LDS atomic a
                // wavefront
                int cnt = 0;
#pragma unroll
                for (int u = 0; u < GR; ++u) cnt += __builtin_popcount(tk[u]);
                const int incl = wave_scan(cnt);
                const int wtot = __builtin_amdgcn_readlane(incl, 63);
                if (wtot == 0) continue;                  // (uniform)
                int at = 0;
                if (lane == 63) at = atomicAdd(&dl.dl.sh[3], wtot);
                int pos = __shfl(at, 63, 64) + incl - cnt;
#pragma unroll
                for (int u = 0; u < GR; ++u) {
                    if (!tk[u]) continue;
                    const int i = base + u * ND + tid;
                    const int c = HL.stile[i / QT] * HT + (i % QT) * 4;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (((tk[u] >> e) & 1u) && pos < FCAP) {
                            dl.keys[pos] = kv[u][e];
                            dl.ids[pos] = c + e;
                        }
                        pos += (tk[u] >> e) & 1u;
                    }
                }
            }
        }
    };
    if (greedy) gather(std::true_type{});
    else gather(std::false_type{});
    if (greedy) {
        block_best(bv, bi, dl);
        if (tid == 0) record_greedy(row, P, bv, bi, maxl, x[0], st, pa.out, pa.diag);
        return;
    }
    myrej = wave_max_u(myrej);
    if (lane == 0) atomicMax(&HL.urej, myrej);
    __syncthreads();
    CertTotals t = dl.ct;
    t.total = dl.dl.sh[3];
    t.rej = HL.urej;
    t.cflag = t.total > FCAP;
    __syncthreads();
    if (tid == 0) dl.ct = t;
    int status;
    if (!(isfinite(msc) && fabsf(msc) < CERT_MSC_MAX)) {
        status = CF_MSC;
    } else if (K <= 64 && t.total <= WAVE_CAND) {
        // one wavefront decides (the row kernel's decision); the others take its status
        if (wv == 0) {
            const int s0 = cert_row_wave(row, P, t, dl.keys, dl.ids, dl.srt, dl.dl.tab, st,
                                         pa.out, pa.diag, hist);
            if (lane == 0) dl.dl.sh[7] = s0;
        }
        __syncthreads();
        status = dl.dl.sh[7];
    } else {
        status = cert_row_block<ND>(row, P, t, dl.keys, dl.ids, dl.srt, dl.dl, st, pa.out,
                                    pa.diag, hist);
    }
    if (status == 0) return;
    __syncthreads();
    exact_row(pa, row, P, t, dl, hist, status);
}

}  // namespace

size_t qs_head_packed_elems(int n_embd, int n_vocab) {
    return (size_t)((n_vocab + HT - 1) / HT) * HT * (size_t)n_embd;
}

int qs_head_pack_launch(const void *d_weight, int n_embd, int n_vocab, void *d_packed,
                        hipStream_t stream) {
    const int ntiles = (n_vocab + HT - 1) / HT;
    const int64_t pieces = (int64_t)qs_head_packed_elems(n_embd, n_vocab) / 8;
    const int64_t want = (pieces + 255) / 256;
    const unsigned grid = (unsigned)(want < 65536 ? want : 65536);
    hipLaunchKernelGGL(k_head_pack, dim3(grid), dim3(256), 0, stream,
                       (const uint16_t *)d_weight, n_embd, n_vocab, ntiles, (uint16_t *)d_packed);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        qs_set_error("head pack launch: %s", hipGetErrorString(e));
        return QS_EDEVICE;
    }
    return 0;
}

int qs_head_prep_launch(int n_rows, int n_vocab, const RowState &st, uint32_t *hbits,
                        hipStream_t stream) {
    HeadArgs a;
    memset(&a, 0, sizeof a);
    a.n_rows = n_rows;
    a.V = n_vocab;
    a.hb = hbits;
    a.st = st;
    hipLaunchKernelGGL(k_head_prep, dim3((unsigned)n_rows), dim3(256), 0, stream, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        qs_set_error("output layer history bitmap launch: %s", hipGetErrorString(e));
        return QS_EDEVICE;
    }
    return 0;
}

int qs_head_decide_launch(float *d_logits, int n_rows, int n_vocab, const RowState &st,
                          const Scratch &sc, HeadRec *rec, int32_t *out, qs_pick_diag *diag,
                          hipStream_t stream) {
    HeadArgs a;
    memset(&a, 0, sizeof a);
    a.n_rows = n_rows;
    a.V = n_vocab;
    a.ntiles = (n_vocab + HT - 1) / HT;
    a.logits = d_logits;
    a.rec = rec;
    a.records = 1;
    a.st = st;
    PartArgs pa;
    pa.logits = d_logits;
    pa.stride = n_vocab;
    pa.vocab = n_vocab;
    pa.n_rows = n_rows;
    pa.parts = 1;
    pa.part_len = n_vocab;
    pa.xcd_map = 0;
    pa.st = st;
    pa.sc = sc;
    pa.out = out;
    pa.diag = diag;
    hipLaunchKernelGGL(k_head_decide, dim3((unsigned)n_rows), dim3(ND), 0, stream, a, pa);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        qs_set_error("output layer decision launch: %s", hipGetErrorString(e));
        return QS_EDEVICE;
    }
    return 0;
}

int qs_head_launch(const void *d_hidden, const void *d_weight, int n_embd, int n_rows,
                   int n_vocab, float *d_logits, const RowState &st, const Scratch &sc,
                   HeadRec *rec, uint32_t *hbits, int32_t *out, qs_pick_diag *diag,
                   hipStream_t stream) {
    HeadArgs a;
    a.h = (const uint16_t *)d_hidden;
    a.w = (const uint16_t *)d_weight;
    a.E = n_embd;
    a.n_rows = n_rows;
    a.V = n_vocab;
    a.ntiles = (n_vocab + HT - 1) / HT;
    a.logits = d_logits;
    a.hb = hbits;
    a.rec = rec;
    a.records = out != nullptr;
    a.st = st;
    if (a.records) {
        hipLaunchKernelGGL(k_head_prep, dim3((unsigned)n_rows), dim3(256), 0, stream, a);
        const hipError_t ep = hipGetLastError();
        if (ep != hipSuccess) {
            qs_set_error("head history bitmap launch: %s", hipGetErrorString(ep));
            return QS_EDEVICE;
        }
    }
    // the smallest row capacity that holds the batch (a deeper ring for fewer rows)
    if (n_rows <= 64)
        hipLaunchKernelGGL(k_head64, dim3((unsigned)a.ntiles), dim3(HNT), 0, stream, a);
    else if (n_rows <= 128)
        hipLaunchKernelGGL(k_head128, dim3((unsigned)a.ntiles), dim3(HNT), 0, stream, a);
    else
        hipLaunchKernelGGL(k_head256, dim3((unsigned)a.ntiles), dim3(HNT), 0, stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        qs_set_error("head launch: %s", hipGetErrorString(e));
        return e == hipErrorOutOfMemory ? QS_ENOMEM : QS_EDEVICE;
    }
    if (!a.records) return 0;
    PartArgs pa;
    pa.logits = d_logits;
    pa.stride = n_vocab;
    pa.vocab = n_vocab;
    pa.n_rows = n_rows;
    pa.parts = 1;
    pa.part_len = n_vocab;
    pa.xcd_map = 0;
    pa.st = st;
    pa.sc = sc;
    pa.out = out;
    pa.diag = diag;
    hipLaunchKernelGGL(k_head_decide, dim3((unsigned)n_rows), dim3(ND), 0, stream, a, pa);
    e = hipGetLastError();
    if (e != hipSuccess) {
        qs_set_error("head decision launch: %s", hipGetErrorString(e));
        return QS_EDEVICE;
    }
    return 0;
}
