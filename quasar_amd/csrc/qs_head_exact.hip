// qs_head_exact.hip - the output layer at the reference's own arithmetic, for the batches of
// a few rows that decoding one sequence at a time produces: logits[b][v] = the float sum
// over k ascending of w[v][k] * xn[b][k], a product then a sum (forward_cpu.c:140-147), with
// w[v] dequantized from its GGUF row exactly as quasar_dequant_row does (quant.c:8-27, 62-70,
// 106-130: F32, F16, Q8_0, Q6_K).  One thread per vocabulary row keeps the reference's order,
// so every logit equals the reference's bit for bit (a NaN's payload aside).
//
// k_exact_pack (once, at model load): the GGUF rows into an interleaved layout, so a
// wavefront's 64 rows read 1 KB contiguous per load: stream A holds 16-byte units (F32: 4
// weights, F16: 8, Q8_0: a block's 32 quants in two units, Q6_K: a super-block's low bits,
// high bits and scales in 13 units), unit u of row 64 g + l at [g][u][l]; stream D the
// binary16 block scales (Q8_0, Q6_K) at [g][block][l].  Rows past the vocabulary are zero.
//
// k_head_exact<type, rows>, 256 threads (256 vocabulary rows, two tiles of 128): the pick's
// hidden rows copied into LDS, the loop over the row's blocks in k order (four elements of a
// hidden row per broadcast read), then the logits written; with records (the fused
// pick), per (hidden row, tile of 128): the repeat penalty (the rows' history ids marked in
// LDS by each workgroup for its vocabulary rows), the penalised max and min keys, the NaN count and the certified sums
// against an integer exponent base, exactly what the other output layer's epilogue
// records, so the same decision kernel (k_head_decide) finishes the pick.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "../../include/quasar_sampler.h"
#include "qs_cert.h"
#include "qs_device.h"
#include "qs_internal.h"
#include "qs_launch.h"

using namespace qs;

namespace {

constexpr int XR = QS_HEAD_EXACT_MAX_ROWS;   // hidden rows per pick at most
constexpr int XNT = 256;                     // threads (vocabulary rows) per workgroup
static_assert(XNT == 2 * QS_HEAD_TILE, "a workgroup covers two tiles");

// Units of stream A and scales of stream D per row, for the four types (0: not taken).
struct XFmt {
    int ua, nd;
};
__host__ __device__ inline XFmt xfmt(int wtype, int E) {
    switch (wtype) {
        case QS_WTYPE_F32: return {E / 4, 0};
        case QS_WTYPE_F16: return {E / 8, 0};
        case QS_WTYPE_Q8_0: return {E / 32 * 2, E / 32};
        case QS_WTYPE_Q6_K: return {E / 256 * 13, E / 256};
        default: return {0, 0};
    }
}
// Bytes of one GGUF row of E elements.
__host__ __device__ inline int64_t xrow_bytes(int wtype, int E) {
    switch (wtype) {
        case QS_WTYPE_F32: return 4 * (int64_t)E;
        case QS_WTYPE_F16: return 2 * (int64_t)E;
        case QS_WTYPE_Q8_0: return (int64_t)E / 32 * 34;
        case QS_WTYPE_Q6_K: return (int64_t)E / 256 * 210;
        default: return 0;
    }
}

// One thread per 16-byte unit of stream A, then per scale of stream D.
__global__ void __launch_bounds__(256) k_exact_pack(const uint8_t *w, int wtype, int E, int V,
                                                    int groups, uint4 *pa, uint16_t *pd) {
    const XFmt f = xfmt(wtype, E);
    const int64_t rb = xrow_bytes(wtype, E);
    const int64_t na = (int64_t)groups * f.ua * 64, nd = (int64_t)groups * f.nd * 64;
    for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < na + nd;
         q += (int64_t)gridDim.x * 256) {
        if (q < na) {
            const int l = (int)(q & 63), u = (int)((q >> 6) % f.ua);
            const int64_t g = (q >> 6) / f.ua, r = g * 64 + l;
            int64_t off;                             // the unit's first byte in the row
            if (wtype == QS_WTYPE_Q8_0) {
                off = (int64_t)(u >> 1) * 34 + 2 + 16 * (u & 1);
            } else if (wtype == QS_WTYPE_Q6_K) {
                const int j = u / 13, v = u - j * 13;
                off = (int64_t)j * 210 + (v < 8 ? 16 * v : v < 12 ? 128 + 16 * (v - 8) : 192);
            } else {
                off = 16 * (int64_t)u;
            }
            uint32_t d[4] = {0u, 0u, 0u, 0u};
            if (r < V) {
                const uint8_t *s = w + r * rb + off;
                for (int i = 0; i < 16; ++i) d[i >> 2] |= (uint32_t)s[i] << (8 * (i & 3));
                // Q6_K's high bits with the upper bit of each pair flipped: the pair is then
                // the top of q ^ 32, the six-bit two's complement of q - 32
                if (wtype == QS_WTYPE_Q6_K && u % 13 >= 8 && u % 13 < 12)
                    for (int i = 0; i < 4; ++i) d[i] ^= 0xAAAAAAAAu;
            }
            pa[q] = make_uint4(d[0], d[1], d[2], d[3]);
        } else {
            const int64_t p = q - na;
            const int l = (int)(p & 63), j = (int)((p >> 6) % f.nd);
            const int64_t g = (p >> 6) / f.nd, r = g * 64 + l;
            uint16_t v = 0;
            if (r < V) {
                const uint8_t *s =
                    w + r * rb + (wtype == QS_WTYPE_Q8_0 ? (int64_t)j * 34 : (int64_t)j * 210 + 208);
                v = (uint16_t)(s[0] | (s[1] << 8));
            }
            pd[p] = v;
        }
    }
}

struct ExactArgs {
    const uint4 *pa;                    // stream A (k_exact_pack)
    const uint16_t *pd;                 // stream D
    const float *x;                     // [n_rows][E] hidden rows (xn)
    int E, V, n_rows, ntiles, ua, nd;
    float *logits;                      // [n_rows][V]
    HeadRec *rec;                       // [n_rows][ntiles]; null: the logits only
    RowState st;
};

// binary16 bits to float: exact for every non-NaN value, as quant.c:8-27.
__device__ __forceinline__ float half_f(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// Four consecutive elements k .. k + 3 (k a multiple of 4): acc[b] = acc[b] + y[e] * x[b][k
// + e] in e order for the pick's rows (forward_cpu.c:146, a product then a sum), x from the
// workgroup's copy in LDS (every lane reads the same address: one broadcast read).
template <int NB>
__device__ __forceinline__ void mac4(float (&acc)[NB], const float (&y)[4], const float *xs,
                                     int E, int k) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const float4 x4 = *(const float4 *)(xs + b * E + k);
        acc[b] = acc[b] + y[0] * x4.x;
        acc[b] = acc[b] + y[1] * x4.y;
        acc[b] = acc[b] + y[2] * x4.z;
        acc[b] = acc[b] + y[3] * x4.w;
    }
}

// The row's logits for the pick's NB hidden rows, in k order.
template <int WT, int NB>
__device__ __forceinline__ void exact_row(const ExactArgs &a, const float *xs, int g, int lane,
                                          float (&acc)[NB]) {
    const int E = a.E;
    const uint4 *pa = a.pa + (int64_t)g * a.ua * 64 + lane;
    const uint16_t *pd = a.pd + (int64_t)g * a.nd * 64 + lane;
    if constexpr (WT == QS_WTYPE_F32) {
        for (int u = 0; u < a.ua; u += 4) {
            uint4 w[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = pa[(int64_t)(u + i) * 64];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float y[4] = {__uint_as_float(w[i].x), __uint_as_float(w[i].y),
                                    __uint_as_float(w[i].z), __uint_as_float(w[i].w)};
                mac4<NB>(acc, y, xs, E, 4 * (u + i));
            }
        }
    } else if constexpr (WT == QS_WTYPE_F16) {
        for (int u = 0; u < a.ua; u += 2) {
            uint4 w[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) w[i] = pa[(int64_t)(u + i) * 64];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint32_t v[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
#pragma unroll
                for (int hq = 0; hq < 2; ++hq) {
                    const float y[4] = {half_f(v[2 * hq]), half_f(v[2 * hq] >> 16),
                                        half_f(v[2 * hq + 1]), half_f(v[2 * hq + 1] >> 16)};
                    mac4<NB>(acc, y, xs, E, 8 * (u + i) + 4 * hq);
                }
            }
        }
    } else if constexpr (WT == QS_WTYPE_Q8_0) {
        for (int j = 0; j < a.nd; ++j) {            // quant.c:62-70: y = d * q
            const uint4 q0 = pa[(int64_t)(2 * j) * 64], q1 = pa[(int64_t)(2 * j + 1) * 64];
            const float d = half_f(pd[(int64_t)j * 64]);
            const uint32_t v[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
            for (int e4 = 0; e4 < 8; ++e4) {
                float y[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) y[e] = d * (float)(int)(int8_t)(v[e4] >> (8 * e));
                mac4<NB>(acc, y, xs, E, 32 * j + 4 * e4);
            }
        }
    } else {
        static_assert(WT == QS_WTYPE_Q6_K, "the four types");
        for (int j = 0; j < a.nd; ++j) {            // quant.c:106-130: y = (d * sc) * (q - 32)
            uint32_t ql[32], qh[16], sc[4];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint4 t = pa[(int64_t)(13 * j + i) * 64];
                ql[4 * i] = t.x;
                ql[4 * i + 1] = t.y;
                ql[4 * i + 2] = t.z;
                ql[4 * i + 3] = t.w;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 t = pa[(int64_t)(13 * j + 8 + i) * 64];
                qh[4 * i] = t.x;
                qh[4 * i + 1] = t.y;
                qh[4 * i + 2] = t.z;
                qh[4 * i + 3] = t.w;
            }
            {
                const uint4 t = pa[(int64_t)(13 * j + 12) * 64];
                sc[0] = t.x;
                sc[1] = t.y;
                sc[2] = t.z;
                sc[3] = t.w;
            }
            // d / 4, exactly (|d| >= 2^-24 or zero, inf or NaN): y = (d sc) (q - 32) is taken
            // as (d sc / 4) (4 (q - 32)), the same product of the same rounded factor, with
            // 4 (q - 32) a signed byte built in place below
            const float d4 = 0.25f * half_f(pd[(int64_t)j * 64]);
            // element k = 256 j + 128 h + 32 qd + l: its low bits in quant byte
            // 64 h + 32 (qd & 1) + l (low nibble for qd < 2, high otherwise), its high bits
            // 2 qd .. 2 qd + 1 of byte 32 h + l (flipped as packed), its scale
            // sc[8 h + l / 16 + 2 qd]
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
#pragma unroll
                    for (int l4 = 0; l4 < 8; ++l4) {
                        // four bytes of 4 (q - 32): q ^ 32 (six-bit two's complement of
                        // q - 32) in bits 2..7, the nibble in 2..5, the flipped pair in 6..7
                        const uint32_t lw = ql[16 * h + 8 * (qd & 1) + l4];
                        const uint32_t ls = qd < 2 ? lw << 2 : lw >> 2;
                        const uint32_t hs = (qh[8 * h + l4] << (6 - 2 * qd)) & 0xC0C0C0C0u;
                        const uint32_t t4 = (ls & 0x3C3C3C3Cu) | hs;
                        const int s = 8 * h + (l4 >> 2) + 2 * qd;
                        const float ds4 = d4 * (float)(int)(int8_t)(sc[s >> 2] >> (8 * (s & 3)));
                        float y[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) y[e] = ds4 * (float)(int)(int8_t)(t4 >> (8 * e));
                        mac4<NB>(acc, y, xs, E, 256 * j + 128 * h + 32 * qd + 4 * l4);
                    }
                }
            }
        }
    }
}

// The records' per-wavefront partials (in the LDS the hidden rows held).
struct XEpi {
    double s[XR][XNT / 64], t[XR][XNT / 64];
    uint32_t mx[XR][XNT / 64], mn[XR][XNT / 64];
    int nan[XR][XNT / 64];
};

template <int WT, int NB>
__global__ void __launch_bounds__(XNT) k_head_exact(ExactArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = blockIdx.x * XNT + tid;          // this thread's vocabulary row
    const int g = blockIdx.x * (XNT / 64) + wv;    // its group of 64 in the packed layout
    extern __shared__ float4 xs4[];                // the pick's hidden rows, n_rows x E
    __shared__ uint32_t s_hb[XNT];                 // bit b: the row in row b's history
    for (int i = tid; i < a.n_rows * a.E / 4; i += XNT) xs4[i] = ((const float4 *)a.x)[i];
    s_hb[tid] = 0u;
    __syncthreads();
    if (a.rec) {
        // sample.c:118-120: the history ids of each pick row that fall in this workgroup's
        // vocabulary rows (duplicates set the same bit); read by the records below
        const int r0 = blockIdx.x * XNT;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const qs_row_param P = row_param(a.st, b);
            const int cap = P.ring_cap;
            int len, head;
            ring_pos(a.st, b, cap, len, head);
            if (!(P.repeat_penalty > 1.0f) || len <= 0 || cap <= 0) continue;
            const int32_t *ring = a.st.ring + (int64_t)b * a.st.ring_stride;
            for (int j = tid; j < len; j += XNT) {
                const int id = ring[qs_ring_slot(cap, head, j)];
                if (id >= r0 && id < r0 + XNT && id < a.V) atomicOr(&s_hb[id - r0], 1u << b);
            }
        }
    }
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
    if (g * 64 < a.V)                              // (uniform) the group is packed
        exact_row<WT, NB>(a, (const float *)xs4, g, lane, acc);
    const int V = a.V;
#pragma unroll
    for (int b = 0; b < NB; ++b)
        if (r < V) a.logits[(int64_t)b * V + r] = acc[b];
    if (!a.rec) return;
    // the sampler's first pass over each (row, tile of 128): tile tid / 128 of the workgroup,
    // its partials in the LDS the hidden rows held
    __syncthreads();
    XEpi &ep = *(XEpi *)xs4;
    auto &s_mx = ep.mx;
    auto &s_mn = ep.mn;
    auto &s_nan = ep.nan;
    auto &s_s = ep.s;
    auto &s_t = ep.t;
    const uint32_t hw = s_hb[tid];                 // bit b: id r in row b's history
    float w[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        w[b] = -INFINITY;
        if (r < V) {
            const qs_row_param P = row_param(a.st, b);
            const float rp = P.repeat_penalty;
            w[b] = (hw >> b) & 1u ? penalise_r(acc[b], rp, 1.0 / (double)rp) : acc[b];
        }
        const bool nan = w[b] != w[b];
        const float mx = nan ? -INFINITY : w[b];
        const float mn = (nan || r >= V) ? INFINITY : w[b];
        const uint32_t mk = wave_max_u(f2key(mx));
        const uint32_t nk = wave_min_u(mn != INFINITY ? f2key(mn) : 0xFFFFFFFFu);
        const int nc = wave_sum_i(nan ? 1 : 0);
        if (lane == 0) {
            s_mx[b][wv] = mk;
            s_mn[b][wv] = nk;
            s_nan[b][wv] = nc;
        }
    }
    __syncthreads();
    const int t2 = wv >> 1;                        // the tile within the workgroup
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const qs_row_param P = row_param(a.st, b);
        const uint32_t maxk = max(s_mx[b][2 * t2], s_mx[b][2 * t2 + 1]);
        float cbase = 0.0f;
        double S = 0.0, T = 0.0;
        const float inv_t = P.inv_t;
        const float Mw = key2f(maxk > KEY_NEG_INF ? maxk : KEY_NEG_INF) * inv_t;
        if (!row_greedy(P) && Mw > -INFINITY && Mw < INFINITY) {   // (uniform per tile)
            cbase = cert_cbase(Mw);
            // sum4's terms, one element a thread
            const float sc = w[b] * inv_t;
            const float t = fmaxf(__builtin_fmaf(sc, CERT_L, -cbase), T_GUARD);
            const float e = __builtin_amdgcn_exp2f(t);
            S = wave_sum_d((double)e);
            T = wave_sum_d((double)(e * t));
        }
        if (lane == 0) {
            s_s[b][wv] = S;
            s_t[b][wv] = T;
        }
        (void)cbase;
    }
    __syncthreads();
    const int tile = blockIdx.x * 2 + t2;
    if ((tid & 127) == 0 && tile < a.ntiles) {
        for (int b = 0; b < NB; ++b) {
            const qs_row_param P = row_param(a.st, b);
            const uint32_t maxk = max(s_mx[b][2 * t2], s_mx[b][2 * t2 + 1]);
            const float Mw = key2f(maxk > KEY_NEG_INF ? maxk : KEY_NEG_INF) * P.inv_t;
            HeadRec h;
            h.maxk = maxk > KEY_NEG_INF ? maxk : KEY_NEG_INF;
            h.mink = min(s_mn[b][2 * t2], s_mn[b][2 * t2 + 1]);
            h.nan = s_nan[b][2 * t2] + s_nan[b][2 * t2 + 1];
            const bool sums = !row_greedy(P) && Mw > -INFINITY && Mw < INFINITY;
            h.c = sums ? cert_cbase(Mw) : 0.0f;
            h.sum = s_s[b][2 * t2] + s_s[b][2 * t2 + 1];
            h.term = -(s_t[b][2 * t2] + s_t[b][2 * t2 + 1]);
            a.rec[(int64_t)b * a.ntiles + tile] = h;
        }
    }
}

template <int WT>
hipError_t launch_exact(const ExactArgs &a, int nb, hipStream_t s) {
    const dim3 grid((unsigned)((a.V + XNT - 1) / XNT)), blk(XNT);
    const size_t lds = std::max(sizeof(float) * (size_t)a.n_rows * a.E, sizeof(XEpi));
    static_assert(XR == 8, "one instance per row count");
    switch (nb) {
        case 1: hipLaunchKernelGGL((k_head_exact<WT, 1>), grid, blk, lds, s, a); break;
        case 2: hipLaunchKernelGGL((k_head_exact<WT, 2>), grid, blk, lds, s, a); break;
        case 3: hipLaunchKernelGGL((k_head_exact<WT, 3>), grid, blk, lds, s, a); break;
        case 4: hipLaunchKernelGGL((k_head_exact<WT, 4>), grid, blk, lds, s, a); break;
        case 5: hipLaunchKernelGGL((k_head_exact<WT, 5>), grid, blk, lds, s, a); break;
        case 6: hipLaunchKernelGGL((k_head_exact<WT, 6>), grid, blk, lds, s, a); break;
        case 7: hipLaunchKernelGGL((k_head_exact<WT, 7>), grid, blk, lds, s, a); break;
        default: hipLaunchKernelGGL((k_head_exact<WT, 8>), grid, blk, lds, s, a); break;
    }
    return hipGetLastError();
}

}  // namespace

int qs_head_exact_shape_ok(int wtype, int n_embd) {
    if (n_embd < 16 || n_embd > QS_HEAD_EXACT_MAX_EMBD) return 0;
    switch (wtype) {
        case QS_WTYPE_F32: return n_embd % 16 == 0;
        case QS_WTYPE_F16: return n_embd % 16 == 0;
        case QS_WTYPE_Q8_0: return n_embd % 32 == 0;
        case QS_WTYPE_Q6_K: return n_embd % 256 == 0;
        default: return 0;
    }
}

size_t qs_head_exact_bytes(int wtype, int n_embd, int n_vocab) {
    if (!qs_head_exact_shape_ok(wtype, n_embd) || n_vocab < 1) return 0;
    const XFmt f = xfmt(wtype, n_embd);
    const size_t groups = ((size_t)n_vocab + 63) / 64;
    const size_t a = groups * f.ua * 64 * 16, d = groups * f.nd * 64 * 2;
    return a + (d + 15) / 16 * 16;
}

int qs_head_exact_pack_launch(const void *d_weight, int wtype, int n_embd, int n_vocab,
                              void *d_packed, hipStream_t stream) {
    const XFmt f = xfmt(wtype, n_embd);
    const int groups = (n_vocab + 63) / 64;
    uint4 *pa = (uint4 *)d_packed;
    uint16_t *pd = (uint16_t *)(pa + (size_t)groups * f.ua * 64);
    hipLaunchKernelGGL(k_exact_pack, dim3(4096), dim3(256), 0, stream, (const uint8_t *)d_weight,
                       wtype, n_embd, n_vocab, groups, pa, pd);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        qs_set_error("exact output layer pack launch: %s", hipGetErrorString(e));
        return QS_EDEVICE;
    }
    return 0;
}

int qs_head_exact_launch(const void *d_packed, int wtype, const float *d_xn, int n_embd,
                         int n_rows, int n_vocab, float *d_logits, const RowState &st,
                         HeadRec *rec, hipStream_t stream) {
    const XFmt f = xfmt(wtype, n_embd);
    const int groups = (n_vocab + 63) / 64;
    ExactArgs a;
    a.pa = (const uint4 *)d_packed;
    a.pd = (const uint16_t *)(a.pa + (size_t)groups * f.ua * 64);
    a.x = d_xn;
    a.E = n_embd;
    a.V = n_vocab;
    a.n_rows = n_rows;
    a.ntiles = (n_vocab + QS_HEAD_TILE - 1) / QS_HEAD_TILE;
    a.ua = f.ua;
    a.nd = f.nd;
    a.logits = d_logits;
    a.rec = rec;
    a.st = st;
    hipError_t e;
    switch (wtype) {
        case QS_WTYPE_F32: e = launch_exact<QS_WTYPE_F32>(a, n_rows, stream); break;
        case QS_WTYPE_F16: e = launch_exact<QS_WTYPE_F16>(a, n_rows, stream); break;
        case QS_WTYPE_Q8_0: e = launch_exact<QS_WTYPE_Q8_0>(a, n_rows, stream); break;
        default: e = launch_exact<QS_WTYPE_Q6_K>(a, n_rows, stream); break;
    }
    if (e != hipSuccess) {
        qs_set_error("exact output layer launch: %s", hipGetErrorString(e));
        return e == hipErrorOutOfMemory ? QS_ENOMEM : QS_EDEVICE;
    }
    return 0;
}
