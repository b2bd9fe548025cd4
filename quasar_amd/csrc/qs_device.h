// qs_device.h - device code shared by the sampler kernels (included by .hip files only).
//
// Conventions: a row is one vector of n_vocab penalised logits; "key" is the
// order-preserving u32 image of a float (f2key); candidates are kept as keys so any
// threshold is a plain integer compare.  Every routine here reproduces a step of the
// reference sampler (sample.c) bit for bit, or is a block-level primitive (select, sort)
// whose result does not depend on thread scheduling.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>

#include "../../include/quasar_sampler.h"
#include "qs_expf.h"
#include "qs_internal.h"
#include "qs_ring.h"

namespace qs {

// Timeline build (-DQS_TIMELINE): QS_TL_HOOK(e) records the 100 MHz clock at step e (< 16)
// of the calling workgroup's row decision (first thread; workgroups below 4096), one copy
// per translation unit (read back by quasar_amd/timeline.py).  Empty otherwise.
#ifdef QS_TIMELINE
static __device__ uint64_t g_tl_hook[4096 * 16];
#define QS_TL_HOOK(e)                                                                         \
    do {                                                                                      \
        if (threadIdx.x == 0 && blockIdx.x < 4096)                                            \
            qs::g_tl_hook[blockIdx.x * 16 + (e)] = __builtin_amdgcn_s_memrealtime();          \
    } while (0)
#else
#define QS_TL_HOOK(e) ((void)0)
#endif

constexpr int K_MAX = 512;        // largest top-k decided from preselected candidates
constexpr int K_OFF = 64;         // candidates aimed for when top-k is off
constexpr int SORT_CAP = 2048;    // candidates the decision step sorts in LDS
constexpr int SPIN_LIMIT = 1 << 20;  // slot lock attempts before giving up (~0.5 s)

// ---- keys, lanes, reductions ---------------------------------------------------------------

// Order-preserving map of float bit patterns to unsigned keys (-0 sorts below +0; NaN
// with the sign bit clear sorts above +inf, so callers filter NaN by float compares).
__device__ __forceinline__ uint32_t f2key(float f) {
    uint32_t b = __float_as_uint(f);
    return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}
constexpr uint32_t KEY_NEG_INF = 0x007FFFFFu;   // f2key(-inf)

__device__ __forceinline__ int lane_prefix(uint64_t m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Wavefront reductions in DPP moves only (no LDS instruction, so they do not queue behind
// other wavefronts' LDS traffic): pairs and quads by quad permutes, 8 and 16 lanes by the
// half-row and row mirrors, then row 1 (3) takes row 0's (2's) lane 15 and rows 2-3 take
// lane 31; lane 63 ends with the whole wavefront and is broadcast.  The combination order
// is fixed by lane positions, so double sums do not depend on timing.  Rows a broadcast
// does not write keep undefined values (a move into a fresh register, no copy first): only
// lane 63's result is read, and it never combines them.
template <int CTRL, int ROWS, typename T>
__device__ __forceinline__ T dpp_move(T x) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values");
    if constexpr (sizeof(T) == 4) {
        const int b = __builtin_bit_cast(int, x);
        return __builtin_bit_cast(T, __builtin_amdgcn_mov_dpp(b, CTRL, ROWS, 0xF, false));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, x);
        const int lo = (int)(uint32_t)u, hi = (int)(uint32_t)(u >> 32);
        const uint32_t rlo = (uint32_t)__builtin_amdgcn_mov_dpp(lo, CTRL, ROWS, 0xF, false);
        const uint32_t rhi = (uint32_t)__builtin_amdgcn_mov_dpp(hi, CTRL, ROWS, 0xF, false);
        return __builtin_bit_cast(T, ((uint64_t)rhi << 32) | rlo);
    }
}
template <typename T, typename F>
__device__ __forceinline__ T wave_reduce(T v, F &&op) {
    v = op(v, dpp_move<0xB1, 0xF>(v));      // quad_perm [1,0,3,2]
    v = op(v, dpp_move<0x4E, 0xF>(v));      // quad_perm [2,3,0,1]
    v = op(v, dpp_move<0x141, 0xF>(v));     // row_half_mirror
    v = op(v, dpp_move<0x140, 0xF>(v));     // row_mirror
    v = op(v, dpp_move<0x142, 0xA>(v));     // row_bcast:15 into rows 1 and 3
    v = op(v, dpp_move<0x143, 0xC>(v));     // row_bcast:31 into rows 2 and 3
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)u, 63);
        const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 63);
        return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
    }
}
__device__ __forceinline__ int wave_sum_i(int v) {
    return wave_reduce(v, [](int a, int b) { return a + b; });
}
__device__ __forceinline__ double wave_sum_d(double v) {
    return wave_reduce(v, [](double a, double b) { return a + b; });
}
__device__ __forceinline__ float wave_max_f(float v) {
    return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
    return wave_reduce(v, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
}
__device__ __forceinline__ uint32_t wave_min_u(uint32_t v) {
    return wave_reduce(v, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
}
__device__ __forceinline__ int wave_or_i(int v) {
    return wave_reduce(v, [](int a, int b) { return a | b; });
}

// The value of lane (lane ^ S), in VALU moves only: DPP for S = 1, 2 (quad permutes) and
// 8 (a rotation by 8 within each row of 16 lanes); for 4, the row shifts by 4 up and down
// and a select by lane bit 2; for 16 and 32, v_permlane16_swap / v_permlane32_swap (each
// lane receives the pair {v[lane & ~S], v[lane | S]}) and a select by lane bit.
template <int S>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
    const bool up = (threadIdx.x & S) != 0;
    if constexpr (S == 1) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
    else if constexpr (S == 2) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);
    else if constexpr (S == 8) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);
    else if constexpr (S == 4) {
        const uint32_t fwd = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x104, 0xF, 0xF, false);  // row_shl:4
        const uint32_t bwd = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);  // row_shr:4
        return up ? bwd : fwd;
    } else if constexpr (S == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return up ? p[0] : p[1];
    } else {
        static_assert(S == 32, "lane distances 1, 2, 4, 8, 16, 32");
        const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return up ? p[0] : p[1];
    }
}
template <int S>
__device__ __forceinline__ uint64_t xor_lane64(uint64_t v) {
    const uint32_t lo = xor_lane<S>((uint32_t)v), hi = xor_lane<S>((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// One compare-exchange step of a bitonic sort over the 64 lanes (descending overall).
template <int SIZE, int S>
__device__ __forceinline__ void bitonic_step(uint64_t &v, int lane) {
    const uint64_t o = xor_lane64<S>(v);
    const bool keep_max = ((lane & S) == 0) == ((lane & SIZE) == 0);
    v = keep_max ? (o > v ? o : v) : (o < v ? o : v);
}
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t v) {
    const int lane = threadIdx.x & 63;
    bitonic_step<2, 1>(v, lane);
    bitonic_step<4, 2>(v, lane);   bitonic_step<4, 1>(v, lane);
    bitonic_step<8, 4>(v, lane);   bitonic_step<8, 2>(v, lane);   bitonic_step<8, 1>(v, lane);
    bitonic_step<16, 8>(v, lane);  bitonic_step<16, 4>(v, lane);  bitonic_step<16, 2>(v, lane);
    bitonic_step<16, 1>(v, lane);
    bitonic_step<32, 16>(v, lane); bitonic_step<32, 8>(v, lane);  bitonic_step<32, 4>(v, lane);
    bitonic_step<32, 2>(v, lane);  bitonic_step<32, 1>(v, lane);
    bitonic_step<64, 32>(v, lane); bitonic_step<64, 16>(v, lane); bitonic_step<64, 8>(v, lane);
    bitonic_step<64, 4>(v, lane);  bitonic_step<64, 2>(v, lane);  bitonic_step<64, 1>(v, lane);
    return v;
}

__device__ __forceinline__ uint64_t lane_u64(uint64_t v, int i) {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, i);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), i);
    return ((uint64_t)hi << 32) | lo;
}

// The K-th largest of the keys a wavefront holds Q per lane (0: no key; keys are >= 1),
// ties kept above it, i.e. the largest th with at least K keys >= th; `total` keys are
// present.  Bit by bit from the highest bit where the largest and smallest keys differ
// (the bits above it are common to all), stopping once exactly K keys lie at or above the
// prefix: the K-th is then the least of them.  With total <= K, the least key.
template <int Q>
__device__ __forceinline__ uint32_t wave_kth(const uint32_t (&k)[Q], int K, int total) {
    uint32_t kmx = 0u, kmn = 0xFFFFFFFFu;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        kmx = k[q] > kmx ? k[q] : kmx;
        kmn = (k[q] != 0u && k[q] < kmn) ? k[q] : kmn;
    }
    kmx = wave_max_u(kmx);
    kmn = wave_min_u(kmn);
    if (kmx == kmn || total <= K) return kmn;
    int b = 31 - __builtin_clz(kmx ^ kmn);
    uint32_t th = kmx & ~((2u << b) - 1u);        // (2u << 31) wraps to 0: no common bits
    int cur = total;                              // keys at or above th
    for (; b >= 0 && cur != K; --b) {
        const uint32_t c = th | (1u << b);
        int cnt = 0;
#pragma unroll
        for (int q = 0; q < Q; ++q) cnt += __popcll(__ballot(k[q] >= c));
        if (cnt >= K) {
            th = c;
            cur = cnt;
        }
    }
    if (cur == K) {
        uint32_t mn = 0xFFFFFFFFu;
#pragma unroll
        for (int q = 0; q < Q; ++q)
            if (k[q] >= th) mn = k[q] < mn ? k[q] : mn;
        th = wave_min_u(mn);
    }
    return th;
}

// A threshold that keeps at least K and, where ties allow, at most `cap` of the keys a
// wavefront holds Q per lane (0: no key): the largest prefix th found bit by bit, as in
// wave_kth, with at least K keys >= th, stopping as soon as at most `cap` keys remain at
// or above it (all keys when `total` <= cap).  Every key among the K largest (ties kept)
// is at or above it.
template <int Q>
__device__ __forceinline__ uint32_t wave_bracket(const uint32_t (&k)[Q], int K, int cap, int total) {
    uint32_t kmx = 0u, kmn = 0xFFFFFFFFu;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        kmx = k[q] > kmx ? k[q] : kmx;
        kmn = (k[q] != 0u && k[q] < kmn) ? k[q] : kmn;
    }
    kmx = wave_max_u(kmx);
    kmn = wave_min_u(kmn);
    if (kmx == kmn || total <= cap) return kmn;
    int b = 31 - __builtin_clz(kmx ^ kmn);
    uint32_t th = kmx & ~((2u << b) - 1u);        // (2u << 31) wraps to 0: no common bits
    int cur = total;                              // keys at or above th
    for (; b >= 0 && cur > cap; --b) {
        const uint32_t c = th | (1u << b);
        int cnt = 0;
#pragma unroll
        for (int q = 0; q < Q; ++q) cnt += __popcll(__ballot(k[q] >= c));
        if (cnt >= K) {
            th = c;
            cur = cnt;
        }
    }
    return th;
}

// The same sort for 32-bit values.
template <int SIZE, int S>
__device__ __forceinline__ void bitonic_step_u32(uint32_t &v, int lane) {
    const uint32_t o = xor_lane<S>(v);
    const bool keep_max = ((lane & S) == 0) == ((lane & SIZE) == 0);
    v = keep_max ? (o > v ? o : v) : (o < v ? o : v);
}
__device__ __forceinline__ uint32_t wave_sort_desc_u32(uint32_t v) {
    const int lane = threadIdx.x & 63;
    bitonic_step_u32<2, 1>(v, lane);
    bitonic_step_u32<4, 2>(v, lane);   bitonic_step_u32<4, 1>(v, lane);
    bitonic_step_u32<8, 4>(v, lane);   bitonic_step_u32<8, 2>(v, lane);
    bitonic_step_u32<8, 1>(v, lane);
    bitonic_step_u32<16, 8>(v, lane);  bitonic_step_u32<16, 4>(v, lane);
    bitonic_step_u32<16, 2>(v, lane);  bitonic_step_u32<16, 1>(v, lane);
    bitonic_step_u32<32, 16>(v, lane); bitonic_step_u32<32, 8>(v, lane);
    bitonic_step_u32<32, 4>(v, lane);  bitonic_step_u32<32, 2>(v, lane);
    bitonic_step_u32<32, 1>(v, lane);
    bitonic_step_u32<64, 32>(v, lane); bitonic_step_u32<64, 16>(v, lane);
    bitonic_step_u32<64, 8>(v, lane);  bitonic_step_u32<64, 4>(v, lane);
    bitonic_step_u32<64, 2>(v, lane);  bitonic_step_u32<64, 1>(v, lane);
    return v;
}

// x from the lane a DPP control names, 0 where there is none (rows outside ROWS, lanes
// shifted in from outside the row).
template <int CTRL, int ROWS, typename T>
__device__ __forceinline__ T dpp_shift(T x) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values");
    if constexpr (sizeof(T) == 4) {
        const int b = __builtin_bit_cast(int, x);
        return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, b, CTRL, ROWS, 0xF, false));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, x);
        const uint32_t rlo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, ROWS, 0xF, false);
        const uint32_t rhi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, ROWS, 0xF, false);
        return __builtin_bit_cast(T, ((uint64_t)rhi << 32) | rlo);
    }
}
// Inclusive prefix sum over the lanes in DPP moves: shifts by 1, 2, 4 and 8 within each
// row of 16, then rows 1 and 3 add lane 15 of the row below, rows 2 and 3 lane 31.
template <typename T>
__device__ __forceinline__ T wave_scan(T v) {
    v += dpp_shift<0x111, 0xF>(v);          // row_shr:1
    v += dpp_shift<0x112, 0xF>(v);          // row_shr:2
    v += dpp_shift<0x114, 0xF>(v);          // row_shr:4
    v += dpp_shift<0x118, 0xF>(v);          // row_shr:8
    v += dpp_shift<0x142, 0xA>(v);          // row_bcast:15 into rows 1 and 3
    v += dpp_shift<0x143, 0xC>(v);          // row_bcast:31 into rows 2 and 3
    return v;
}
__device__ __forceinline__ double wave_scan_d(double v) { return wave_scan(v); }
// Three independent inclusive scans in the same fixed order as wave_scan, interleaved step
// by step (one chain's latency for the three).
__device__ __forceinline__ void wave_scan3(double &a, double &b, double &c) {
#define QS_SCAN3(CTRL, ROWS)                                                                  \
    {                                                                                         \
        const double xa = dpp_shift<CTRL, ROWS>(a), xb = dpp_shift<CTRL, ROWS>(b),            \
                     xc = dpp_shift<CTRL, ROWS>(c);                                           \
        a += xa;                                                                              \
        b += xb;                                                                              \
        c += xc;                                                                              \
    }
    QS_SCAN3(0x111, 0xF)
    QS_SCAN3(0x112, 0xF)
    QS_SCAN3(0x114, 0xF)
    QS_SCAN3(0x118, 0xF)
    QS_SCAN3(0x142, 0xA)
    QS_SCAN3(0x143, 0xC)
#undef QS_SCAN3
}

// Reductions over lanes 0-15 (quad permutes, the half-row and the row mirror): every one
// of lanes 0-15 ends with the combination of all sixteen, read from lane 0.
template <typename T, typename F>
__device__ __forceinline__ T lane16_reduce(T v, F &&op) {
    v = op(v, dpp_move<0xB1, 0xF>(v));
    v = op(v, dpp_move<0x4E, 0xF>(v));
    v = op(v, dpp_move<0x141, 0xF>(v));
    v = op(v, dpp_move<0x140, 0xF>(v));
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)u, 0);
        const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 0);
        return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
    }
}

// Reductions over lanes 0-7 (quad permutes, then the half-row mirror): every one of lanes
// 0-7 ends with the combination of all eight, read from lane 0.
template <typename T, typename F>
__device__ __forceinline__ T lane8_reduce(T v, F &&op) {
    v = op(v, dpp_move<0xB1, 0xF>(v));
    v = op(v, dpp_move<0x4E, 0xF>(v));
    v = op(v, dpp_move<0x141, 0xF>(v));
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)u, 0);
        const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 0);
        return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
    }
}

// (value desc, index asc) with index < 0 meaning "none": the greedy combine.
__device__ __forceinline__ void best_combine(float &v, int &i, float ov, int oi) {
    if (oi >= 0 && (i < 0 || ov > v || (ov == v && oi < i))) { v = ov; i = oi; }
}
__device__ __forceinline__ void wave_best(float &v, int &i) {
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const int oi = __shfl_xor(i, o, 64);
        best_combine(v, i, ov, oi);
    }
}

// ---- data shared between workgroups of one launch ----------------------------------------
//
// Loads and stores at device scope (sc1: coherent across the XCDs' L2 caches), ordered by
// waiting for the stores to complete before the relaxed counter update that announces
// them.  No L2 writeback or invalidation is issued, so the streaming loads of the other
// workgroups keep their cache lines.
template <typename T>
__device__ __forceinline__ void st_dev(T *p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ld_dev(const T *p) {
    return __hip_atomic_load(const_cast<T *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Every vector memory operation of the calling wavefront has completed.
__device__ __forceinline__ void stores_done() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
template <typename T>
__device__ __forceinline__ T add_dev(T *p, T v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- the reference's scalar steps ----------------------------------------------------------

// sample.c:124: a history logit is divided by the penalty when positive, multiplied
// otherwise (so -0, NaN and -inf are unchanged, +inf stays +inf).
__device__ __forceinline__ float penalise(float l, float rp) {
    return l > 0.0f ? l / rp : l * rp;
}

// penalise() without the divide: for l > 0, l / rp (rounded to float) equals
// (float)((double)l * rinv) with rinv = 1.0 / (double)rp.  The double product is within
// 2^-52 (relative) of the exact quotient q = l / rp, and q lies more than 2^-49 from every
// point halfway between two floats: with l = L 2^a, rp = B 2^c (L, B 24-bit integers) and
// m a midpoint at ulp 2^d, l - m rp is a nonzero multiple of 2^(c+d-1), so |q - m| / q >
// 2^-49 (in the subnormal range the absolute gap, 2^-174, exceeds the product's error, below
// 2^-178).  So both round to the same float.  Branch-free: no divide sequence per element.
__device__ __forceinline__ float penalise_r(float l, float rp, double rinv) {
    const float q = (float)((double)l * rinv);
    return l > 0.0f ? q : l * rp;
}

// sample.c:72-81: xorshift64, the xorshift64* output multiplier, top 53 bits.
__device__ __forceinline__ double rng_unit(uint64_t &st) {
    uint64_t x = st;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    st = x;
    return (double)((x * 0x2545F4914F6CDD1Dull) >> 11) * (1.0 / 9007199254740992.0);
}

// sample.c:83-92: append, or overwrite the oldest once the ring is full (qs_ring_put;
// `cap` is the row's clamped capacity, row_param).  With the row's history length and head
// already loaded (len, head).
__device__ __forceinline__ void ring_record_at(int32_t *ring, int32_t *hlen, int32_t *hhead,
                                               int cap, int id, int len, int head) {
    const int s = qs_ring_put(cap, &len, &head);
    if (s < 0) return;
    ring[s] = id;
    *hlen = len;
    *hhead = head;
}
__device__ __forceinline__ void ring_record(int32_t *ring, int32_t *hlen, int32_t *hhead,
                                            int cap, int id) {
    if (cap <= 0) return;
    ring_record_at(ring, hlen, hhead, cap, id, *hlen, *hhead);
}

__host__ __device__ __forceinline__ bool row_greedy(const qs_row_param &p) {
    return p.temperature <= 0.0f;      // sample.c:130 (a NaN temperature samples)
}

// Candidates the decision step aims to keep for a sampling row.  Any value is correct:
// the decision proves the preselection or hands the row to the full-window path.
__host__ __device__ __forceinline__ int row_ksel(const qs_row_param &p) {
    return p.top_k > 0 ? (p.top_k < K_MAX ? p.top_k : K_MAX) : K_OFF;
}

// ---- per-row device state and scratch ----------------------------------------------------

struct RowState {
    const qs_row_param *prm;
    uint64_t *rng;
    int32_t *ring;
    int32_t *hlen;
    int32_t *hhead;
    int ring_stride;
};

// A row's stored parameters with its ring capacity clamped to the ring's storage
// (qs_ring_cap): every kernel loads them through this.
__device__ __forceinline__ qs_row_param row_param(const RowState &st, int row) {
    qs_row_param P = st.prm[row];
    P.ring_cap = qs_ring_cap(P.ring_cap, st.ring, st.ring_stride);
    return P;
}
// A row's history length and head, clamped to `cap` (the row's clamped capacity).
__device__ __forceinline__ void ring_pos(const RowState &st, int row, int cap, int &len,
                                         int &head) {
    len = st.hlen[row];
    head = st.hhead[row];
    qs_ring_clamp(cap, &len, &head);
}

// One wavefront's results for one part in the streaming kernel (32 bytes).
struct WaveRec {
    double sum;           // its approximate numerators' sum
    float term;           // minus its sum of e * t
    uint32_t mink;        // its least non-NaN penalised logit (key; 0xFFFFFFFF: none)
    int32_t nan;          // its NaN count
    uint32_t maxk;        // the part's largest penalised logit (key)
    uint32_t rej;         // the part's bound on every logit not among its candidates (key)
    int32_t cnt;          // candidates it found (above the list capacity: overflowed)
};

struct Scratch {
    float *smax;          // [rows*S] slice max of penalised logits
    float *bestv;         // [rows*S] greedy: slice max value
    int32_t *besti;       // [rows*S] greedy: its first index (-1: none)
    uint32_t *sth;        // [rows*S] slice candidate threshold (key)
    uint32_t *ckey;       // [rows*S*ccap] candidate keys
    int32_t *cid;         // [rows*S*ccap] candidate ids
    int32_t *ccnt;        // [rows*S] candidates per slice
    uint32_t *crej;       // [rows*S] bound on rejected keys (0: nothing rejected)
    int32_t *cflag;       // [rows*S] 1: candidate buffer overflowed
    double *psum;         // [rows*S] double partial softmax denominators
    int32_t *pcnt;        // [rows*S] window counts
    int32_t *locks;       // [nslots] full-window scratch slot locks
    uint64_t *full_keys;  // [nslots][2][vocab]
    uint32_t *full_bm;    // [nslots][vocab/32+1]
    int32_t *err;         // [1] sticky error flag (a full-window slot wait gave up)
    WaveRec *wrec;        // [rows*parts*8] streaming kernel: per-wavefront results
    uint2 *pcand;         // [rows*parts*256] streaming kernel: (key, id) candidates
    // [rows] streaming kernel, greedy rows decided by their last part (null: by k_decide):
    // the largest (penalised key, ~id) over the parts done, their largest max key, and the
    // parts done; zero between picks (the last part resets them)
    uint64_t *gbest;
    uint32_t *gmaxk;
    uint32_t *gcnt;
    int nslots;
    int ccap;             // candidates per slice list
    int spin_limit;       // full-window slot lock: attempts before giving up
    int sum_in_order;     // 1: the exact path always sums the denominator in id order (a
                          // test hook); 0: only when its fixed-order sum leaves inv open
};

struct Geometry {
    const float *logits;
    int64_t stride;
    int vocab;
    int n_rows;
    int slices;
    int slice_len;
    int bm_words;         // LDS bitmap words per slice
};

// History membership of [lo, hi) as a bitmap (LDS or global); ids outside are skipped and
// duplicates set the same bit, so each id is penalised once (sample.c:120).
template <int NT>
__device__ __forceinline__ void build_bitmap(uint32_t *bm, int words, int lo, int hi, const RowState &st,
                             int row, int cap) {
    for (int j = threadIdx.x; j < words; j += NT) bm[j] = 0u;
    __syncthreads();
    int len, head;
    ring_pos(st, row, cap, len, head);
    const int32_t *ring = st.ring + (int64_t)row * st.ring_stride;
    for (int j = threadIdx.x; j < len; j += NT) {
        const int id = ring[qs_ring_slot(cap, head, j)];
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

// ---- block-level select and sort -----------------------------------------------------------

// K-th largest of n keys in LDS (1 <= k <= n), by 8-bit radix select: four rounds of a
// 256-bin histogram restricted to the prefix found so far.
template <int NT>
__device__ __forceinline__ uint32_t block_kth(const uint32_t *keys, int n, int k, uint32_t *hist, int *sh) {
    const int tid = threadIdx.x, lane = tid & 63;
    uint32_t prefix = 0u, pmask = 0u;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int j = tid; j < 256; j += NT) hist[j] = 0u;
        __syncthreads();
        for (int j0 = 0; j0 < n; j0 += NT) {
            const int j = j0 + tid;
            const uint32_t u = j < n ? keys[j] : 0u;
            bool hit = j < n && (u & pmask) == prefix;
            const uint32_t bin = (u >> shift) & 255u;
            // the lanes in the first hitting lane's bin add together (keys of one row share
            // their leading bytes, so one bin takes most of them), the rest one by one
            const uint64_t m = __ballot(hit);
            if (m) {
                const uint32_t b0 = (uint32_t)__shfl((int)bin, __ffsll((unsigned long long)m) - 1, 64);
                const uint64_t same = __ballot(hit && bin == b0);
                if (lane == __ffsll((unsigned long long)m) - 1) atomicAdd(&hist[b0], (uint32_t)__popcll(same));
                if (bin == b0) hit = false;
                if (hit) atomicAdd(&hist[bin], 1u);
            }
        }
        __syncthreads();
        if (tid < 64) {
            uint32_t c[4];
            for (int q = 0; q < 4; ++q) c[q] = hist[4 * lane + q];
            const uint32_t mine = c[0] + c[1] + c[2] + c[3];
            uint32_t incl = mine;                       // sum over lanes >= this one
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_down(incl, o, 64);
                if (lane + o < 64) incl += t;
            }
            const uint32_t excl = incl - mine;
            if (excl < (uint32_t)k && (uint32_t)k <= incl) {
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

// Sort n_pad (a power of two) 64-bit keys in LDS, descending.
template <int NT>
__device__ __forceinline__ void bitonic_desc(uint64_t *s, int n_pad) {
    for (int size = 2; size <= n_pad; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < (n_pad >> 1); i += NT) {
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

// The same sort by one wavefront over 64*Q keys held Q per lane (element q*64 + lane in
// v[q]): strides below 64 exchange lanes, larger ones exchange registers of a lane.  The
// compare-exchange network is bitonic_desc's, so the order is the same; no barrier.
template <int Q, int SIZE, int S>
__device__ __forceinline__ void bitonic_step_q(uint64_t (&v)[Q], int lane) {
    if constexpr (S >= 64) {
        constexpr int R = S / 64;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            if ((q & R) == 0) {
                const bool desc = ((q * 64) & SIZE) == 0;
                const uint64_t a = v[q], b = v[q | R];
                const bool sw = (a < b) == desc;
                v[q] = sw ? b : a;
                v[q | R] = sw ? a : b;
            }
        }
    } else {
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const uint64_t o = xor_lane64<S>(v[q]);
            const bool desc = SIZE >= 64 ? (((q * 64) & SIZE) == 0) : ((lane & SIZE) == 0);
            const bool keep_max = ((lane & S) == 0) == desc;
            v[q] = keep_max ? (o > v[q] ? o : v[q]) : (o < v[q] ? o : v[q]);
        }
    }
}
template <int Q, int SIZE, int S>
__device__ __forceinline__ void bitonic_strides_q(uint64_t (&v)[Q], int lane) {
    if constexpr (S >= 1) {
        bitonic_step_q<Q, SIZE, S>(v, lane);
        bitonic_strides_q<Q, SIZE, S / 2>(v, lane);
    }
}
template <int Q, int SIZE>
__device__ __forceinline__ void bitonic_sizes_q(uint64_t (&v)[Q], int lane) {
    if constexpr (SIZE <= 64 * Q) {
        bitonic_strides_q<Q, SIZE, SIZE / 2>(v, lane);
        bitonic_sizes_q<Q, SIZE * 2>(v, lane);
    }
}
// Sort s[0, n) descending in place, n <= 64*Q, by the calling wavefront; slots from n on
// enter as 0 (below every key) and are neither read nor written.
template <int Q>
__device__ __forceinline__ void wave_sort_lds_desc(uint64_t *s, int n) {
    const int lane = threadIdx.x & 63;
    uint64_t v[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) v[q] = q * 64 + lane < n ? s[q * 64 + lane] : 0ull;
    bitonic_sizes_q<Q, 2>(v, lane);
#pragma unroll
    for (int q = 0; q < Q; ++q)
        if (q * 64 + lane < n) s[q * 64 + lane] = v[q];
}

// One direction of a bitonic merge over a wavefront's 64 keys (strides 32 down to 1).
__device__ __forceinline__ uint64_t wave_merge_dir(uint64_t v, bool desc, int lane) {
    auto step = [&](uint64_t o, int S) {
        const bool keep_max = ((lane & S) == 0) == desc;
        v = keep_max ? (o > v ? o : v) : (o < v ? o : v);
    };
    step(xor_lane64<32>(v), 32);
    step(xor_lane64<16>(v), 16);
    step(xor_lane64<8>(v), 8);
    step(xor_lane64<4>(v), 4);
    step(xor_lane64<2>(v), 2);
    step(xor_lane64<1>(v), 1);
    return v;
}

// bitonic_desc's network over s[0, 64*W) with W = n/64 wavefronts (n a power of two,
// 128 <= n <= NT): element i in lane i%64 of wavefront i/64; strides below 64 move
// between lanes, larger ones through s with a barrier pair.  Every thread of the block
// calls this; s[0, n) ends sorted descending.
template <int NT>
__device__ __forceinline__ void block_sort_desc_waves(uint64_t *s, int n) {
    const int i = threadIdx.x, lane = i & 63, w = i >> 6;
    const bool part = i < n;
    uint64_t v = 0ull;
    if (part) {
        v = s[i];
        bitonic_step<2, 1>(v, lane);
        bitonic_step<4, 2>(v, lane);   bitonic_step<4, 1>(v, lane);
        bitonic_step<8, 4>(v, lane);   bitonic_step<8, 2>(v, lane);   bitonic_step<8, 1>(v, lane);
        bitonic_step<16, 8>(v, lane);  bitonic_step<16, 4>(v, lane);  bitonic_step<16, 2>(v, lane);
        bitonic_step<16, 1>(v, lane);
        bitonic_step<32, 16>(v, lane); bitonic_step<32, 8>(v, lane);  bitonic_step<32, 4>(v, lane);
        bitonic_step<32, 2>(v, lane);  bitonic_step<32, 1>(v, lane);
        v = wave_merge_dir(v, (w & 1) == 0, lane);              // size 64
    }
    for (int size = 128; size <= n; size <<= 1) {
        for (int S = size >> 1; S >= 64; S >>= 1) {
            __syncthreads();                                     // last exchange read
            if (part) s[i] = v;
            __syncthreads();
            if (part) {
                const uint64_t o = s[i ^ S];
                const bool keep_max = ((i & S) == 0) == ((i & size) == 0);
                v = keep_max ? (o > v ? o : v) : (o < v ? o : v);
            }
        }
        if (part) v = wave_merge_dir(v, (i & size) == 0, lane);
    }
    __syncthreads();
    if (part) s[i] = v;
    __syncthreads();
}

// (p, id) sort key: p's bits above, ~id below, so descending order is p desc, id asc
// (sample.c:151 under glibc's stable merge sort on ascending ids).
__device__ __forceinline__ uint64_t pid_key(float p, int id) {
    return ((uint64_t)__float_as_uint(p) << 32) | (uint32_t)~(uint32_t)id;
}
__device__ __forceinline__ float key_p(uint64_t k) { return __uint_as_float((uint32_t)(k >> 32)); }
__device__ __forceinline__ int key_id(uint64_t k) { return (int)~(uint32_t)(k & 0xFFFFFFFFull); }

// ---- the decision over sorted candidates (one thread) --------------------------------------

// sample.c:153-178 over the first positions of the (p desc, id asc) order: pf(i) is the
// probability and idf(i) the id at position i (in-window candidates come first).
// Positions [0, E) are known to be positions of the full order; nwin is the window size.
// Returns false (nothing consumed) when the cuts or the draw would read a position >= E;
// otherwise advances rs and fills id and d.  Every loop index is uniform, so a wavefront
// can run it with pf/idf reading lanes.
template <typename PF, typename IF>
__device__ __forceinline__ bool decide_prefix_f(PF &&pf, IF &&idf, int E, int nwin,
                                                const qs_row_param &P, uint64_t &rs, int &id,
                                                qs_pick_diag &d) {
    if (E < 1) return false;
    int n = nwin;                                             // sample.c:153-154
    if (P.top_k > 0 && P.top_k < n) n = P.top_k;
    d.keep_topk = n;
    if (P.top_p < 1.0f) {                                     // sample.c:155-160
        double cum = 0.0;
        int keep = n;
        for (int i = 0; i < n; ++i) {
            if (i >= E) return false;
            cum += pf(i);
            if (cum >= P.top_p) { keep = i + 1; break; }
        }
        n = keep;
    }
    d.keep_topp = n;
    if (P.min_p > 0.0f) {                                     // sample.c:161-168
        const float floor_p = P.min_p * pf(0);
        int keep = n;
        for (int i = 1; i < n; ++i) {
            if (i >= E) return false;
            if (pf(i) < floor_p) { keep = i; break; }
        }
        n = keep;
    }
    if (n < 1) n = 1;
    if (n > E) return false;
    double rsum = 0.0;                                        // sample.c:170-175
    for (int i = 0; i < n; ++i) rsum += pf(i);
    const double u = rng_unit(rs);
    const double r = u * rsum;
    double acc = 0.0;
    int rank = n - 1;
    for (int i = 0; i < n; ++i) {
        acc += pf(i);
        if (r <= acc) { rank = i; break; }
    }
    id = idf(rank);
    d.keep = n;
    d.rank = rank;
    d.rsum = rsum;
    d.u = u;
    d.p0 = pf(0);
    return true;
}

// f(i, p) over the probabilities of s[lo, hi) in order until it returns true; returns
// that i, or hi.  Eight keys are read ahead of their turn (indexes clamped to hi - 1), so
// one thread's ordered sums wait on the LDS once per eight positions.
template <typename F>
__device__ __forceinline__ int scan_p(const uint64_t *s, int lo, int hi, F &&f) {
    for (int i0 = lo; i0 < hi; i0 += 8) {
        float p[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) p[k] = key_p(s[min(i0 + k, hi - 1)]);
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (i0 + k < hi && f(i0 + k, p[k])) return i0 + k;
    }
    return hi;
}

// decide_prefix_f over sorted keys in LDS, one thread: the same cuts, sums (in the same
// order) and results, each loop a scan_p.
__device__ __forceinline__ bool decide_prefix(const uint64_t *srt, int E, int nwin,
                                              const qs_row_param &P, uint64_t &rs, int &id,
                                              qs_pick_diag &d) {
    if (E < 1) return false;
    int n = nwin;                                             // sample.c:153-154
    if (P.top_k > 0 && P.top_k < n) n = P.top_k;
    d.keep_topk = n;
    if (P.top_p < 1.0f) {                                     // sample.c:155-160
        double cum = 0.0;
        const int lim = min(n, E);
        const int j = scan_p(srt, 0, lim, [&](int, float p) {
            cum += p;
            return cum >= P.top_p;
        });
        if (j < lim) n = j + 1;
        else if (n > E) return false;                         // the cut reads past E
    }
    d.keep_topp = n;
    const float p0 = key_p(srt[0]);
    if (P.min_p > 0.0f) {                                     // sample.c:161-168
        const float floor_p = P.min_p * p0;
        const int lim = min(n, E);
        const int j = scan_p(srt, 1, lim, [&](int, float p) { return p < floor_p; });
        if (j < lim) n = j;
        else if (n > E) return false;
    }
    if (n < 1) n = 1;
    if (n > E) return false;
    double rsum = 0.0;                                        // sample.c:170-175
    scan_p(srt, 0, n, [&](int, float p) {
        rsum += p;
        return false;
    });
    const double u = rng_unit(rs);
    const double r = u * rsum;
    double acc = 0.0;
    const int j = scan_p(srt, 0, n, [&](int, float p) {
        acc += p;
        return r <= acc;
    });
    const int rank = j < n ? j : n - 1;
    id = key_id(srt[rank]);
    d.keep = n;
    d.rank = rank;
    d.rsum = rsum;
    d.u = u;
    d.p0 = p0;
    return true;
}

// decide_prefix_f for a wavefront whose lane i holds the (p, id) key of position i (lanes
// past the candidates hold 0).  When every probability at positions below min(E, 64) is 0
// or at least 2^-24, each is a multiple of 2^-47 and every partial sum of them lies below
// 2, so binary64 holds every partial sum exactly: the running sums of sample.c:157, 171
// and 174 then equal an inclusive lane scan (whatever the order of its additions) and
// each cut is the first lane that passes its test.  Otherwise the sequential loops run.
__device__ __forceinline__ bool decide_prefix_wave(uint64_t pk, int E, int nwin,
                                                   const qs_row_param &P, uint64_t &rs,
                                                   int &id, qs_pick_diag &d) {
    const int lane = threadIdx.x & 63;
    const float p = key_p(pk);
    const int lim = E < 64 ? E : 64;
    const bool inb = lane < lim;
    if (__ballot(inb && p != 0.0f && !(p >= 0x1p-24f)))
        return decide_prefix_f([&](int i) { return key_p(lane_u64(pk, i)); },
                               [&](int i) { return key_id(lane_u64(pk, i)); }, E, nwin, P, rs,
                               id, d);
    if (E < 1) return false;
    const double cum = wave_scan_d(inb ? (double)p : 0.0);
    int n = nwin;                                             // sample.c:153-154
    if (P.top_k > 0 && P.top_k < n) n = P.top_k;
    d.keep_topk = n;
    if (P.top_p < 1.0f) {                                     // sample.c:155-160
        const uint64_t hit = __ballot(inb && lane < n && cum >= (double)P.top_p);
        if (hit) n = __builtin_ctzll(hit) + 1;
        else if (n > E) return false;
    }
    d.keep_topp = n;
    const float p0 = __shfl(p, 0, 64);
    if (P.min_p > 0.0f) {                                     // sample.c:161-168
        const float floor_p = P.min_p * p0;
        const uint64_t hit = __ballot(inb && lane >= 1 && lane < n && p < floor_p);
        if (hit) n = __builtin_ctzll(hit);
        else if (n > E) return false;
    }
    if (n < 1) n = 1;
    if (n > E) return false;
    const double rsum = __shfl(cum, n - 1, 64);               // sample.c:170-175
    const double u = rng_unit(rs);
    const double r = u * rsum;
    const uint64_t hit = __ballot(lane < n && r <= cum);
    const int rank = hit ? __builtin_ctzll(hit) : n - 1;
    id = key_id(lane_u64(pk, rank));
    d.keep = n;
    d.rank = rank;
    d.rsum = rsum;
    d.u = u;
    d.p0 = p0;
    return true;
}

// ---- the full-window path ------------------------------------------------------------------

// Stable LSD radix sort of n 64-bit keys, descending, 8 bits per pass; each wavefront
// owns a contiguous range and ranks equal digits by lane order (ballot multisplit).
// Returns the buffer holding the result (a or b).  whist: NT/64*256 words, sh: 1 int.
template <int NT>
__device__ __forceinline__ uint64_t *radix_sort_desc(uint64_t *a, uint64_t *b, int n, uint32_t *whist,
                                     uint32_t *wsum, int *sh) {
    constexpr int NWV = NT / 64;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int ch = (n + NWV - 1) / NWV;
    const int beg = min(wv * ch, n), end = min(beg + ch, n);
    const uint64_t lt = lane ? (~0ull >> (64 - lane)) : 0ull;
    uint64_t *src = a, *dst = b;
    for (int shift = 0; shift < 64; shift += 8) {
        for (int j = tid; j < NWV * 256; j += NT) whist[j] = 0u;
        if (tid == 0) sh[0] = 0;
        __syncthreads();
        for (int base = beg; base < end; base += 64) {
            const int j = base + lane;
            if (j < end) atomicAdd(&whist[wv * 256 + 255 - (int)((src[j] >> shift) & 255u)], 1u);
        }
        __syncthreads();
        // exclusive offsets in (digit, wave) order; a pass where one digit holds every
        // key moves nothing and is skipped.  Threads 0..255 own one digit each.
        uint32_t tot = 0, incl = 0;
        if (tid < 256) {
            for (int w = 0; w < NWV; ++w) tot += whist[w * 256 + tid];
            if (tot == (uint32_t)n) sh[0] = 1;
            incl = tot;
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_up(incl, o, 64);
                if (lane >= o) incl += t;
            }
            if (lane == 63) wsum[wv] = incl;
        }
        __syncthreads();
        if (tid < 256) {
            uint32_t run = incl - tot;
            for (int w = 0; w < wv; ++w) run += wsum[w];
            for (int w = 0; w < NWV; ++w) {
                const uint32_t c = whist[w * 256 + tid];
                whist[w * 256 + tid] = run;
                run += c;
            }
        }
        __syncthreads();
        const bool skip = sh[0] != 0;
        __syncthreads();           // every thread has read sh[0] before the next pass resets it
        if (skip) continue;
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
                if ((peers >> lane) == 1ull) whist[wv * 256 + dg] += (uint32_t)__popcll(peers);
            }
        }
        __syncthreads();
        uint64_t *t = src;
        src = dst;
        dst = t;
    }
    return src;
}

// Shared memory a full-window pass needs (static per kernel).
template <int NT>
struct FullLds {
    uint32_t whist[(NT / 64) * 256];
    uint32_t wsum[NT / 64];
    int sh[4];
};

// The whole window of one row, sorted on the device, then sample.c:153-178 sequentially.
// Takes a scratch slot (bounded wait on running holders; on giving up the row gets id -3,
// its generator state and history stay as they were, and the sticky error flag is set).
// maxl/sum are the row's max penalised logit and exact softmax denominator.
template <int NT>
__device__ __forceinline__ void full_row(const float *x, int V, int row, const qs_row_param &P, float maxl,
                         double sum, const RowState &st, const Scratch &sc, int32_t *out,
                         qs_pick_diag *diag, const uint64_t *tab, FullLds<NT> &fl,
                         int fixed_slot) {
    const int tid = threadIdx.x, lane = tid & 63;
    int32_t *ring = st.ring + (int64_t)row * st.ring_stride;
    const bool locked = fixed_slot < 0;
    if (tid == 0) {
        int slot = fixed_slot;
        if (locked)
            for (int it = 0; it < sc.spin_limit; ++it) {
                const int s = (row + it) % sc.nslots;
                if (atomicCAS(&sc.locks[s], 0, 1) == 0) { slot = s; break; }
                if ((it + 1) % sc.nslots == 0) __builtin_amdgcn_s_sleep(16);
            }
        fl.sh[0] = slot;
    }
    __syncthreads();
    const int slot = fl.sh[0];
    __syncthreads();
    if (slot < 0) {
        if (tid == 0) {
            atomicOr(sc.err, 1);
            out[row] = -3;
        }
        return;
    }
    uint64_t *ka = sc.full_keys + (int64_t)slot * 2 * V;
    uint64_t *kb = ka + V;
    uint32_t *bm = sc.full_bm + (int64_t)slot * (V / 32 + 1);

    const float inv_t = P.inv_t;
    const float msc = maxl * inv_t;
    const float thr = msc - 30.0f;
    const bool deg = !isfinite(msc);       // every p is NaN (sample.c:148 on inf - inf)
    const float inv = (float)(1.0 / sum);
    const float rp = P.repeat_penalty;
    const bool pen = rp > 1.0f && st.hlen[row] > 0 && P.ring_cap > 0;
    if (pen) build_bitmap<NT>(bm, V / 32 + 1, 0, V, st, row, P.ring_cap);
    if (tid == 0) fl.sh[1] = 0;
    __syncthreads();
    for (int i0 = 0; i0 < V; i0 += NT) {
        const int i = i0 + tid;
        bool in = false;
        uint64_t key = 0ull;
        if (i < V) {
            float w = x[i];
            if (pen && ((bm[i >> 5] >> (i & 31)) & 1u)) w = penalise(w, rp);
            const float s = w * inv_t;
            if (s >= thr) {
                in = true;
                const float p = deg ? 0.0f : qs_expf_core(s - msc, tab) * inv;
                key = pid_key(p, i);
            }
        }
        const uint64_t m = __ballot(in);
        int base = 0;
        if (lane == 0 && m) base = atomicAdd(&fl.sh[1], __popcll(m));
        base = __shfl(base, 0, 64);
        if (in) ka[base + lane_prefix(m)] = key;
    }
    __syncthreads();
    const int nw = fl.sh[1];
    __syncthreads();
    // Every read below is of the first min(top_k, nw) positions.  With top_k below the
    // window size the K-th largest p is selected first (four 8-bit radix passes over the p
    // bits, non-negative floats ordering as their bits do) and only the keys with p at or
    // above it are sorted: at least K keys, among them every key of the first K positions of
    // the window's order, in that order.
    const uint64_t *srt;
    if (P.top_k > 0 && P.top_k < nw) {
        uint32_t prefix = 0u, pmask = 0u;
        int need = P.top_k;
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int j = tid; j < 256; j += NT) fl.whist[j] = 0u;
            __syncthreads();
            for (int i = tid; i < nw; i += NT) {
                const uint32_t hb = (uint32_t)(ka[i] >> 32);
                if ((hb & pmask) == prefix) atomicAdd(&fl.whist[(hb >> shift) & 255u], 1u);
            }
            __syncthreads();
            if (tid < 64) {
                // lane l holds digits 4l..4l+3; the digit taken is the largest d with at
                // least `need` keys at digit d or above (among those matching the prefix)
                uint32_t c[4], t = 0u;
                for (int q = 0; q < 4; ++q) t += (c[q] = fl.whist[4 * lane + q]);
                const uint32_t incl = wave_scan(t);
                const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
                uint32_t above = total - incl;          // keys at digits above 4l+3
                int dl = -1;
                uint32_t nl = 0u;
                for (int q = 3; q >= 0 && dl < 0; --q) {
                    if (above + c[q] >= (uint32_t)need) {
                        dl = 4 * lane + q;
                        nl = (uint32_t)need - above;
                    }
                    above += c[q];
                }
                const uint64_t has = __ballot(dl >= 0);
                const int top = 63 - __builtin_clzll(has);   // the lane of the largest digit
                if (lane == top) {
                    fl.sh[2] = dl;
                    fl.sh[3] = (int)nl;
                }
            }
            __syncthreads();
            prefix |= (uint32_t)fl.sh[2] << shift;
            pmask |= 255u << shift;
            need = fl.sh[3];
            __syncthreads();
        }
        if (tid == 0) fl.sh[1] = 0;
        __syncthreads();
        for (int i0 = 0; i0 < nw; i0 += NT) {
            const int i = i0 + tid;
            const uint64_t key = i < nw ? ka[i] : 0ull;
            const bool take = i < nw && (uint32_t)(key >> 32) >= prefix;
            const uint64_t m = __ballot(take);
            int base = 0;
            if (lane == 0 && m) base = atomicAdd(&fl.sh[1], __popcll(m));
            base = __shfl(base, 0, 64);
            if (take) kb[base + lane_prefix(m)] = key;
        }
        __syncthreads();
        const int nsel = fl.sh[1];
        __syncthreads();
        srt = radix_sort_desc<NT>(kb, ka, nsel, fl.whist, fl.wsum, &fl.sh[2]);
    } else {
        srt = radix_sort_desc<NT>(ka, kb, nw, fl.whist, fl.wsum, &fl.sh[2]);
    }
    if (tid == 0) {
        qs_pick_diag d;
        memset(&d, 0, sizeof d);
        uint64_t rs = st.rng[row];
        int id = 0;
        if (nw == 0) {
            // empty window: sample.c returns the id its scratch still holds; here 0
            d.u = rng_unit(rs);
            d.path = QS_PATH_EMPTY;
            d.keep = 1;
        } else {
            const float qnan = __builtin_nanf("");
#define QS_PF(i) (deg ? qnan : key_p(srt[(i)]))
            int n = nw;                                           // sample.c:153-168
            if (P.top_k > 0 && P.top_k < n) n = P.top_k;
            d.keep_topk = n;
            if (P.top_p < 1.0f) {
                double cum = 0.0;
                int keep = n;
                for (int i = 0; i < n; ++i) {
                    cum += QS_PF(i);
                    if (cum >= P.top_p) { keep = i + 1; break; }
                }
                n = keep;
            }
            d.keep_topp = n;
            if (P.min_p > 0.0f) {
                const float floor_p = P.min_p * QS_PF(0);
                int keep = n;
                for (int i = 1; i < n; ++i)
                    if (QS_PF(i) < floor_p) { keep = i; break; }
                n = keep;
            }
            if (n < 1) n = 1;
            double rsum = 0.0;                                    // sample.c:170-175
            for (int i = 0; i < n; ++i) rsum += QS_PF(i);
            const double u = rng_unit(rs);
            const double r = u * rsum;
            double acc = 0.0;
            int rank = n - 1;
            for (int i = 0; i < n; ++i) {
                acc += QS_PF(i);
                if (r <= acc) { rank = i; break; }
            }
            id = key_id(srt[rank]);
            d.keep = n;
            d.rank = rank;
            d.rsum = rsum;
            d.u = u;
            d.p0 = QS_PF(0);
#undef QS_PF
            d.path = QS_PATH_FULL;
        }
        st.rng[row] = rs;
        ring_record(ring, st.hlen + row, st.hhead + row, P.ring_cap, id);
        out[row] = id;
        d.id = id;
        d.n_window = nw;
        d.n_cand = nw;
        d.maxl = maxl;
        d.msc = msc;
        d.inv = deg ? __builtin_nanf("") : inv;
        d.inv_hi = d.inv;
        d.sum = deg ? (double)__builtin_nanf("") : sum;
        d.sum_hi = d.sum;
        if (diag) diag[row] = d;
        if (locked) {
            __threadfence();
            atomicExch(&sc.locks[slot], 0);
        }
    }
    __syncthreads();
}

// ---- everything after the two streaming passes, for one sampling row ------------------------

// Row totals gathered from the streaming passes.
struct RowTotals {
    float maxl;      // max penalised logit
    double sum;      // double softmax denominator (fixed-order partial sums)
    int nwin;        // window size
    int cflag;       // some candidate list overflowed
    uint32_t rej;    // bound on every logit not among the candidates (key; 0: none)
    int total;       // gathered candidates (keys[], ids[])
};

// LDS a decision needs besides the gathered candidates.
template <int NT>
struct DecideLds {
    uint64_t tab[QS_EXPF_TAB_N];
    uint32_t hist[256];
    int sh[8];
    uint32_t shu[2];
};

// decide_prefix by one wavefront over positions [0, 64*Q) of sorted keys in LDS, from
// inclusive prefix sums in double instead of running sums.  They are the same numbers
// when every probability read is 0 or in [2^-29, 2) and their total is below 2: every
// such float is a multiple of 2^-52, so every partial sum is a multiple of 2^-52 below 2
// and exact in double, whatever the order of the additions.  Returns 1 when decided (rs,
// id and d as decide_prefix gives them), 0 where decide_prefix returns false, -1 (nothing
// consumed) when the sums might not be exact or the positions do not fit: the caller
// then runs decide_prefix.  Every lane of the wavefront gets the same results.
template <int Q>
__device__ __forceinline__ int decide_prefix_par(const uint64_t *srt, int E, int nwin,
                                                 const qs_row_param &P, uint64_t &rs, int &id,
                                                 qs_pick_diag &d) {
    const int lane = threadIdx.x & 63;
    if (E < 1) return 0;
    int n = nwin;                                             // sample.c:153-154
    if (P.top_k > 0 && P.top_k < n) n = P.top_k;
    const int lim = min(n, E);          // the loops of decide_prefix read positions < lim
    if (lim < 1 || lim > 64 * Q) return -1;
    float p[Q];
    double c[Q];
    double carry = 0.0;
    bool bad = false;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int i = q * 64 + lane;
        p[q] = i < lim ? key_p(srt[i]) : 0.0f;
        const uint32_t b = __float_as_uint(p[q]);
        bad |= (b != 0u && b < 0x31000000u) || b >= 0x40000000u;   // not 0 or [2^-29, 2)
        double x = (double)p[q];
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const double y = __shfl_up(x, o, 64);
            if (lane >= o) x += y;
        }
        c[q] = x + carry;
        carry = __shfl(c[q], 63, 64);
    }
    if (__ballot(bad) != 0ull || !(carry < 2.0)) return -1;
    // the first position below `end` (and from `beg`) where pred holds, or `end`
    auto first = [&](int beg, int end, auto &&pred) {
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int i = q * 64 + lane;
            const uint64_t m = __ballot(i >= beg && i < end && pred(q));
            if (m) return q * 64 + (int)__builtin_ctzll(m);
        }
        return end;
    };
    d.keep_topk = n;
    if (P.top_p < 1.0f) {                                     // sample.c:155-160
        const int j = first(0, lim, [&](int q) { return c[q] >= P.top_p; });
        if (j < lim) n = j + 1;
        else if (n > E) return 0;
    }
    d.keep_topp = n;
    const float p0 = __shfl(p[0], 0, 64);
    if (P.min_p > 0.0f) {                                     // sample.c:161-168
        const float floor_p = P.min_p * p0;
        const int lim2 = min(n, E);
        const int j = first(1, lim2, [&](int q) { return p[q] < floor_p; });
        if (j < lim2) n = j;
        else if (n > E) return 0;
    }
    if (n < 1) n = 1;
    if (n > E) return 0;
    double cl = 0.0;                                          // sample.c:170-175
#pragma unroll
    for (int q = 0; q < Q; ++q)
        if (q == ((n - 1) >> 6)) cl = c[q];
    const double rsum = __shfl(cl, (n - 1) & 63, 64);
    const double u = rng_unit(rs);
    const double r = u * rsum;
    const int j = first(0, n, [&](int q) { return r <= c[q]; });
    const int rank = j < n ? j : n - 1;
    id = key_id(srt[rank]);
    d.keep = n;
    d.rank = rank;
    d.rsum = rsum;
    d.u = u;
    d.p0 = p0;
    return 1;
}

// sample.c:136-178 for a sampling row whose candidates (keys[0..t.total), ids) are in LDS:
// radix-select the top K by logit, exact p, bitonic sort, prove the prefix, decide and
// record; rows the proof does not cover go through full_row.  fcap bounds t.total,
// srt holds SC keys.  fixed_slot >= 0 names a full-window scratch slot owned by the
// caller, -1 takes one under the slot locks.  All threads of the block call this.  PAR:
// the cuts and the draw come from decide_prefix_par where its sums are exact (same
// results; more code in the caller's kernel).
template <int NT, int SC = SORT_CAP, bool PAR = false>
__device__ __forceinline__ void decide_row(int row, const qs_row_param &P, const RowTotals &t, int fcap,
                           uint32_t *keys, int32_t *ids, uint64_t *srt, DecideLds<NT> &dl,
                           FullLds<NT> &fl, const float *x, int V, const RowState &st,
                           const Scratch &sc, int32_t *out, qs_pick_diag *diag,
                           int fixed_slot) {
    const int tid = threadIdx.x, lane = tid & 63;
    int32_t *ring = st.ring + (int64_t)row * st.ring_stride;
    const uint64_t *tab = dl.tab;
    const float inv_t = P.inv_t;
    const float msc = t.maxl * inv_t;
    const float thr = msc - 30.0f;
    if (isnan(msc)) {
        // Empty window (thr is NaN): sample.c returns the id its scratch still holds; 0 here.
        if (tid == 0) {
            uint64_t rs = st.rng[row];
            const double u = rng_unit(rs);
            st.rng[row] = rs;
            ring_record(ring, st.hlen + row, st.hhead + row, P.ring_cap, 0);
            out[row] = 0;
            if (diag) {
                qs_pick_diag d;
                memset(&d, 0, sizeof d);
                d.path = QS_PATH_EMPTY;
                d.u = u;
                d.maxl = t.maxl;
                d.msc = msc;
                d.keep = 1;
                diag[row] = d;
            }
        }
        __syncthreads();
        return;
    }
    bool full = !isfinite(msc) || t.cflag != 0 || t.total > fcap;
    int nkept = 0;
    uint32_t rej = t.rej;
    if (!full) {
        // every gathered candidate when they fit the sort, else the row's top K by logit
        // (ties kept), everything dropped raising `rej`.  Keeping them all matters where
        // the K-th and the next logit differ but their probabilities round equal: sorted
        // by (p, id) the dropped one may come first in the reference's order, so its p
        // bounds the proven prefix below K and the row would take the whole window.
        const int K = row_ksel(P);
        const uint32_t th = t.total > K && t.total > SC
                                ? block_kth<NT>(keys, t.total, K, dl.hist, dl.sh + 4) : 0u;
        if (tid == 0) { dl.sh[3] = 0; dl.shu[0] = rej; }
        __syncthreads();
        const float inv = (float)(1.0 / t.sum);
        uint32_t myrej = 0u;
        for (int j0 = 0; j0 < t.total; j0 += NT) {
            const int j = j0 + tid;
            const bool valid = j < t.total;
            const uint32_t k = valid ? keys[j] : 0u;
            const bool keep = valid && k >= th;
            if (valid && !keep) myrej = k > myrej ? k : myrej;
            const uint64_t m = __ballot(keep);
            int wbase = 0;
            if (lane == 0 && m) wbase = atomicAdd(&dl.sh[3], __popcll(m));
            wbase = __shfl(wbase, 0, 64);
            if (keep) {
                const int pos = wbase + lane_prefix(m);
                if (pos < SC) {
                    const float s = key2f(k) * inv_t;
                    uint64_t key = 0ull;               // out of the window: sorts last
                    if (s >= thr) key = pid_key(qs_expf_core(s - msc, tab) * inv, ids[j]);
                    srt[pos] = key;
                }
            }
        }
        myrej = wave_max_u(myrej);
        if (lane == 0) atomicMax(&dl.shu[0], myrej);
        __syncthreads();
        nkept = dl.sh[3];
        rej = dl.shu[0];
        if (nkept > SC) full = true;
    }
    if (!full) {
        int npad = 1;
        while (npad < nkept) npad <<= 1;
        for (int j = nkept + tid; j < npad; j += NT) srt[j] = 0ull;
        __syncthreads();
        if (npad >= 128 && npad <= 512 && npad <= NT) {
            block_sort_desc_waves<NT>(srt, npad);       // npad / 64 wavefronts
        } else if (npad <= 512) {                   // one wavefront, no barriers
            if (tid < 64) {
                if (npad <= 64) wave_sort_lds_desc<1>(srt, npad);
                else if (npad <= 128) wave_sort_lds_desc<2>(srt, npad);
                else if (npad <= 256) wave_sort_lds_desc<4>(srt, npad);
                else wave_sort_lds_desc<8>(srt, npad);
            }
            __syncthreads();
        } else {
            bitonic_desc<NT>(srt, npad);
        }
        const float inv = (float)(1.0 / t.sum);
        // in-window candidates (p > 0) sort first: m is the first position with p = 0
        if (tid == 0) { dl.sh[1] = nkept; dl.sh[2] = nkept; }
        __syncthreads();
        for (int j = tid; j < nkept; j += NT)
            if ((srt[j] >> 32) == 0ull) atomicMin(&dl.sh[1], j);
        __syncthreads();
        const int m = dl.sh[1];
        // The largest probability any rejected logit can have (p is monotone in it).
        float p_rej = -1.0f;
        if (rej > KEY_NEG_INF) {
            const float s = key2f(rej) * inv_t;
            if (s >= thr) p_rej = qs_expf_core(s - msc, tab) * inv;
        }
        // Positions [0, E) of the sorted candidates are positions of the full order: E is
        // the first position whose p is at most p_rej (when the window is not all here).
        if (m < t.nwin)
            for (int j = tid; j < m; j += NT)
                if (key_p(srt[j]) <= p_rej) atomicMin(&dl.sh[2], j);
        __syncthreads();
        const int E = min(m, dl.sh[2]);
        // lane 0 records a decided row and sets dl.sh[0] to 0, or to 1 for the whole window
        auto record = [&](bool ok, uint64_t rs, int id, qs_pick_diag &d) {
            if (ok) {
                st.rng[row] = rs;
                ring_record(ring, st.hlen + row, st.hhead + row, P.ring_cap, id);
                out[row] = id;
                if (diag) {
                    d.id = id;
                    d.path = QS_PATH_FAST;
                    d.n_window = t.nwin;
                    d.n_cand = m;
                    d.maxl = t.maxl;
                    d.msc = msc;
                    d.inv = inv;
                    d.inv_hi = inv;
                    d.sum = t.sum;
                    d.sum_hi = t.sum;
                    diag[row] = d;
                }
                dl.sh[0] = 0;
            } else {
                dl.sh[0] = 1;
            }
        };
        if constexpr (PAR) {
            if (tid < 64) {
                qs_pick_diag d;
                memset(&d, 0, sizeof d);
                uint64_t rs = st.rng[row];
                int id = -1;
                int ok = -1;
                if (npad <= 64) ok = decide_prefix_par<1>(srt, E, t.nwin, P, rs, id, d);
                else if (npad <= 128) ok = decide_prefix_par<2>(srt, E, t.nwin, P, rs, id, d);
                else if (npad <= 256) ok = decide_prefix_par<4>(srt, E, t.nwin, P, rs, id, d);
                else if (npad <= 512) ok = decide_prefix_par<8>(srt, E, t.nwin, P, rs, id, d);
                if (tid == 0) {
                    if (ok < 0) ok = decide_prefix(srt, E, t.nwin, P, rs, id, d) ? 1 : 0;
                    record(ok != 0, rs, id, d);
                }
            }
        } else if (tid == 0) {
            qs_pick_diag d;
            memset(&d, 0, sizeof d);
            uint64_t rs = st.rng[row];
            int id = -1;
            const bool ok = decide_prefix(srt, E, t.nwin, P, rs, id, d);
            record(ok, rs, id, d);
        }
        __syncthreads();
        full = dl.sh[0] != 0;
        __syncthreads();
    }
    if (full) full_row<NT>(x, V, row, P, t.maxl, t.sum, st, sc, out, diag, tab, fl, fixed_slot);
}

// ---- the decision by one wavefront ----------------------------------------------------------

constexpr int WAVE_CAND = 256;   // candidates the one-wavefront decision takes (4 per lane)

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor((uint32_t)v, m, 64), hi = __shfl_xor((uint32_t)(v >> 32), m, 64);
    return ((uint64_t)hi << 32) | lo;
}

// A row's generator state and history position, loaded ahead of its decision.
struct RowHist {
    uint64_t rng;
    int len, head;
};
__device__ __forceinline__ RowHist row_hist(const RowState &st, int row) {
    return RowHist{st.rng[row], st.hlen[row], st.hhead[row]};
}

// decide_row's decision for one row by one wavefront, in registers: a threshold keeping
// the K largest candidate keys and at most 64 (a bit-serial ballot bracket), exact p per
// lane, a 64-lane bitonic sort by (p desc, id asc), the proof of the prefix and
// sample.c:153-178 through lane reads.  Keys below the threshold bound the probability of
// everything not kept, as the parts' rejected keys do.  For rows with at most WAVE_CAND
// gathered candidates and top-k at most 64 whose top K (ties kept) are at most 64.
// Returns 0 when the row is decided and recorded, 1 when it needs decide_row (too many
// candidates, non-finite maximum, overflowed lists), 2 when the proof does not cover the
// cuts (the caller runs full_row).  scratch: 64 u64 of LDS private to this wavefront.
__device__ __forceinline__ int decide_row_wave(int row, const qs_row_param &P, const RowTotals &t,
                                               const uint32_t *keys, const int32_t *ids,
                                               uint64_t *scratch, const uint64_t *tab,
                                               const RowState &st, int32_t *out,
                                               qs_pick_diag *diag, const RowHist &h) {
    const int lane = threadIdx.x & 63;
    const float inv_t = P.inv_t;
    const float msc = t.maxl * inv_t;
    const float thr = msc - 30.0f;
    if (!isfinite(msc) || t.cflag || t.total > WAVE_CAND) return 1;
    uint64_t rs = h.rng;
    const int hl = h.len, hh = h.head;
    uint32_t k[4];
    int idv[4];
    bool valid[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int j = q * 64 + lane;
        valid[q] = j < t.total;
        k[q] = valid[q] ? keys[j] : 0u;
        idv[q] = valid[q] ? ids[j] : 0;
    }
    // a threshold keeping the K largest keys (ties kept) and at most 64 in all
    const int K = row_ksel(P);
    if (K > 64) return 1;
    uint32_t th = 0u;
    if (t.total > 64) {
        uint32_t kk[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) kk[q] = valid[q] ? k[q] : 0u;
        th = wave_bracket(kk, K, 64, t.total);
    }
    int n_kept = 0;
    uint32_t myrej = 0u;
    bool keep[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        keep[q] = valid[q] && k[q] >= th;
        if (valid[q] && !keep[q]) myrej = k[q] > myrej ? k[q] : myrej;
        n_kept += __popcll(__ballot(keep[q]));
    }
    if (n_kept > 64) return 1;
    const uint32_t wrej = wave_max_u(myrej);
    const uint32_t rej = t.rej > wrej ? t.rej : wrej;
    // the kept candidates, one per lane
    int base = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint64_t m = __ballot(keep[q]);
        if (keep[q]) scratch[base + lane_prefix(m)] = ((uint64_t)k[q] << 32) | (uint32_t)idv[q];
        base += __popcll(m);
    }
    __builtin_amdgcn_wave_barrier();
    const float inv = (float)(1.0 / t.sum);
    uint64_t pk = 0ull;                            // out of the window: sorts last
    if (lane < n_kept) {
        const uint64_t e = scratch[lane];
        const float s = key2f((uint32_t)(e >> 32)) * inv_t;
        if (s >= thr) pk = pid_key(qs_expf_core(s - msc, tab) * inv, (int)(uint32_t)e);
    }
    pk = wave_sort_desc(pk);
    const int m = __popcll(__ballot((pk >> 32) != 0ull));
    // the largest probability any rejected logit can have (p is monotone in it)
    float p_rej = -1.0f;
    if (rej > KEY_NEG_INF) {
        const float s = key2f(rej) * inv_t;
        if (s >= thr) p_rej = qs_expf_core(s - msc, tab) * inv;
    }
    int E = m;
    if (m < t.nwin) {
        const uint64_t below = __ballot(lane < m && key_p(pk) <= p_rej);
        if (below) E = __builtin_ctzll(below);
    }
    qs_pick_diag d;
    memset(&d, 0, sizeof d);
    int id = -1;
    const bool ok = decide_prefix_wave(pk, E, t.nwin, P, rs, id, d);
    if (!ok) return 2;
    if (lane == 0) {
        int32_t *ring = st.ring + (int64_t)row * st.ring_stride;
        st.rng[row] = rs;
        ring_record_at(ring, st.hlen + row, st.hhead + row, P.ring_cap, id, hl, hh);
        out[row] = id;
        if (diag) {
            d.id = id;
            d.path = QS_PATH_FAST;
            d.n_window = t.nwin;
            d.n_cand = m;
            d.maxl = t.maxl;
            d.msc = msc;
            d.inv = inv;
            d.inv_hi = inv;
            d.sum = t.sum;
            d.sum_hi = t.sum;
            diag[row] = d;
        }
    }
    return 0;
}

// decide_row with the one-wavefront decision first: all threads of the block call it,
// with the gathered candidates in keys/ids (LDS) and the block synchronised.
template <int NT, int SC = SORT_CAP, bool PAR = false>
__device__ __forceinline__ void decide_row_fast(int row, const qs_row_param &P, const RowTotals &t,
                                                int fcap, uint32_t *keys, int32_t *ids,
                                                uint64_t *srt, DecideLds<NT> &dl,
                                                FullLds<NT> &fl, const float *x, int V,
                                                const RowState &st, const Scratch &sc,
                                                int32_t *out, qs_pick_diag *diag,
                                                int fixed_slot, const RowHist *pre = nullptr) {
    if (threadIdx.x < 64) {
        const RowHist h = pre ? *pre : row_hist(st, row);   // loaded by the caller, or now
        const int status = decide_row_wave(row, P, t, keys, ids, srt, dl.tab, st, out, diag, h);
        if (threadIdx.x == 0) dl.sh[7] = status;
    }
    __syncthreads();
    const int status = dl.sh[7];
    __syncthreads();
    if (status == 1)
        decide_row<NT, SC, PAR>(row, P, t, fcap, keys, ids, srt, dl, fl, x, V, st, sc, out, diag,
                           fixed_slot);
    else if (status == 2)
        full_row<NT>(x, V, row, P, t.maxl, t.sum, st, sc, out, diag, dl.tab, fl, fixed_slot);
}

// Whether a fixed-order binary64 sum s of n nonnegative numbers gives the reference's
// inv = (float)(1 / sum) (sample.c:149), whose sum adds the same numbers in id order: both
// sums lie within (n - 1) 2^-53 of the numbers' exact total, so within 2 n 2^-53 of each
// other, and (float)(1 / x) is monotone in x, so one float at both ends of that reach is
// the reference's.
__device__ __forceinline__ bool inv_settled(double s, int n) {
    const double reach = 2.0 * (double)n * 0x1p-53 * s * (1.0 + 0x1p-20);
    return (float)(1.0 / (s - reach)) == (float)(1.0 / (s + reach));
}

// The row's softmax denominator exactly as sample.c:147-149 adds it: the window's
// numerators in id order, one binary64 addition after another (a numerator outside the
// window is 0 here and adds nothing).  All NT threads of the workgroup take part in the
// history bitmaps (blocks of BLK logits in `bm`, BLK / 32 words); wavefront 0 computes 64
// numerators at a time and adds them in order, lane by lane.  About 1 ms for 151,936
// logits: taken only where the fixed-order sum does not settle inv (inv_settled).  `xch`:
// one double of LDS for the result.
template <int NT, int BLK>
__device__ __forceinline__ double sum_in_id_order(const float *x, int V, const RowState &st,
                                                  int row, const qs_row_param &P, float msc,
                                                  uint32_t *bm, const uint64_t *tab,
                                                  double *xch) {
    static_assert(BLK % 64 == 0, "whole batches of 64 ids a block");
    const int tid = threadIdx.x, lane = tid & 63;
    const float rp = P.repeat_penalty, inv_t = P.inv_t, thr = msc - 30.0f;
    const int cap = P.ring_cap;                   // (clamped: row_param)
    int len, head;
    ring_pos(st, row, cap, len, head);
    const bool pen = rp > 1.0f && len > 0 && cap > 0;
    const int32_t *ring = st.ring + (int64_t)row * st.ring_stride;
    double acc = 0.0;
    for (int lo = 0; lo < V; lo += BLK) {
        const int hi = min(lo + BLK, V);
        if (pen) {                                    // sample.c:118-120: each id once
            for (int j = tid; j < BLK / 32; j += NT) bm[j] = 0u;
            __syncthreads();
            for (int j = tid; j < len; j += NT) {
                const int id = ring[qs_ring_slot(cap, head, j)];
                if (id >= lo && id < hi) atomicOr(&bm[(id - lo) >> 5], 1u << ((id - lo) & 31));
            }
            __syncthreads();
        }
        if (tid < 64) {
            for (int b0 = lo; b0 < hi; b0 += 64) {
                const int id = b0 + lane;
                double e = 0.0;
                if (id < hi) {
                    float w = x[id];
                    const int q = id - lo;
                    if (pen && ((bm[q >> 5] >> (q & 31)) & 1u)) w = penalise(w, rp);
                    const float sc = w * inv_t;
                    if (sc >= thr) e = (double)qs_expf_core(sc - msc, tab);
                }
                const uint64_t eb = (uint64_t)__double_as_longlong(e);
                const int lo32 = (int)(uint32_t)eb, hi32 = (int)(uint32_t)(eb >> 32);
                const int n = min(64, hi - b0);
                for (int j = 0; j < n; ++j) {         // (uniform) ids b0, b0 + 1, ... in turn
                    const uint64_t v =
                        ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi32, j) << 32) |
                        (uint32_t)__builtin_amdgcn_readlane(lo32, j);
                    acc += __longlong_as_double((long long)v);
                }
            }
        }
        if (pen) __syncthreads();                     // the block's bitmap is read
    }
    if (tid == 0) *xch = acc;
    __syncthreads();
    const double r = *xch;
    __syncthreads();
    return r;
}

// sample.c:130-134 from per-slice (value, first index) bests: nothing beats a NaN at index
// 0 and a row with nothing above -inf stays at 0.  One thread.
__device__ __forceinline__ void record_greedy(int row, const qs_row_param &P, float bv, int bi, float maxl,
                              float x0, const RowState &st, int32_t *out, qs_pick_diag *diag) {
    int32_t *ring = st.ring + (int64_t)row * st.ring_stride;
    const int id = (bi < 0 || isnan(x0)) ? 0 : bi;
    ring_record(ring, st.hlen + row, st.hhead + row, P.ring_cap, id);
    out[row] = id;
    if (diag) {
        qs_pick_diag d;
        memset(&d, 0, sizeof d);
        d.id = id;
        d.path = QS_PATH_GREEDY;
        d.maxl = maxl;
        d.keep = 1;
        diag[row] = d;
    }
}

}  // namespace qs
