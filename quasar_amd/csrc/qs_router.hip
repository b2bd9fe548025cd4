// qs_router.hip - the mixture-of-experts router's expert choice on the device: per token,
// the softmax of its router logits and the n_used most probable experts, with the
// optional renormalisation of their weights (forward_cpu.c:296-304 with the softmax of
// forward_cpu.c:165-172), bit for bit.
//
// Four tokens per wavefront, one per 16-lane row: n_expert <= 256 logits, lane l of a row
// holding experts l, l+16, ... (16 at most).  Maxima and arg-maxima are row reductions
// over DPP moves (quad permutes and the half-row and row mirrors: every lane of the row
// ends with the result).  The reference's sums are sequential float sums in expert (or
// slot) order, which no tree reproduces: the row's first lane adds the probabilities'
// numerators in expert order out of an LDS copy, the four rows of a wavefront at once;
// the slot-order sum of the chosen weights is kept by every lane as the choices are
// made.  The expf is the library's libm-equal routine.  The choice is a sequence of row
// arg-maxima over (probability, -index) keys: the reference's strict `>` scan from index
// 0 takes the lowest index among equal probabilities, and never a NaN.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "../../include/quasar_sampler.h"
#include "qs_device.h"
#include "qs_internal.h"

namespace {

using namespace qs;

constexpr int RT_WAVES = 4;          // wavefronts per workgroup
constexpr int RT_TOK = 4;            // tokens per wavefront (16 lanes each)
constexpr int RT_MAX_E = 256;        // experts (forward_cpu.c:299 keeps taken[256])
constexpr int RT_MAX_U = 64;         // experts used (forward_cpu.c:298 keeps idx[64])
constexpr int RT_PER_LANE = RT_MAX_E / 16;
constexpr int RT_SLOTS = RT_MAX_U / 16;   // chosen slots per lane (slot s on lane s % 16)

__constant__ uint64_t c_exp_tab_r[QS_EXPF_TAB_N] = QS_EXPF_TABLE_INIT;

// (probability bits + 1) above, ~expert below: larger is chosen first; 0 never is (NaN,
// and lanes past the experts).  Probabilities are never negative, so their bits order
// them; +0 keys as 1.
__device__ __forceinline__ uint64_t choice_key(float p, int e) {
    if (p != p) return 0ull;
    return ((uint64_t)(__float_as_uint(p) + 1u) << 32) | (uint32_t)~(uint32_t)e;
}

// Reductions over each 16-lane row; every lane of the row gets the row's result.
template <typename T, typename F>
__device__ __forceinline__ T row_reduce(T v, F &&op) {
    v = op(v, dpp_move<0xB1, 0xF>(v));      // quad_perm [1,0,3,2]
    v = op(v, dpp_move<0x4E, 0xF>(v));      // quad_perm [2,3,0,1]
    v = op(v, dpp_move<0x141, 0xF>(v));     // row_half_mirror
    v = op(v, dpp_move<0x140, 0xF>(v));     // row_mirror
    return v;
}

__global__ void __launch_bounds__(64 * RT_WAVES)
k_router(const float *logits, int64_t stride, int n_tokens, int n_expert, int n_used,
         int norm, int32_t *out_idx, float *out_wt) {
    __shared__ uint64_t tab[QS_EXPF_TAB_N];
    __shared__ float num[RT_WAVES][RT_TOK][RT_MAX_E];   // the numerators, in expert order
    if (threadIdx.x < QS_EXPF_TAB_N) tab[threadIdx.x] = c_exp_tab_r[threadIdx.x];
    __syncthreads();
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int row = lane >> 4, l16 = lane & 15;
    const int64_t t = ((int64_t)blockIdx.x * RT_WAVES + wv) * RT_TOK + row;
    const bool live = t < n_tokens;
    const int nq = (n_expert + 15) >> 4;
    const float *a = logits + (live ? t * stride : 0);

    // forward_cpu.c:166-167: mx = a[0], then every later a[i] > mx replaces it: a NaN
    // a[0] stays, later NaNs never enter.  fmaxf drops NaNs the same way.
    float v[RT_PER_LANE];
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < RT_PER_LANE; ++q) {
        const int e = 16 * q + l16;
        v[q] = (q < nq && live && e < n_expert) ? a[e] : -INFINITY;
        m = fmaxf(m, v[q]);
    }
    m = row_reduce(m, [](float x, float y) { return fmaxf(x, y); });
    const float a0 = __shfl(v[0], lane & 48, 64);      // the row's element 0
    const float mx = (a0 != a0) ? a0 : m;

    // forward_cpu.c:169-171: e = expf(a - mx); sum in order; inv = 1/sum; p = e * inv
    float *nrow = num[wv][row];
#pragma unroll
    for (int q = 0; q < RT_PER_LANE; ++q) {
        const int e = 16 * q + l16;
        if (q < nq) {
            v[q] = qs_expf_tab(v[q] - mx, tab);
            if (e < n_expert) nrow[e] = v[q];
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float sum = 0.0f;
    if (l16 == 0) {
        int i = 0;
        for (; i + 4 <= n_expert; i += 4) {
            const float4 f = *(const float4 *)(nrow + i);
            sum += f.x;
            sum += f.y;
            sum += f.z;
            sum += f.w;
        }
        for (; i < n_expert; ++i) sum += nrow[i];
    }
    const float inv = 1.0f / __shfl(sum, lane & 48, 64);
    uint64_t key[RT_PER_LANE];
#pragma unroll
    for (int q = 0; q < RT_PER_LANE; ++q) {
        const int e = 16 * q + l16;
        key[q] = (q < nq && live && e < n_expert) ? choice_key(v[q] * inv, e) : 0ull;
    }

    // forward_cpu.c:300-303: n_used arg-maxima; a slot with nothing left to take (all
    // remaining probabilities NaN) reports expert -1 with weight 0.  forward_cpu.c:304: sm
    // is the weights' sum in slot order; if sm > 0 each is divided by it.
    float wt_mine[RT_SLOTS];
    int idx_mine[RT_SLOTS];
#pragma unroll
    for (int j = 0; j < RT_SLOTS; ++j) {
        wt_mine[j] = 0.0f;
        idx_mine[j] = -1;
    }
    float sm = 0.0f;
    for (int s = 0; s < n_used; ++s) {
        uint64_t k = key[0];
#pragma unroll
        for (int q = 1; q < RT_PER_LANE; ++q)
            if (q < nq) k = key[q] > k ? key[q] : k;
        const uint64_t best = row_reduce(k, [](uint64_t x, uint64_t y) { return x > y ? x : y; });
        int e = -1;
        float w = 0.0f;
        if (best != 0ull) {
            e = (int)~(uint32_t)best;
            w = __uint_as_float((uint32_t)(best >> 32) - 1u);
#pragma unroll
            for (int q = 0; q < RT_PER_LANE; ++q)
                if (16 * q + l16 == e) key[q] = 0ull;   // taken
        }
        sm += w;
#pragma unroll
        for (int j = 0; j < RT_SLOTS; ++j)
            if (16 * j + l16 == s) {
                wt_mine[j] = w;
                idx_mine[j] = e;
            }
    }
#pragma unroll
    for (int j = 0; j < RT_SLOTS; ++j) {
        const int s = 16 * j + l16;
        if (live && s < n_used) {
            out_idx[t * n_used + s] = idx_mine[j];
            out_wt[t * n_used + s] = (norm && sm > 0.0f) ? wt_mine[j] / sm : wt_mine[j];
        }
    }
}

}  // namespace

extern "C" {

int qs_router_topk(const float *d_logits, int64_t row_stride, int n_tokens, int n_expert,
                   int n_used, int norm_topk, int32_t *d_idx, float *d_wt, void *stream) {
    if (!d_logits || !d_idx || !d_wt || n_tokens < 0 || n_expert < 1 ||
        n_expert > RT_MAX_E || n_used < 1 || n_used > RT_MAX_U || n_used > n_expert ||
        row_stride < n_expert) {
        qs_set_error("qs_router_topk: bad arguments");
        return QS_EINVAL;
    }
    if (n_tokens == 0) return 0;
    const int64_t per_block = (int64_t)RT_WAVES * RT_TOK;
    const unsigned blocks = (unsigned)(((int64_t)n_tokens + per_block - 1) / per_block);
    hipLaunchKernelGGL(k_router, dim3(blocks), dim3(64 * RT_WAVES), 0, (hipStream_t)stream,
                       d_logits, row_stride, n_tokens, n_expert, n_used, norm_topk ? 1 : 0,
                       d_idx, d_wt);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        qs_set_error("k_router launch: %s", hipGetErrorString(e));
        return QS_EDEVICE;
    }
    return 0;
}

int qs_router_time(const float *d_logits, int64_t row_stride, int n_tokens, int n_expert,
                   int n_used, int norm_topk, int32_t *d_idx, float *d_wt, int iters,
                   float *ms) {
    if (iters < 1 || !ms) {
        qs_set_error("qs_router_time: bad arguments");
        return QS_EINVAL;
    }
    hipStream_t st = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = 0;
    if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
        qs_set_error("qs_router_time: stream or event creation failed");
        rc = QS_EDEVICE;
    }
    if (!rc && hipEventRecord(e0, st) != hipSuccess) rc = QS_EDEVICE;
    for (int i = 0; !rc && i < iters; ++i)
        rc = qs_router_topk(d_logits, row_stride, n_tokens, n_expert, n_used, norm_topk, d_idx,
                            d_wt, st);
    if (!rc && (hipEventRecord(e1, st) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
                hipEventElapsedTime(ms, e0, e1) != hipSuccess)) {
        qs_set_error("qs_router_time: timing failed");
        rc = QS_EDEVICE;
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (st) (void)hipStreamDestroy(st);
    return rc;
}

}  // extern "C"
