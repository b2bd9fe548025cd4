// qs_router.hip - the mixture-of-experts router's expert choice on the device: per token,
// the softmax of its router logits and the n_used most probable experts, with the
// optional renormalisation of their weights (forward_cpu.c:296-304 with the softmax of
// forward_cpu.c:165-172), bit for bit.
//
// One wavefront per token: n_expert <= 256 logits, four per lane at most (lane l holds
// experts l, l+64, l+128, l+192).  The reference's sums are sequential float sums in
// expert (or slot) order, which no tree reproduces: lane 0 adds the values in that order,
// reading them out of the other lanes with readlane (a chain of n_expert float adds, a
// few hundred cycles per token; tokens run in parallel, one per wavefront).  The expf is
// the library's libm-equal routine.  The choice is a sequence of wavefront arg-maxima
// over (probability, -index) keys: the reference's strict `>` scan from index 0 takes
// the lowest index among equal probabilities, and never a NaN.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "../../include/quasar_sampler.h"
#include "qs_device.h"
#include "qs_internal.h"

namespace {

using namespace qs;

constexpr int RT_WAVES = 4;          // tokens per workgroup (one wavefront each)
constexpr int RT_MAX_E = 256;        // experts (forward_cpu.c:299 keeps taken[256])
constexpr int RT_MAX_U = 64;         // experts used (forward_cpu.c:298 keeps idx[64])
constexpr int RT_PER_LANE = RT_MAX_E / 64;

__constant__ uint64_t c_exp_tab_r[QS_EXPF_TAB_N] = QS_EXPF_TABLE_INIT;

// (probability bits + 1) above, ~expert below: larger is chosen first; 0 never is (NaN,
// and lanes past the experts).  Probabilities are never negative, so their bits order
// them; +0 keys as 1.
__device__ __forceinline__ uint64_t choice_key(float p, int e) {
    if (p != p) return 0ull;
    return ((uint64_t)(__float_as_uint(p) + 1u) << 32) | (uint32_t)~(uint32_t)e;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {   // DPP moves, no LDS
    return wave_reduce(v, [](uint64_t x, uint64_t y) { return x > y ? x : y; });
}

// Sequential float sum of lane values v[j] (expert 64 j + lane) for experts [0, n), in
// expert order, as forward_cpu.c:169 adds them; the result in every lane.
__device__ __forceinline__ float ordered_sum(const float (&v)[RT_PER_LANE], int n) {
    float s = 0.0f;
    for (int i = 0; i < n; ++i) {
        const int j = i >> 6, l = i & 63;
        float x = v[0];
#pragma unroll
        for (int q = 1; q < RT_PER_LANE; ++q)
            if (j == q) x = v[q];
        s += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
    }
    return s;
}

__global__ void __launch_bounds__(64 * RT_WAVES)
k_router(const float *logits, int64_t stride, int n_tokens, int n_expert, int n_used,
         int norm, int32_t *out_idx, float *out_wt) {
    __shared__ uint64_t tab[QS_EXPF_TAB_N];
    if (threadIdx.x < QS_EXPF_TAB_N) tab[threadIdx.x] = c_exp_tab_r[threadIdx.x];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * RT_WAVES + (threadIdx.x >> 6);
    if (t >= n_tokens) return;                       // whole wavefronts
    const float *a = logits + t * stride;

    // forward_cpu.c:166-167: mx = a[0], then every later a[i] > mx replaces it: a NaN
    // a[0] stays, later NaNs never enter.  fmaxf drops NaNs the same way.
    float v[RT_PER_LANE];
    float m = -INFINITY;
#pragma unroll
    for (int q = 0; q < RT_PER_LANE; ++q) {
        const int e = 64 * q + lane;
        v[q] = e < n_expert ? a[e] : -INFINITY;
        m = fmaxf(m, v[q]);
    }
    m = wave_max_f(m);
    const float a0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[0]), 0));
    const float mx = (a0 != a0) ? a0 : m;

    // forward_cpu.c:169-171: e = expf(a - mx); sum in order; inv = 1/sum; p = e * inv
#pragma unroll
    for (int q = 0; q < RT_PER_LANE; ++q) v[q] = qs_expf_tab(v[q] - mx, tab);
    const float inv = 1.0f / ordered_sum(v, n_expert);
    uint64_t key[RT_PER_LANE];
#pragma unroll
    for (int q = 0; q < RT_PER_LANE; ++q) {
        const int e = 64 * q + lane;
        const float p = v[q] * inv;
        v[q] = p;
        key[q] = e < n_expert ? choice_key(p, e) : 0ull;
    }

    // forward_cpu.c:300-303: n_used arg-maxima; a slot with nothing left to take (all
    // remaining probabilities NaN) reports expert -1 with weight 0
    float wt_mine = 0.0f;                             // lane s < n_used: slot s
    int idx_mine = -1;
    for (int s = 0; s < n_used; ++s) {
        uint64_t k = key[0];
#pragma unroll
        for (int q = 1; q < RT_PER_LANE; ++q) k = key[q] > k ? key[q] : k;
        const uint64_t best = wave_max_u64(k);
        int e = -1;
        float w = 0.0f;
        if (best != 0ull) {
            e = (int)~(uint32_t)best;
            w = __uint_as_float((uint32_t)(best >> 32) - 1u);
#pragma unroll
            for (int q = 0; q < RT_PER_LANE; ++q)
                if (64 * q + lane == e) key[q] = 0ull;   // taken
        }
        if (lane == s) {
            wt_mine = w;
            idx_mine = e;
        }
    }

    // forward_cpu.c:304: sm = sum of the weights in slot order; if sm > 0 each is divided
    if (norm) {
        float sm = 0.0f;
        for (int s = 0; s < n_used; ++s)
            sm += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wt_mine), s));
        if (sm > 0.0f) wt_mine = wt_mine / sm;
    }
    if (lane < n_used) {
        out_idx[t * n_used + lane] = idx_mine;
        out_wt[t * n_used + lane] = wt_mine;
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
    const unsigned blocks = (unsigned)(((int64_t)n_tokens + RT_WAVES - 1) / RT_WAVES);
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
