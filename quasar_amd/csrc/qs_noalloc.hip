// qs_noalloc.hip - qs_pick_noalloc: the streaming pick with every buffer either the
// caller's (logits, row state, ids) or this file's static device array `scratch`, so the
// call makes no device allocation (for code under graph capture, serving loops that may
// not allocate, and similar callers).
//
// scratch holds, per GPU the library runs on, the per-part results of the streaming kernel
// for at most QS_NOALLOC_MAX_PARTS row-parts, the whole-window fallback's key and bitmap
// slots for QS_NOALLOC_SLOTS rows at a time up to QS_NOALLOC_MAX_VOCAB logits, the slot
// locks and the error flag.  Its device address is taken once per device with that device
// current (hipGetSymbolAddress) and used for every kernel argument and fill; the locks and
// the flag are cleared by a fill kernel at the start of each call (no memset node, so the
// call can be captured).  Calls on one GPU share the array: calls that overlap on one GPU
// race and must be ordered by the caller (one stream, or events).

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstring>
#include <mutex>

#include "../../include/quasar_sampler.h"
#include "qs_device.h"
#include "qs_internal.h"
#include "qs_launch.h"

using namespace qs;

namespace {

constexpr size_t align256(size_t n) { return (n + 255) / 256 * 256; }

constexpr size_t WREC_BYTES = align256(sizeof(WaveRec) * QS_PART_WAVES * (size_t)QS_NOALLOC_MAX_PARTS);
constexpr size_t CAND_BYTES = align256(sizeof(uint2) * QS_PART_CANDS * (size_t)QS_NOALLOC_MAX_PARTS);
constexpr size_t KEYS_BYTES =
    align256(sizeof(uint64_t) * 2 * (size_t)QS_NOALLOC_MAX_VOCAB * QS_NOALLOC_SLOTS);
constexpr size_t BM_BYTES =
    align256(sizeof(uint32_t) * (size_t)(QS_NOALLOC_MAX_VOCAB / 32 + 1) * QS_NOALLOC_SLOTS);
constexpr size_t FLAG_BYTES = align256(sizeof(int32_t) * (QS_NOALLOC_SLOTS + 1));
constexpr size_t SCRATCH_BYTES = WREC_BYTES + CAND_BYTES + KEYS_BYTES + BM_BYTES + FLAG_BYTES;
static_assert(SCRATCH_BYTES == QS_NOALLOC_SCRATCH_BYTES, "header states the scratch size");

static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
uint8_t *g_ptr[MAX_DEVICES];          // scratch's address on each device (nullptr: not yet)
int g_resident[MAX_DEVICES];          // streaming workgroups the device holds at once

__global__ void k_zero(int32_t *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

// scratch's address on the current device (and its resident workgroup count), taken once.
int device_scratch(uint8_t **ptr, int *resident) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        qs_set_error("qs_pick_noalloc: hipGetDevice: %s", hipGetErrorString(e));
        return QS_EDEVICE;
    }
    if (dev < 0 || dev >= MAX_DEVICES) {
        qs_set_error("qs_pick_noalloc: device %d beyond %d", dev, MAX_DEVICES);
        return QS_EINVAL;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            qs_set_error("qs_pick_noalloc: hipGetSymbolAddress(scratch): %s",
                         hipGetErrorString(e));
            return QS_EDEVICE;
        }
        g_ptr[dev] = (uint8_t *)p;
        const int r = qs_part_resident();
        g_resident[dev] = r > 0 ? r : 512;
    }
    *ptr = g_ptr[dev];
    *resident = g_resident[dev];
    return 0;
}

}  // namespace

int qs_pick_noalloc(const float *d_logits, int64_t row_stride, int n_rows, int n_vocab,
                    const qs_row_config *d_config, uint64_t *d_rng, int32_t *d_ring,
                    int ring_stride, int32_t *d_hist_len, int32_t *d_hist_head,
                    int32_t *d_out, void *stream) {
    if (!d_logits || !d_config || !d_rng || !d_hist_len || !d_hist_head || !d_out ||
        n_rows < 1 || n_vocab < 1 || row_stride < n_vocab || ring_stride < 0 ||
        (ring_stride > 0 && !d_ring)) {
        qs_set_error("qs_pick_noalloc: bad arguments");
        return QS_EINVAL;
    }
    if (!qs_part_supported(n_rows, n_vocab, row_stride, d_logits)) {
        qs_set_error("qs_pick_noalloc: logits must be 16-byte aligned with the vocabulary "
                     "and row stride multiples of 4 (at most %d parts per row)",
                     QS_PART_MAX_PARTS);
        return QS_EINVAL;
    }
    const int64_t parts = (int64_t)qs_part_parts(n_vocab) * n_rows;
    if (parts > QS_NOALLOC_MAX_PARTS || n_vocab > QS_NOALLOC_MAX_VOCAB) {
        qs_set_error("qs_pick_noalloc: %d rows x %d logits need %lld row-parts (at most %d) "
                     "and vocabulary at most %d", n_rows, n_vocab, (long long)parts,
                     QS_NOALLOC_MAX_PARTS, QS_NOALLOC_MAX_VOCAB);
        return QS_EINVAL;
    }
    uint8_t *base = nullptr;
    int resident = 0;
    if (const int rc = device_scratch(&base, &resident)) return rc;
    Scratch sc;
    std::memset(&sc, 0, sizeof sc);
    sc.wrec = (WaveRec *)base;
    sc.pcand = (uint2 *)(base + WREC_BYTES);
    sc.full_keys = (uint64_t *)(base + WREC_BYTES + CAND_BYTES);
    sc.full_bm = (uint32_t *)(base + WREC_BYTES + CAND_BYTES + KEYS_BYTES);
    sc.locks = (int32_t *)(base + WREC_BYTES + CAND_BYTES + KEYS_BYTES + BM_BYTES);
    sc.err = sc.locks + QS_NOALLOC_SLOTS;
    sc.nslots = QS_NOALLOC_SLOTS;
    sc.ccap = 0;
    sc.spin_limit = SPIN_LIMIT;
    sc.sum_in_order = 0;
    static_assert(sizeof(qs_row_config) == sizeof(qs_row_param), "row config layout");
    // the kernels clamp each row's ring capacity to ring_stride (0: no ring, whatever the
    // row configs say) and its history length and head to that capacity (qs_ring.h), so
    // the caller's state arrays never send an access outside a row's own ring
    RowState st{(const qs_row_param *)d_config, d_rng, ring_stride > 0 ? d_ring : nullptr,
                d_hist_len, d_hist_head, ring_stride};
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_zero, dim3(1), dim3(64), 0, s, sc.locks, QS_NOALLOC_SLOTS + 1);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        qs_set_error("qs_pick_noalloc: launch: %s", hipGetErrorString(e));
        return QS_EDEVICE;
    }
    return qs_part_launch(d_logits, row_stride, n_rows, n_vocab, st, sc, d_out, nullptr,
                          resident, s);
}

void qs_row_config_set(qs_row_config *c, float temperature, float top_p, int top_k,
                       float min_p, float repeat_penalty, int repeat_last_n) {
    if (!c) return;
    qs_row_param p;
    uint64_t rng = 0;
    qs_clamp_config(temperature, top_p, top_k, min_p, repeat_penalty, repeat_last_n, 1, 0, &p,
                    &rng);
    std::memcpy(c, &p, sizeof p);
}
