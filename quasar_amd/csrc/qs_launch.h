// qs_launch.h - host-side entry points between the HIP translation units (C++ only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "qs_device.h"

// ---- the one-pass kernel (qs_onepass.hip) ----

constexpr int QS_OP_CPS = 256;    // candidates kept per (row, slice)
constexpr int QS_OP_S_MAX = 64;   // slices per row
constexpr int QS_OP_CTR_STRIDE = 64;   // u32 per row counter line (256 bytes)

// Per-(row, slice) results of the one-pass kernel, read by the row's finalizing workgroup.
struct OpScratch {
    int32_t *ctl;       // [2] queue: next ticket, workgroups finished (both 0 between picks)
    uint32_t *ctr;      // [rows * QS_OP_CTR_STRIDE] per-row max key, arrivals, completions
    double *psum;       // [slice_cap] double partial softmax denominators
    int32_t *pcnt;      // [slice_cap] window counts
    uint32_t *rej;      // [slice_cap] bound on the keys of rejected logits
    int32_t *ccnt;      // [slice_cap] candidates kept, | 1 << 30 when some were dropped
    uint32_t *ckey;     // [slice_cap * QS_OP_CPS] candidate keys
    int32_t *cid;       // [slice_cap * QS_OP_CPS] candidate ids
    float *bestv;       // [slice_cap] greedy rows: slice max
    int32_t *besti;     // [slice_cap] greedy rows: its first index (-1: none)
    int slice_cap;
};

// Slices per row for a pick (0: the vocabulary does not fit); *slice_len receives the
// slice length.  kmax is the largest top-k candidate count of the pick's sampling rows,
// per_xcd the resident workgroups per XCD.
int qs_onepass_geometry(int n_rows, int n_vocab, int kmax, int per_xcd, int *slice_len);
// (row, slice) entries the scratch needs for batches up to max_rows x max_vocab.
int qs_onepass_slice_cap(int max_rows, int max_vocab);
// Resident workgroups of the one-pass kernel on this device (0 when unknown).
int qs_onepass_grid(void);
// Enqueue the one-pass pick on `stream` over at most grid_cap workgroups.
int qs_onepass_launch(const float *logits, int64_t row_stride, int n_rows, int n_vocab, int kmax,
                      const qs::RowState &st, const qs::Scratch &sc, const OpScratch &op,
                      int32_t *out, qs_pick_diag *diag, int grid_cap, hipStream_t stream);

// ---- the queue kernel (qs_queue.hip) ----

int qs_queue_slice_cap(int max_rows, int max_vocab);
int qs_queue_grid(void);
// lag_rows: rows whose scans run ahead of the first sums (0: about half a grid of tasks).
int qs_queue_launch(const float *logits, int64_t row_stride, int n_rows, int n_vocab, int kmax,
                    const qs::RowState &st, const qs::Scratch &sc, const OpScratch &op,
                    int32_t *out, qs_pick_diag *diag, int grid_cap, int lag_rows,
                    hipStream_t stream);

// ---- the pipelined kernel (qs_pipe.hip) ----

// Whether the pipelined kernel (qs_pipe.hip) handles this pick on a grid of `grid`
// persistent workgroups.
int qs_pipe_supported(int n_rows, int n_vocab, int64_t row_stride, const void *logits, int grid);
// Dynamic LDS bytes of that kernel for a vocabulary width.
size_t qs_pipe_lds_bytes(int n_vocab);
// Rows are split in this many parts (the per-part scratch needs rows * parts entries).
int qs_pipe_grid(int max_vocab);
int qs_pipe_parts(void);
// Cooperative launch of the pipelined pick on `stream`.
int qs_pipe_launch(const float *logits, int64_t row_stride, int n_rows, int n_vocab,
                   const qs::RowState &st, const qs::Scratch &sc, int32_t *out,
                   qs_pick_diag *diag, int grid, int wide_k, hipStream_t stream);
