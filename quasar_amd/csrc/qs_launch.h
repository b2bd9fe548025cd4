// qs_launch.h - host-side entry points between the HIP translation units (C++ only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "qs_device.h"

// Whether the pipelined kernel (qs_pipe.hip) handles this pick on a grid of `grid`
// persistent workgroups.
int qs_pipe_supported(int n_rows, int n_vocab, int64_t row_stride, const void *logits, int grid);
// Dynamic LDS bytes of that kernel for a vocabulary width.
size_t qs_pipe_lds_bytes(int n_vocab);
// Rows are split in this many parts (the per-part scratch needs rows * parts entries).
int qs_pipe_parts(void);
// Cooperative launch of the pipelined pick on `stream`.
int qs_pipe_launch(const float *logits, int64_t row_stride, int n_rows, int n_vocab,
                   const qs::RowState &st, const qs::Scratch &sc, int32_t *out,
                   qs_pick_diag *diag, int grid, hipStream_t stream);
