// qs_launch.h - host-side entry points between the HIP translation units (C++ only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "qs_device.h"

// ---- the streaming kernel (qs_part.hip) ----

// Parts per row the streaming kernel supports (lanes of its row decision), wavefronts of
// its workgroups (one candidate list each) and candidates per part.
#define QS_PART_MAX_PARTS 64
#define QS_PART_WAVES 8
#define QS_PART_CANDS 256

// Whether the streaming kernel handles this pick (16-byte aligned rows, vocabulary and row
// stride multiples of 4, at most QS_PART_MAX_PARTS parts).
int qs_part_supported(int n_rows, int n_vocab, int64_t row_stride, const void *logits);
// Parts per row at this vocabulary (the per-part scratch needs rows * parts entries).
int qs_part_parts(int n_vocab);
// Workgroups of the streaming kernel the device holds at once (0 when unknown).
int qs_part_resident(void);
// Enqueue the streaming pick on `stream`: the streaming kernel over a grid of about
// `resident` workgroups, then the decision kernel (ordinary launches: no workgroup waits
// for another).
// `mid`, when given, is recorded on the stream between the two kernels (timing).  When
// every row is greedy (`all_greedy`) and sc.gbest is set, each row is decided by its last
// part in the streaming kernel and the decision kernel is not launched.
int qs_part_launch(const float *logits, int64_t row_stride, int n_rows, int n_vocab,
                   const qs::RowState &st, const qs::Scratch &sc, int32_t *out,
                   qs_pick_diag *diag, int resident, hipStream_t stream,
                   hipEvent_t mid = nullptr, bool all_greedy = false);

// ---- the row kernel (qs_row.hip) ----

// Longest row the row kernel supports (its history bitmap is in LDS).
#define QS_ROW_MAX_VOCAB 262144
// Largest candidate target (top-k, or 64 when top-k is off) for which AUTO picks the row
// kernel; larger ones take the streaming kernels (the row kernel's lists hold 4096
// candidates a row at 8 wavefronts, 2048 at 16).
#define QS_ROW_AUTO_KSEL 256

// Whether the row kernel handles this pick (16-byte aligned rows, vocabulary and row
// stride multiples of 4, vocabulary at most QS_ROW_MAX_VOCAB).
int qs_row_supported(int n_rows, int n_vocab, int64_t row_stride, const void *logits);
// Enqueue the row pick on `stream`: one workgroup of `waves` (16 or 8) wavefronts per row.
int qs_row_launch(const float *logits, int64_t row_stride, int n_rows, int n_vocab,
                  const qs::RowState &st, const qs::Scratch &sc, int32_t *out,
                  qs_pick_diag *diag, int waves, hipStream_t stream);
// Workgroups of the row kernel with `waves` (16 or 8) wavefronts one CU holds at once (0
// when unknown): 1 and 2 by design (registers and LDS).
int qs_row_resident(int waves);
// The row kernel's timeline stamps (the timeline build only; QS_EINVAL otherwise).
int qs_row_timeline_read(uint64_t *dst, int n);

// ---- the output layer with the sampler's streaming pass (qs_head.hip) ----

#define QS_HEAD_TILE 128                 // vocabulary columns per tile workgroup
#define QS_HEAD_MAX_ROWS 256             // rows (hidden states) per pick
#define QS_HEAD_MAX_VOCAB 262144
#define QS_HEAD_MAX_TILES (QS_HEAD_MAX_VOCAB / QS_HEAD_TILE)

// What k_head's epilogue records per (row, tile of QS_HEAD_TILE columns): the penalised
// max and min keys, the NaN count, and the certified sums of the tile's terms against the
// integer exponent base c (qs_cert.h: sum of e^, sum of e^ * (-t)).
struct HeadRec {
    uint32_t maxk, mink;
    int32_t nan;
    float c;
    double sum, term;
};

// The history bitmap of the pick's rows (hbits zero before; the output layer's epilogue
// clears the bits it reads), and the row decisions from the tile records and the written
// logits: shared by both output layers.
int qs_head_prep_launch(int n_rows, int n_vocab, const qs::RowState &st, uint32_t *hbits,
                        hipStream_t stream);
int qs_head_decide_launch(float *d_logits, int n_rows, int n_vocab, const qs::RowState &st,
                          const qs::Scratch &sc, HeadRec *rec, int32_t *out, qs_pick_diag *diag,
                          hipStream_t stream);

// ---- the output layer at the reference's arithmetic (qs_head_exact.hip) ----

// Whether the exact layer takes this weight type and embedding size; the packed matrix's
// bytes (0: not taken).
int qs_head_exact_shape_ok(int wtype, int n_embd);
size_t qs_head_exact_bytes(int wtype, int n_embd, int n_vocab);
// Enqueue: the GGUF rows at d_weight (n_vocab rows of wtype) into the packed layout.
int qs_head_exact_pack_launch(const void *d_weight, int wtype, int n_embd, int n_vocab,
                              void *d_packed, hipStream_t stream);
// Enqueue: d_logits[n_rows][n_vocab] from the packed matrix and d_xn[n_rows][n_embd]
// (n_rows <= QS_HEAD_EXACT_MAX_ROWS); with rec, also the tile records for
// qs_head_decide_launch (the repeat penalty from the rows' rings, read by each workgroup).
int qs_head_exact_launch(const void *d_packed, int wtype, const float *d_xn, int n_embd,
                         int n_rows, int n_vocab, float *d_logits, const qs::RowState &st,
                         HeadRec *rec, hipStream_t stream);

// Elements of the packed output matrix (the vocabulary rounded up to whole tiles).
size_t qs_head_packed_elems(int n_embd, int n_vocab);
// Enqueue on `stream`: the bf16 [n_vocab][n_embd] output matrix into the tile order the
// output-layer kernel reads (qs_head_packed_elems elements at d_packed).
int qs_head_pack_launch(const void *d_weight, int n_embd, int n_vocab, void *d_packed,
                        hipStream_t stream);
// Enqueue on `stream`: logits = hidden . weight^T (bf16 [n_rows][n_embd] and the packed
// [n_vocab][n_embd] matrix, fp32 accumulation) into d_logits[n_rows][n_vocab]; with `out`, also
// the pick of every row from them (rec: n_rows x ceil(n_vocab / QS_HEAD_TILE) records,
// hbits: (QS_HEAD_MAX_ROWS / 32) x n_vocab words, zero before the call and left zero).
int qs_head_launch(const void *d_hidden, const void *d_weight, int n_embd, int n_rows,
                   int n_vocab, float *d_logits, const qs::RowState &st, const qs::Scratch &sc,
                   HeadRec *rec, uint32_t *hbits, int32_t *out, qs_pick_diag *diag,
                   hipStream_t stream);
