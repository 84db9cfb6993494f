// Attention entry points used by the token loop (see attention.hip).
#pragma once

#include "fmlh_internal.h"

namespace fmlh {

bool attn_head_dim_supported(int hd);

// Copies the K and V thirds of qkv rows into the cache ([seq][head][pos][hd] for one layer).
int kv_scatter(const float* qkv, int qkv_ld, float* kc, float* vc, int rows, int rows_per_seq,
               int C, int H, int T, const int* d_pos, int pos0, hipStream_t s);

// Causal attention for `batch` sequences of rows_per_seq rows starting at position 0.
int attn_prefill(const float* qkv, int qkv_ld, const float* kc, const float* vc, float* y,
                 int y_ld, int batch, int rows_per_seq, int H, int HDv, int T, float scale,
                 hipStream_t s);

// Floats of workspace attn_decode needs for up to max_batch sequences (0 when one chunk covers
// block_size).  Zero it once before the first call: its head holds one arrival count per
// (sequence, head) of max_batch sequences, which every call leaves at zero, at offsets that do
// not depend on the batch of a call (the chunk partials follow them).
size_t attn_decode_workspace(int max_batch, int H, int HDv, int T);

// One query row per sequence at position *d_pos against cached keys 0..*d_pos.
// qkv_splits > 0: qkv holds that many split-K partial sums of the QKV product ([split][batch]
// [qkv_ld]; 1: the product itself); the kernel reduces them and writes the step's K / V rows to
// the caches itself.
// ws: attn_decode_workspace(max_batch, ...) floats, batch <= max_batch.
int attn_decode(const float* qkv, int qkv_ld, float* kc, float* vc, float* y, int y_ld,
                int batch, int H, int HDv, int T, const int* d_pos, float scale, float* ws,
                int max_batch, hipStream_t s, int qkv_splits = 0);

}  // namespace fmlh
