// Persistent decode kernel interface (see decode_persistent.hip).
#pragma once

#include "fmlh_internal.h"

namespace fmlh {

constexpr int kMaxPersistBatch = 8;

// One layer's weights as the persistent kernel reads them: one output per contiguous row.
struct PersistLayer {
    const float* wqkvT;  // 3C x C   (W_qkv transposed)
    const float* wproj;  // C x C    (stored out x in already)
    const float* wfcT;   // 4C x C   (W_fc transposed)
    const float* w2T;    // C x 4C   (W_proj2 transposed)
    const float *ln0g, *ln0b, *ln1g, *ln1b;
};

struct PersistArgs {
    int B, C, H, L, V, T, HS, Bmax;
    int key_chunk, max_chunks;
    int wcap;                    // LDS floats reserved for a hop's weight slice
    int n_steps, pos0, gen0;
    uint32_t epoch_base;
    float scale;
    const PersistLayer* layers;  // device array of L entries
    const float *tok, *pos_emb, *lnf_g, *lnf_b, *lm;
    float *kc, *vc;              // [L][Bmax][H][T][hd]
    int32_t* hist;               // [Bmax][HS]
    int* st_pos;                 // {pos, gen} updated at the end
    float* logits;               // B x V (last step)
    float* logit_hist;           // optional [slots][B][V]
    size_t hist_slots;
    uint64_t *q, *kn, *vn, *att, *dx1, *hb, *dx2, *am;  // exchange words
    unsigned* err;
    unsigned long long* trace;   // optional: WG 0 timestamps (kTracePoints per step, 4 steps)
};

constexpr int kTraceSteps = 4;
constexpr int kTracePoints = 128;

struct PersistPlan {
    bool ok = false;
    int G = 0, wcap = 0, key_chunk = 64, max_chunks = 0;
    size_t smem = 0;
};

size_t smem_limit();
// Whether (and how) the persistent kernel runs this shape on a device with `cus` CUs.
PersistPlan persist_plan(int B, int C, int H, int L, int V, int T, int cus);
int persist_decode(const PersistArgs& a, const PersistPlan& p, int hd, hipStream_t s);
// out (cols x rows) = in (rows x cols)^T.
int persist_transpose(float* out, const float* in, int rows, int cols, hipStream_t s);

}  // namespace fmlh
