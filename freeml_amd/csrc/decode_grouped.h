// Grouped persistent decode (decode_grouped_kernel.h, decode_grouped.hip): batches of more than
// one group of sequences in one cooperative launch per decode call.
#pragma once

#include "decode_persistent.h"

namespace fmlh {

constexpr int kGroupBatch = 8;   // sequences per group: the batch columns of the MFMA tiles
constexpr int kMaxGroups = 8;    // groups per launch (64 sequences)
constexpr int kGroupedMaxT = 256;  // attention keys per (sequence, head) held in registers
constexpr int kMaxGroupWGs = 48;   // workgroups per group at most (also below the argmax gather's 128)

struct GroupedArgs {
    int B, L, V, T, HS, Bmax;
    int groups, Bg;              // group k decodes sequences [k Bg, k Bg + Bg) (the last may have fewer)
    size_t gw_c, gw_am;          // exchange words per group: C-long rows (x Bg), argmax candidates
    int n_steps, pos0, gen0;
    uint32_t epoch_base;
    float scale;
    const PersistLayer* layers;  // device array of L entries (rows of every product contiguous)
    const float *tok, *pos_emb, *lnf_g, *lnf_b, *lm;
    float *kc, *vc;              // [L][Bmax][H][T][hd]
    int32_t* hist;               // [Bmax][HS]
    int* st_pos;                 // {pos, gen} after the launch
    float* logits;               // B x V (last step)
    float* logit_hist;           // optional [slots][B][V]
    size_t hist_slots;
    // Exchange words, per group (pointer + group * words per group).  q, k_new and v_new of all
    // groups are one array: k_new = q + qkv_stride, v_new = q + 2 qkv_stride.  part: the proj2
    // partial sums, [group][workgroup][kGroupBatch][C] (256 * kGroupBatch * C words in all).
    uint64_t *q, *y, *dx1, *part, *dx2, *am;
    size_t qkv_stride;
    unsigned* err;
    // Optional timeline (FMLH_GROUPED_TRACE): device wall clock (100 MHz) at kGroupedTracePoints
    // points of the first kGroupedTraceSteps steps, for workgroups 0 .. kGroupedTraceWGs - 1:
    // slot 0 the step start, 1 + 16 l + k point k of layer l (the names are in
    // freeml_amd/timeline.py), 1 + 16 L + 0 / 1 the lm_head products / the token pick.
    unsigned long long* trace;
};

constexpr int kGroupedTraceSteps = 2;
constexpr int kGroupedTracePoints = 128;
constexpr int kGroupedTraceWGs = 256;

struct GroupedPlan {
    bool ok = false;
    int groups = 0, Bg = 0, G = 0;  // G workgroups per group, one per CU
    int tq = 0;                     // 16-row tiles of the 3C / 4C-row products per workgroup
    size_t smem = 0;
};

// Whether (and how) the grouped kernel decodes B sequences of this shape on `cus` CUs.
GroupedPlan grouped_plan(int B, int C, int H, int L, int V, int T, int cus);
// Exchange words per group for groups of up to kGroupBatch sequences and up to G_max
// workgroups: {C-long rows, argmax candidates}; the proj2 partials take 256 kGroupBatch C
// words for all groups together.
void grouped_group_words(int C, int G_max, size_t out[2]);
int grouped_decode(const GroupedArgs& a, const GroupedPlan& p, int C, int hd, hipStream_t s);

}  // namespace fmlh
