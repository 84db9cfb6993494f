// Wide decode (decode_wide.hip): every decode step of a greedy batch of up to 8 sequences in one
// cooperative launch, for models whose weights do not fit on the chip (c4: 494 MB) or whose
// contexts are long (c5: 4096 keys) -- the shapes the relay, grouped and persistent kernels
// refuse, which otherwise take ~5 dependent launches per layer (each 5-15 us of ramp and
// memory latency for a few megabytes).
//
// All G workgroups (one per CU) take part in every product, each streaming its own slice of
// the weights from HBM straight into registers one hand-off ahead of its use, so the weight
// stream overlaps the hand-off waits.  Every workgroup keeps the whole residual stream x[B][C]
// in LDS and recomputes the LayerNorms itself; per layer and step, hand-offs through
// {payload, epoch} exchange words (agent-scope stores and polls, as the other decode kernels);
// seven per layer:
//   H1  dx2 of the previous layer (every WG gathers B C words)  -> x += dx2, LN0, QKV rows
//                                                               -> q / k_new / v_new words
//   H2  attention items: (sequence, head, key slice), S = G / (B H) slices per pair; the last
//       slice takes the step's own key from the words and writes it to the caches
//                                                              -> (max, sum, P.V) records
//   H3  one WG per (sequence, head) merges its S records in slice order -> y words
//   H4  every WG gathers y, attention-projection rows          -> dx1 words
//   H5  every WG gathers dx1: x += dx1, LN1, FC rows + GELU      -> h words
//   H6  teams of 8 WGs share their FC columns (h of the team's rows); each member forms the
//       MLP-projection partials of its C / 8 outputs over those columns -> B C / 8 words per WG
//   H7  WG w adds, for its C / G outputs, the 32 team partials in team order -> dx2 words
// then, after the last layer, x += dx2, ln_f, lm_head rows (balanced over the WGs, streamed),
// per-WG first-maximum candidates, and every WG picks the tokens from the G candidates itself.
#pragma once

#include "decode_persistent.h"

namespace fmlh {

constexpr int kWideMaxBatch = 8;   // sequences of one launch (compile-time bound of the row loops)
constexpr int kWideHD = 64;        // head_dim compiled
constexpr int kWideMaxT = 4096;    // block_size

// One layer's weights as the wide kernel reads them (rows are contiguous).
struct WideLayer {
    const float* wqkvT;  // 3C x C
    const float* wproj;  // C x C
    const float* wfcT;   // 4C x C
    const float* w2;     // 4C x C: W_proj2 as FreeML stores it (row j = input j of every output)
    const float *ln0g, *ln0b, *ln1g, *ln1b;  // LayerNorm gains and biases (biases may be null)
};

struct WideArgs {
    int B, C, H, L, V, T, HS, Bmax;
    int G;                       // workgroups
    int S;                       // attention items (key slices) per (sequence, head) pair
    int n_steps, pos0, gen0;
    uint32_t epoch_base;
    float scale;
    const WideLayer* layers;     // device array of L entries
    const float *tok, *pos_emb, *lnf_g, *lnf_b, *lm;
    float *kc, *vc;              // [L][Bmax][H][T][hd]
    int32_t* hist;               // [Bmax][HS]
    int* st_pos;                 // {pos, gen} after the launch
    float* logits;               // [B][V] (last step)
    float* logit_hist;           // optional [slots][B][V]
    size_t hist_slots;
    // Exchange words (epoch per (step, layer, hand-off), wide_epochs() per launch):
    uint64_t* wq;     // [B][3C]      q, k_new, v_new
    uint64_t* wpart;  // [P S <= G][hd + 2] attention records (max, sum, P.V)
    uint64_t* wy;     // [B][C]
    uint64_t* wdx1;   // [B][C]
    uint64_t* wh;     // [B][4C]      FC outputs (after GELU)
    uint64_t* wp2;    // [G][32][B][C / G]  MLP-projection partials: owner, team, sequence, output
    uint64_t* wdx2;   // [B][C]
    uint64_t* wcand;  // [G][B][2]    first-maximum candidates (value, index)
    unsigned* err;
    // Optional timeline (FMLH_WIDE_TRACE): device wall clock (100 MHz) of every WG at
    // kWideTracePoints points of step trace_step: [WG][12 l + k] for layer l (k: 0 start, 1 LN0
    // done, 2 QKV out, 3 attention item out, 4 merge out, 5 y in, 6 projection out, 7 dx1 in,
    // 8 FC done, 9 partials out, 10 partials in, 11 dx2 out), [WG][12 L + k] for the lm_head
    // (0 x in, 1 logits done, 2 candidate out, 3 tokens in); models deeper than the buffer
    // (12 L + 4 > kWideTracePoints) decode untraced.
    unsigned long long* trace;
    int trace_step;
};

constexpr int kWideTracePoints = 160;

struct WidePlan {
    bool ok = false;
    int G = 0, S = 0;
    size_t smem = 0;
};

// Whether the wide kernel decodes B sequences of this shape on `cus` CUs (head_dim 64, n_embed
// 256 / 512 / 768 / 1024, block_size <= 4096, B <= 8, B * n_head <= CUs).
WidePlan wide_plan(int B, int C, int H, int L, int V, int T, int cus);
// Exchange words per buffer for up to Bmax sequences: {wq, wpart, wy/wdx1/wdx2 each, wp2, wcand, wh}.
void wide_words(int C, int H, int Bmax, int G, int S_max, size_t out[6]);
// Epochs one launch of n_steps steps uses.
constexpr unsigned kWideHops = 7;  // exchange-word hand-offs per layer (q, attention records, y, dx1, h, partials, dx2)
inline uint64_t wide_epochs(int L, int n_steps) { return (uint64_t)n_steps * (kWideHops * L + 1u) + 1u; }
int wide_decode(const WideArgs& a, const WidePlan& p, hipStream_t s);

}  // namespace fmlh
