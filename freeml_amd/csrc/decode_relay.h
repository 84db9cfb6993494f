// Relay decode (decode_relay_kernel.h, decode_relay.hip): every decode step of a batch of up to
// kRelayMaxBatch sequences in one cooperative launch, with each product computed by a small
// team of workgroups.
//
// The persistent kernel (decode_persistent_kernel.h) spreads every product over all 256
// workgroups, so each of its 31 hand-offs per token is an all-to-all among 256 producers
// (~2.65 us each on MI355X).  A hand-off among a few producers costs about half of that
// (16 -> 16 workgroups: ~1.5 us, see the exchange probe), so here each product of each layer
// has its own team, whose weight slice stays in its registers for the whole launch:
//   Q(l, i)  nq workgroups: x_l, LN0, 96 rows of W_qkv^T                -> q, k_new, v_new
//   A(l, h)  one per head:  attention of head h, then its share of the attention projection
//                           (W_proj columns of the head, every output)  -> dx1 partial of h
//   F(l, i)  nf workgroups: x_l + the H dx1 partials, LN1, 64 rows of W_fc^T, GELU -> its 64
//                           entries of h; then the proj2 partial of every output over those
//                           64 columns of W_proj2 (a column split: h never travels)
//                                                                       -> dx2 partial of i
//                           then, for its C / nf rows, x' + the nf partials in team order
//                                                                       -> rows of x_{l+1}
//   lm       one:           x_L, ln_f, lm_head rows, first maximum     -> the next token, and
//                           its embedding (token + position rows)      -> x_0 of the next step
// so a token costs 4 hand-offs per layer plus the lm_head's, each among at most 24 producers,
// and no workgroup gathers more than H C + C words per hand-off (the exchange cost grows with
// the words a consumer gathers).  Two other team cuts: at batch 1 (qa) each attention role
// forms its head's q itself and the Q team only k_new / v_new; from kRelayBigBatch sequences
// (big) the Q team has 192-row slices (half the workgroups) and the row sums move from the FC
// team to a team of their own,
//   F2(l, k) nf2 workgroups: for its C / nf2 rows, x' (published by the FC team) + the nf
//                           partials in team order                     -> rows of x_{l+1}
// so that no FC workgroup waits for the others' partials (with them in the FC team, the team
// moves at its slowest member's pace); from kRelaySplitBatch (split) each head also has two
// attention workgroups and the model two lm_head workgroups, each taking every other sequence,
// paid for with FC slices of 96 rows; from kRelayHBatch at n_embed 384 (the h cut) the MLP
// projection moves to the F2 team as a row split:
//   F(l, i)  12 workgroups: x_l + the dx1 partials, LN1, 128 rows of W_fc^T, GELU -> h words
//   F2(l, k) 12 workgroups: all 4C words of h, 32 rows of W_proj2, x' -> rows of x_{l+1}
// so the FC and F2 teams share the MLP's work.  Roles run in step order; role r goes to
// workgroup r mod G, so when there are more roles than workgroups a workgroup takes two, far
// apart in the step (it reloads its weights in between); the others keep theirs for the whole
// launch.
//
// A batch flows through the teams as a pipeline: every role takes the batch's sequences in
// order, each with its own exchange words, so while the lm_head role picks sequence b's token
// the earlier teams already work on sequences b + 1, b + 2, ..., and sequence b's next step
// starts as soon as its token exists.  A step then costs about the busiest team's time for the
// batch, or one sequence's latency through all teams when that is longer.
#pragma once

#include "decode_persistent.h"

namespace fmlh {

constexpr int kRelayMaxT = 256;                 // K/V rows of a head held in registers
constexpr int kRelayMaxBatch = 64;              // sequences of one launch
constexpr int kRelayLagBatch = 32;              // batches from which F's row sums lag two items
constexpr int kRelayDefaultMaxBatch = 64;       // above (FMLH_RELAY=1 aside): the grouped kernel by default
constexpr int kRelayTeamRows = 96;              // rows of W_qkv^T per Q workgroup
constexpr int kRelayQaMaxBatch = 1;             // up to this batch each attention role forms its q
constexpr int kRelayBigBatch = 16;              // from this batch: the big team cut
constexpr int kRelayBigTeamRows = 192;          // rows of W_qkv^T per Q workgroup (big)
constexpr int kRelayF2Rows = 64;                // rows of x_{l+1} per F2 workgroup (big)
constexpr int kRelaySplitBatch = 16;            // from this batch (big, n_embed 256 / 384): the split cut
constexpr int kRelaySplitFRows = 96;            // rows of W_fc^T per F workgroup (split)
constexpr int kRelayHBatch = 33;                // from this batch (split, n_embed 384): the h cut
constexpr int kRelayHRows = 128;                // rows of W_fc^T per F workgroup (h cut)
constexpr int kRelayHF2Rows = 32;               // rows of W_proj2 (of x_{l+1}) per F2 workgroup (h cut)
constexpr int kRelayFRows = 64;                 // rows of W_fc^T (columns of W_proj2^T) per F workgroup
constexpr int kRelayMaxVocab = 96;              // lm_head rows held by the lm workgroup
constexpr int kRelayTraceSteps = 4;             // steps of a launch the timeline covers
constexpr int kRelayTracePoints = 8;            // per role and step (decode_relay_kernel.h: stamp, Meter)

struct RelayArgs {
    int B, L, V, T, HS, Bmax;
    int nq, nf, nf2;             // workgroups per layer of the QKV, FC and row-sum teams
    int nA, nlm;                 // attention workgroups per head, lm_head workgroups (split: 2;
                                 // each takes every nA-th / nlm-th sequence)
    int roles;                   // L (nq + nA H + nf + nf2) + nlm
    int n_steps, pos0, gen0;
    int lag_rows;                // F adds up an item's rows two items later (large batches)
    uint32_t epoch_base;
    float scale;
    const PersistLayer* layers;  // device array of L entries
    const float *tok, *pos_emb, *lnf_g, *lnf_b, *lm;
    float *kc, *vc;              // [L][Bmax][H][T][hd]
    int32_t* hist;               // [B][HS]
    int* st_pos;                 // {pos, gen} after the launch
    float* logits;               // [B][V] (last step)
    float* logit_hist;           // optional [slots][B][V]
    size_t hist_slots;
    // Exchange words, each written once per step (epoch = epoch_base + step + 1):
    uint64_t* xw;     // [L + 1][B][C]: x entering layer l (l = 0: the lm_head role's next
                      // embedding; l = L feeds lm_head)
    uint64_t* partw;  // [L][B][nf][C]: dx2 partials of the FC team
    uint64_t* qkvw;   // [L][B][3C]
    uint64_t* dx1w;   // [L][B][H][C]: per-head attention-projection partials
    uint64_t* xpw;    // [L][B][C]: x' = x + the dx1 partials, from the FC team (big)
    unsigned* err;
    // Optional timeline (FMLH_RELAY_TRACE): device wall clock (100 MHz) at kRelayTracePoints
    // points of every role in the first kRelayTraceSteps steps, for sequence 0:
    // [step][role][point].
    unsigned long long* trace;
};

struct RelayPlan {
    bool ok = false;
    bool qa = false;   // q formed by the attention roles (the Q team: k / v rows only)
    bool big = false;    // 192-row Q slices, row sums in their own team (nf2)
    bool split = false;  // big, and two attention / lm_head workgroups per head / model (384: 96-row FC slices)
    bool hcut = false;   // split at 384, with the MLP projection in the F2 team (FC team: h only)
    int nq = 0, nf = 0, nf2 = 0, nA = 1, nlm = 1, roles = 0, G = 0;
    size_t smem = 0;
};

// Whether (and how) the relay kernel decodes B sequences of this shape on `cus` CUs.
RelayPlan relay_plan(int B, int C, int H, int L, int V, int T, int cus);
// Exchange words the buffers above need: {xw, partw, qkvw, dx1w, xpw} for L layers and B
// sequences.
void relay_words(int C, int H, int L, int B, size_t out[5]);
int relay_decode(const RelayArgs& a, const RelayPlan& p, int C, int hd, hipStream_t s);

}  // namespace fmlh
