// Persistent decode kernel interface (decode_persistent.hip, decode_persistent_kernel.h).
#pragma once

#include "fmlh_internal.h"

namespace fmlh {

constexpr int kMaxPersistBatch = 8;    // sequences per group (the compile-time batch tile)
constexpr int kMaxPersistGroups = 8;   // groups per launch: up to 64 sequences
constexpr int kPersistItemKeys = 64;  // keys per attention item (one WG)
constexpr int kMaxPersistG = 256;     // workgroups of the persistent kernel at most
// Returned (never past the C ABI) when the runtime refuses the cooperative launch: the
// device's cooperative-launch resource (global wave sync) can be held by one process at a
// time, so a second process that decodes meanwhile takes the graph path instead.
constexpr int kPersistRefused = -100;

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
    // The launch's WGs form `groups` equal groups; group k decodes sequences [k Bg, k Bg + Bg)
    // (the last one may have fewer) with its own slices of the exchange buffers.
    int groups, Bg;
    size_t gw_qkv, gw_att, gw_c, gw_h4, gw_am;  // words per group: q/kn/vn (each), att, dx, h, am
    int max_chunks;              // key chunks of kPersistItemKeys keys at the largest position
    int h4p;                     // LDS row length of 4C-long rows (multiple of 512 floats)
    int wcap;                    // LDS floats of one weight-slice buffer (two are kept)
    int ufloats;                 // LDS floats of the shared region (partials, h rows, ...)
    int kv_sep;                  // K/V rows have their own LDS region (else they share U)
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
    int G = 0;         // workgroups per group (one per CU)
    int groups = 1, Bg = 1;  // sequence groups and sequences per group
    int bt = 0;        // compile-time batch tile: 1, 2, 4 or 8 rows
    int nqc = 0;       // C-long rows padded to 256 * nqc floats in LDS
    int h4p = 0, wcap = 0, ufloats = 0, max_chunks = 0;
    bool kv_sep = false;
    size_t smem = 0;
};

size_t smem_limit();
// Whether (and how) the persistent kernel runs this shape on a device with `cus` CUs.  The
// workgroup count per group depends on C, the device and the group count only
// (FMLH_PERSIST_G overrides it for tuning).
PersistPlan persist_plan(int B, int C, int H, int L, int V, int T, int cus);
// Per-group words of each exchange buffer when groups hold up to Bg_max sequences and up to
// G_max WGs: {q/kn/vn each, att, dx1/dx2 each, h, am}.
void persist_group_words(int C, int H, int hd, int max_chunks, int G_max, int Bg_max, size_t out[5]);
int persist_decode(const PersistArgs& a, const PersistPlan& p, int hd, hipStream_t s);
// out (cols x rows) = in (rows x cols)^T.
int persist_transpose(float* out, const float* in, int rows, int cols, hipStream_t s);

// Per-head-dimension launchers (decode_persistent_hd*.hip).
int persist_launch_hd16(const PersistArgs& a, const PersistPlan& p, hipStream_t s);
int persist_launch_hd32(const PersistArgs& a, const PersistPlan& p, hipStream_t s);
int persist_launch_hd64(const PersistArgs& a, const PersistPlan& p, hipStream_t s);

}  // namespace fmlh
