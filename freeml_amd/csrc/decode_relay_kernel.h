// Relay decode kernel (see decode_relay.h for the team layout and the batch pipeline).
//
// Step s of a launch decodes position pos = pos0 + s of every sequence.  Every exchange word of
// the step carries epoch e(s) = epoch_base + s + 1 and every word is written once per step, so
// one epoch per step suffices.  Single buffers are safe because every consumer of a sequence's
// word reads it before it publishes its own outputs for that sequence, and everything it
// publishes leads to that sequence's next token: a word is only rewritten (next step) after the
// token of this step exists, i.e. after all its consumers have read it.  Every role takes the
// work in the same order (step, then sequence) and waits only for earlier roles of the same
// (step, sequence) or for the lm_head role's token of the step before, so the waits cannot
// form a cycle.
//
// Eight waves per workgroup (two per SIMD).  Products are VALU dot products with DPP reductions
// and the weights in registers (wr), loaded when the role starts:
//   rows of K = C (Q, F, lm): 16 lanes per row, row 32 p + 4 wave + g in pass p (g = lane / 16),
//                  lane t holding columns 4 (16 j + t) .. of the row in wr[NE p + j]
//   F's proj2 columns: output 64 p + 8 wave + lane / 8, columns 96 idx + 12 (lane % 8) .. in
//                  wr[3 NE + 3 p + c] (8 lanes per output)
//   A's share of W_proj: output 128 p + 16 wave + lane / 4, columns 64 h + 16 (lane % 4) ..
//                  in wr[4 p + c]
// A workgroup with one role loads its weights once, before the first step; one with two
// loads a role's weights when it starts the role, so they stream while it waits for that
// role's inputs.
//
// Attention (A): keys 0..pos-1 of one head, 16-key groups w, w + 8 per wave w (block_size <= 256:
// at most two groups), K/V rows in registers through bounded buffer loads (rows from pos on
// read as zero) requested before q is polled; key pos (k_new, v_new: the Q team's words) is
// folded into the merged rows last.  Small batches (QA) form each head's q in its attention
// role from x (W_q rows in LDS), so the Q team holds only the k / v rows and the role's first
// wait is for x, not for the Q team.  Then the head's share of the attention projection, and
// last the step's K/V cache rows (the only workgroup that reads them later is this one, the
// same role of later steps).
//
// Every wait is bounded (ll_keep_polling): a protocol error sets the error word and ends the
// kernel instead of hanging it.
#pragma once

#include "decode_relay.h"
#include "decode_persistent_kernel.h"

namespace fmlh {
namespace relay {

using persist::gelu_ref;
using persist::ll_float;
using persist::ll_issue_n;
using persist::ll_load;
using persist::ll_put;
using persist::ll_put_bits;
using persist::ll_settle_n;
using persist::quad_sum;
using persist::wave_argmax;

typedef float floatx4 __attribute__((ext_vector_type(4)));

// Eight waves per workgroup, two per SIMD: one wave issues a VALU instruction only every ~5
// cycles, a second one on the same SIMD runs at the same rate, so the products take half as long.
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kHD = 64;          // head_dim
constexpr int kKeyGroup = 16;    // keys per wave pass
constexpr int kGroupsPerWave = kRelayMaxT / kKeyGroup / kWaves;  // 2
constexpr int kRowsPerPass = 4 * kWaves;                         // rows of K = C per pass of the WG
constexpr int kPasses = kRelayTeamRows / kRowsPerPass;           // 3 (Q, lm)
constexpr int kBigPasses = kRelayBigTeamRows / kRowsPerPass;     // 6 (Q, big)
constexpr int kFPasses = kRelayFRows / kRowsPerPass;             // 2 (F)
constexpr int kScratch = 3 * kHD + kWaves * 256;                 // attention scratch (floats)
constexpr int kRawBufferFlags = 0x00020000;  // raw buffer, 32-bit data: loads past the records read 0
static_assert(kRelayTeamRows % kRowsPerPass == 0 && kRelayFRows % kRowsPerPass == 0 &&
                  kRelayMaxVocab <= kRelayTeamRows, "whole passes");
static_assert(kRelayFRows % 32 == 0, "F: 8 lanes per proj2 output, whole float4 columns");

enum RoleKind : int { kQ = 0, kA = 1, kF = 2, kLm = 3, kF2 = 4 };

// Lane and wave ids through an empty asm statement: per-lane addresses are then formed where
// they are used, not hoisted into registers held across the whole kernel.
__device__ __forceinline__ int thread_id() {
    int t = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(t));
    return t;
}
__device__ __forceinline__ int lane_id() { return thread_id() & 63; }
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(thread_id() >> 6); }

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// Barrier for LDS data only (__syncthreads would also wait for every global load in flight).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
#pragma clang diagnostic pop

__device__ __forceinline__ floatx4 lds4(const float* p) { return *reinterpret_cast<const floatx4*>(p); }
// Loads from global memory as such (global_load: the weight pointers come from a device table,
// so the compiler cannot tell their address space and would emit flat loads, which also count
// in lgkmcnt and so delay every LDS wait behind them).
typedef const __attribute__((address_space(1))) floatx4* gfloatx4_ptr;
typedef const __attribute__((address_space(1))) float* gfloat_ptr;
__device__ __forceinline__ floatx4 ld4(const float* p) { return *(gfloatx4_ptr)(p); }
__device__ __forceinline__ float ld1(const float* p) { return *(gfloat_ptr)(p); }
__device__ __forceinline__ float dot4(floatx4 a, floatx4 b) { return a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3]; }
// acc + a . b as four chained FMAs (one instruction per product).
__device__ __forceinline__ float fma4(floatx4 a, floatx4 b, float acc) {
    acc = fmaf(a[0], b[0], acc);
    acc = fmaf(a[1], b[1], acc);
    acc = fmaf(a[2], b[2], acc);
    return fmaf(a[3], b[3], acc);
}
__device__ __forceinline__ floatx4 bload4(__amdgpu_buffer_rsrc_t r, int e) {
    return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, e * 4, 0, 0));
}

template <int kCtrl>
__device__ __forceinline__ float row16_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}
// Sum over the 16 lanes of a DPP row, in every lane of the row (row_ror 8, 4, 2, 1).
__device__ __forceinline__ float row16_sum(float v) {
    v += row16_move<0x128>(v);
    v += row16_move<0x124>(v);
    v += row16_move<0x122>(v);
    v += row16_move<0x121>(v);
    return v;
}
// Sum over each group of 8 lanes, in every lane of the group (two quad permutations, then
// row_half_mirror: lane i of a half row takes lane 7 - i, which is in the other quad).
__device__ __forceinline__ float oct_sum(float v) {
    v += row16_move<0xb1>(v);   // quad_perm [1,0,3,2]
    v += row16_move<0x4e>(v);   // quad_perm [2,3,0,1]
    v += row16_move<0x141>(v);  // row_half_mirror
    return v;
}

struct Role {
    int kind, layer, idx, sub;  // sub: which of the every-n-th sequences an A / lm role takes
};

__device__ __forceinline__ Role role_of(const RelayArgs& a, int H, int r) {
    const int per = a.nq + a.nA * H + a.nf + a.nf2;
    Role ro;
    ro.layer = r / per;
    int o = r - ro.layer * per;
    if (ro.layer >= a.L) return Role{kLm, a.L, 0, o};  // lm_head role o of a.nlm
    if (o < a.nq) return Role{kQ, ro.layer, o, 0};
    o -= a.nq;
    if (o < a.nA * H) return Role{kA, ro.layer, o % H, o / H};  // head o % H, sequences o / H + nA k
    o -= a.nA * H;
    if (o < a.nf) return Role{kF, ro.layer, o, 0};
    return Role{kF2, ro.layer, o - a.nf, 0};
}

// Registers of a role kind's weights (float4): Q and lm kPasses NE rows of K = C; F kFPasses NE
// rows plus its proj2 columns (C / (8 kWaves) = NE passes of kRelayFRows / 32); A its share of
// W_proj, NE / 2 passes of 4, and under QA then its head's hd rows of W_q (kQaPasses NE, the
// layout of rows of K = C).
constexpr int kFCols4 = kRelayFRows / 32;  // float4 of proj2 columns per lane and pass
constexpr int kQaPasses = kHD / kRowsPerPass;
// (BIG: the Q team's kBigPasses NE; F2 holds no weights, one unused register.  FR: the FC
// team's rows per workgroup, FR / 32 passes and FR / 32 float4 of proj2 columns per pass.  The h
// cut, FR = kRelayHRows: F holds its FC rows only, and F2 its kRelayHF2Rows rows of W_proj2, K =
// 4C: lane t of a row's 16 holds float4 chunks t + 16 j, j < 4 NE.)
template <int NE, int K, bool QA, bool BIG, int FR>
constexpr int wr_count() {
    return K == kA    ? 2 * NE + (QA ? kQaPasses * NE : 0)
           : K == kF && FR == kRelayHRows ? (FR / kRowsPerPass) * NE
           : K == kF  ? (FR / kRowsPerPass) * NE + (FR / 32) * NE
           : K == kF2 && FR == kRelayHRows ? 4 * NE
           : K == kF2 ? 1
           : K == kQ && BIG ? kBigPasses * NE
                            : kPasses * NE;
}

// Requests the weights of role ro (of kind K) into wr.  Nothing waits for them here.  QA: each
// head's q is formed by its attention role, and the Q team holds only the k and v rows.
template <int NE, int K, bool QA, bool BIG, int FR>
__device__ __forceinline__ void load_weights(const RelayArgs& a, const Role& ro,
                                             floatx4 (&wr)[wr_count<NE, K, QA, BIG, FR>()]) {
    constexpr int C = 64 * NE;
    const int lane = lane_id(), wave = wave_id();
    if constexpr (K == kF2 && FR == kRelayHRows) {  // rows r0 + 4 wave + g of W_proj2 (w2T: [C][4C])
        const float* src = a.layers[ro.layer].w2T +
                           (size_t)(kRelayHF2Rows * ro.idx + 4 * wave + (lane >> 4)) * 4 * C + 4 * (lane & 15);
#pragma unroll
        for (int j = 0; j < 4 * NE; ++j) wr[j] = ld4(src + 64 * j);
    } else if constexpr (K == kF2) {
        wr[0] = floatx4{0.f, 0.f, 0.f, 0.f};
    } else if constexpr (K == kA) {
        const PersistLayer& lw = a.layers[ro.layer];
        const float* src = lw.wproj + (size_t)(16 * wave + (lane >> 2)) * C + kHD * ro.idx + 16 * (lane & 3);
#pragma unroll
        for (int p = 0; p < NE / 2; ++p)
#pragma unroll
            for (int c = 0; c < 4; ++c) wr[4 * p + c] = ld4(src + (size_t)p * 16 * kWaves * C + 4 * c);
        if constexpr (QA) {  // rows h hd + 32 p + 4 wave + g of W_qkv^T (the head's q rows)
            const int t = lane & 15, g = lane >> 4;
            const float* wq = lw.wqkvT + ((size_t)kHD * ro.idx + 4 * wave + g) * C + 4 * t;
#pragma unroll
            for (int p = 0; p < kQaPasses; ++p)
#pragma unroll
                for (int j = 0; j < NE; ++j) wr[2 * NE + NE * p + j] = ld4(wq + (size_t)kRowsPerPass * p * C + 64 * j);
        }
    } else {
        const float* src;
        int rows;
        if constexpr (K == kLm) {
            src = a.lm;
            rows = a.V;
        } else {
            const PersistLayer& lw = a.layers[ro.layer];
            const int team = K == kQ ? (BIG ? kRelayBigTeamRows : kRelayTeamRows) : FR;
            // Q: rows idx team of W_qkv^T, after the q rows under QA
            src = K == kQ ? lw.wqkvT + ((size_t)(QA ? C : 0) + (size_t)ro.idx * team) * C
                          : lw.wfcT + (size_t)ro.idx * team * C;
            rows = team;
            if constexpr (K == kF && FR != kRelayHRows) {  // W_proj2^T[o][FR idx + FR / 8 (lane % 8) ..], o = 64 p + 8 wave + lane / 8
                constexpr int FP = FR / kRowsPerPass, FC4 = FR / 32;
                const float* w2 = lw.w2T + (size_t)(8 * wave + (lane >> 3)) * 4 * C + FR * ro.idx + 4 * FC4 * (lane & 7);
                static_assert(C / (8 * kWaves) == NE && FP * NE + FC4 * NE == wr_count<NE, K, QA, BIG, FR>(),
                              "F registers");
#pragma unroll
                for (int p = 0; p < NE; ++p)
#pragma unroll
                    for (int c = 0; c < FC4; ++c)
                        wr[FP * NE + FC4 * p + c] = ld4(w2 + (size_t)p * 8 * kWaves * 4 * C + 4 * c);
            }
        }
        const int t = lane & 15, g = lane >> 4;
        constexpr int P = K == kF ? FR / kRowsPerPass : K == kQ && BIG ? kBigPasses : kPasses;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const float* w = src + (size_t)min(kRowsPerPass * p + 4 * wave + g, rows - 1) * C + 4 * t;
#pragma unroll
            for (int j = 0; j < NE; ++j) wr[NE * p + j] = ld4(w + 64 * j);
        }
    }
}

// The role's rows (wr, layout above) times xn (LDS).  emit(row, value) runs once per row, after
// the last pass, in lane t == p of the row's 16 lanes (which keeps pass p's sum); rows >= `rows`
// emit nothing.
template <int NE, int P = kPasses, class Emit>
__device__ __forceinline__ void gemv_regs(const floatx4* wr, const float* xn, int rows, Emit emit) {
    const int lane = lane_id(), wave = wave_id();
    const int t = lane & 15, g = lane >> 4;
    floatx4 xq[NE];
#pragma unroll
    for (int j = 0; j < NE; ++j) xq[j] = lds4(xn + 4 * (16 * j + t));
    float mine = 0.f;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < NE; ++j) acc = fma4(wr[NE * p + j], xq[j], acc);
        acc = row16_sum(acc);
        mine = t == p ? acc : mine;
    }
    const int row = kRowsPerPass * t + 4 * wave + g;
    if (t < P && row < rows) emit(row, mine);
}

// LayerNorm applied after the product: for a row w, LN(x).w = inv_std (sum w g x - mean sum w g)
// + sum w b, so the product runs on g x (written while x arrives) while every wave forms x's mean
// and 1 / std itself (layer_norm's two-pass order), and no wave waits for a normalised row.
// gx: g[o] of thread o < C; sg, sb: the emitting lane's row sums of w g and w b, formed by
// gemv_regs when the role starts (so they sit in the lanes that emit those rows later).
struct LnPost {
    float gx, sg, sb;
};
template <int NE, int P>
__device__ __forceinline__ LnPost ln_post_setup(const floatx4* wr, float* xn, const float* g, const float* b,
                                                int rows) {
    constexpr int C = 64 * NE;
    LnPost lp{0.f, 0.f, 0.f};
    const int o = thread_id();
    if (o < C) xn[o] = lp.gx = ld1(g + o);
    lds_barrier();
    gemv_regs<NE, P>(wr, xn, rows, [&](int, float v) { lp.sg = v; });
    lds_barrier();
    if (o < C) xn[o] = b ? ld1(b + o) : 0.f;
    lds_barrier();
    gemv_regs<NE, P>(wr, xn, rows, [&](int, float v) { lp.sb = v; });
    lds_barrier();
    return lp;
}
// Mean and 1 / std of the C floats at xs, in every lane of every wave (layer_norm's order).
template <int NE>
__device__ __forceinline__ void ln_stats(const float* xs, float& mean, float& inv_std) {
    constexpr int C = 64 * NE;
    const int lane = lane_id();
    float v[NE];
#pragma unroll
    for (int m = 0; m < NE; ++m) v[m] = xs[lane + 64 * m];
    float s = 0.f;
#pragma unroll
    for (int m = 0; m < NE; ++m) s += v[m];
    mean = wave_sum(s) * (1.0f / C);
    float q = 0.f;
#pragma unroll
    for (int m = 0; m < NE; ++m) {
        const float d = v[m] - mean;
        q += d * d;
    }
    inv_std = __builtin_amdgcn_rsqf(wave_sum(q) * (1.0f / C) + 1e-5f);  // v_rsq_f32: 1 ulp
}
__device__ __forceinline__ float ln_apply(const LnPost& lp, float v, float mean, float inv_std) {
    return (v - mean * lp.sg) * inv_std + lp.sb;
}

// ---- polled inputs -------------------------------------------------------------------------

// N exchange words at base + k kStride bytes (k < N), plus the lane's `off` bytes, in flight:
// poll_issue loads them all; poll_settle then loads the stale ones again in rounds until every
// one carries `ep` (wave-uniform exit, as ll_settle_n).  Buffer loads with sc1 (the agent-scope
// coherent load that ll_load is), so a word's address is an SGPR offset from the lane's and no
// 64-bit address is held per word; each round starts with a compiler memory barrier, so no load
// of a round is merged with or hoisted above an earlier one.
constexpr int kPollAux = 0x10;  // sc1
template <int N, int kStride>
struct Poll {
    const uint64_t* base;
    int off;
    uint32_t ep;
    uint64_t v[N];
};
template <int N, int kStride>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t poll_rsrc(const uint64_t* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(base), 0, N * kStride, kRawBufferFlags);
}
template <int N, int kStride>
__device__ __forceinline__ void poll_issue(Poll<N, kStride>& p, const uint64_t* base, int off, uint32_t ep) {
    p.base = base;
    p.off = off;
    p.ep = ep;
    const auto r = poll_rsrc<N, kStride>(base);
#pragma unroll
    for (int k = 0; k < N; ++k)
        p.v[k] = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(r, off, k * kStride, kPollAux));
}
template <int N, int kStride>
__device__ __forceinline__ void poll_settle(Poll<N, kStride>& p, int* bail, unsigned* err) {
    const auto r = poll_rsrc<N, kStride>(p.base);
    int it = 0;
    while (true) {
        bool stale = false;
#pragma unroll
        for (int k = 0; k < N; ++k) stale |= !persist::ll_current(p.v[k], p.ep);
        if (__builtin_amdgcn_ballot_w64(stale) == 0 || !persist::ll_keep_polling(it, bail, err)) return;
        asm volatile("" ::: "memory");
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const bool need = !persist::ll_current(p.v[k], p.ep);
            uint64_t nv = p.v[k];
            if (need) nv = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(r, p.off, k * kStride, kPollAux));
            p.v[k] = need ? nv : p.v[k];
        }
    }
}

// ---- work items ------------------------------------------------------------------------------

// A role's work comes as items (step, sequence), taken in that order.
struct Item {
    int step, b;
};
// The item after it within steps [0, s1); false past the last.
__device__ __forceinline__ bool next_item(const RelayArgs& a, Item it, int s1, Item& nx) {
    nx = it;
    if (++nx.b == a.B) {
        nx.b = 0;
        ++nx.step;
    }
    return nx.step < s1;
}
// The same for a role taking sequences first, first + stride, ... of every step.
__device__ __forceinline__ bool next_item_of(const RelayArgs& a, Item it, int s1, int first, int stride, Item& nx) {
    nx = it;
    nx.b += stride;
    if (nx.b >= a.B) {
        nx.b = first;
        ++nx.step;
    }
    return nx.step < s1;
}
__device__ __forceinline__ uint32_t epoch_of(const RelayArgs& a, int step) {
    return a.epoch_base + static_cast<uint32_t>(step) + 1u;
}

// LDS of a workgroup (floats): sv (kScratch: attention scratch of A, h / partials / kept x rows
// of F, logits of lm) | xs (C) | xn (C) | flags (4 ints: bail, token) | lm only: the token
// embedding table (V x C) and the next step's position row (C).
template <int NE>
struct Lds {
    float *sv, *xs, *xn;
    int* flags;
    float *tokt, *posrow;
    __device__ __forceinline__ explicit Lds(float* lds, int V) {
        constexpr int C = 64 * NE;
        sv = lds;
        xs = sv + kScratch;
        xn = xs + C;
        flags = reinterpret_cast<int*>(xn + C);
        tokt = xn + C + 4;
        posrow = tokt + (size_t)V * C;
    }
};

// Timeline (FMLH_RELAY_TRACE): stamp() records points 0-4 of sequence 0's item of a step.
// Meter accumulates, over all items of a step, the time spent waiting for inputs (item start
// to inputs settled) and the rest (inputs settled to item end), and records both with the end
// of the step's last item: points 5 (end), 6 (wait ticks), 7 (busy ticks).
__device__ __forceinline__ void stamp(const RelayArgs& a, int r, Item it, int point) {
    if (a.trace && thread_id() == 0 && it.b == 0 && it.step < kRelayTraceSteps)
        a.trace[((size_t)it.step * a.roles + r) * kRelayTracePoints + point] = wall_clock64();
}
struct Meter {
    unsigned long long t0 = 0, t1 = 0, wait = 0, busy = 0;
    __device__ __forceinline__ void start(const RelayArgs& a) {
        if (a.trace && thread_id() == 0) t0 = wall_clock64();
    }
    __device__ __forceinline__ void settled(const RelayArgs& a) {
        if (a.trace && thread_id() == 0) t1 = wall_clock64();
    }
    // (stride: the role takes every stride-th sequence, so its last item of a step is the one
    // within stride of the batch's end.)
    __device__ __forceinline__ void end(const RelayArgs& a, int r, Item it, int stride = 1) {
        if (!a.trace || thread_id() != 0) return;
        const unsigned long long t = wall_clock64();
        wait += t1 - t0;
        busy += t - t1;
        if (it.b + stride >= a.B) {
            if (it.step < kRelayTraceSteps) {
                unsigned long long* p = a.trace + ((size_t)it.step * a.roles + r) * kRelayTracePoints;
                p[5] = t;
                p[6] = wait;
                p[7] = busy;
            }
            wait = busy = 0;
        }
    }
};

// ---- Q: x_l, LN0, rows of W_qkv^T -> q / k_new / v_new words (k_new / v_new under QA) --------
// Items of steps [s0, s1).  prefetch: the next item's x words are requested as soon as this
// item's have arrived, so they are in flight during this item's products.
template <int NE, bool QA, bool BIG>
__device__ __forceinline__ void loop_q(const RelayArgs& a, const Role& ro, int r, const floatx4* wr, float* lds,
                                       int s0, int s1, bool prefetch) {
    constexpr int C = 64 * NE;
    constexpr int kRows = BIG ? kRelayBigTeamRows : kRelayTeamRows, P = BIG ? kBigPasses : kPasses;
    const Lds<NE> s(lds, a.V);
    const int l = ro.layer;
    auto src = [&](Item it) { return a.xw + ((size_t)l * a.B + it.b) * C; };
    Poll<1, C * 8> px;
    Item it{s0, 0};
    if (thread_id() < C) poll_issue(px, src(it), 8 * thread_id(), epoch_of(a, it.step));
    const LnPost lp = ln_post_setup<NE, P>(wr, s.xn, a.layers[l].ln0g, a.layers[l].ln0b, kRows);
    Meter mt;
    while (true) {
        stamp(a, r, it, 0);
        mt.start(a);
        Item nx;
        const bool more = next_item(a, it, s1, nx);
        if (thread_id() < C) {
            poll_settle(px, s.flags, a.err);
            const float xv = ll_float(px.v[0]);
            s.xs[thread_id()] = xv;
            s.xn[thread_id()] = xv * lp.gx;
            if (prefetch && more) poll_issue(px, src(nx), 8 * thread_id(), epoch_of(a, nx.step));
        }
        lds_barrier();
        stamp(a, r, it, 1);
        mt.settled(a);
        float mean, inv_std;
        ln_stats<NE>(s.xs, mean, inv_std);
        stamp(a, r, it, 2);
        const uint32_t ep = epoch_of(a, it.step);
        uint64_t* dst = a.qkvw + ((size_t)l * a.B + it.b) * 3 * C + (QA ? C : 0) + (size_t)ro.idx * kRows;
        gemv_regs<NE, P>(wr, s.xn, kRows,
                         [&](int row, float v) { ll_put(&dst[row], ln_apply(lp, v, mean, inv_std), ep); });
        stamp(a, r, it, 3);
        lds_barrier();  // every wave is done with this item's LDS before the next writes it
        mt.end(a, r, it);
        if (!more) return;
        if (!prefetch && thread_id() < C) poll_issue(px, src(nx), 8 * thread_id(), epoch_of(a, nx.step));
        it = nx;
    }
}

// ---- A: attention of head h, then its attention-projection partial -----------------------------

constexpr int kNCK = kHD / 16;
struct KvRegs {
    floatx4 k[kGroupsPerWave][kNCK], v[kGroupsPerWave][4];
};
// Requests item it's cached K/V rows 0..pos-1 of head h into registers: key kk = lane / 4 of each
// of the wave's 16-key groups (dims 16 (lane % 4) ..) and V rows kq + 4 i (dims 4 (lane % 16) ..)
// through bounded buffer loads (rows from pos on read as zero).
template <int NE>
__device__ __forceinline__ void kv_issue(const RelayArgs& a, int l, int h, Item it, KvRegs& kv) {
    constexpr int C = 64 * NE, H = C / kHD;
    const int pos = a.pos0 + it.step, lane = lane_id(), wave = wave_id();
    const size_t slab = (((size_t)l * a.Bmax + it.b) * H + h) * (size_t)a.T * kHD;
    const int bytes = pos * kHD * static_cast<int>(sizeof(float));
    const auto rk = __builtin_amdgcn_make_buffer_rsrc(a.kc + slab, 0, bytes, kRawBufferFlags);
    const auto rv = __builtin_amdgcn_make_buffer_rsrc(a.vc + slab, 0, bytes, kRawBufferFlags);
    const int kk = lane >> 2, part = lane & 3, d4 = lane & 15, kq = lane >> 4;
#pragma unroll
    for (int gi = 0; gi < kGroupsPerWave; ++gi) {
        const int base = kKeyGroup * (wave + kWaves * gi);
        if (base <= pos) {
#pragma unroll
            for (int c = 0; c < kNCK; ++c) kv.k[gi][c] = bload4(rk, (base + kk) * kHD + part * 16 + 4 * c);
#pragma unroll
            for (int i = 0; i < 4; ++i) kv.v[gi][i] = bload4(rv, (base + kq + 4 * i) * kHD + 4 * d4);
        } else {  // unused this item; written so that no earlier item's rows stay live in the set
#pragma unroll
            for (int c = 0; c < kNCK; ++c) kv.k[gi][c] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i) kv.v[gi][i] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
    }
}

// One item of an A role with its K/V rows in cur; the next item's rows are requested into nxt
// (within the step, prefetch; across steps only after this step's cache rows are written).
// The attention runs over the cached keys 0..pos-1; the step's own key (pos: k_new, v_new) is
// folded in last.  QA: the role forms its head's q itself (x_l, LN0 after the product, hd rows
// of W_q in wr after its W_proj share) while the Q team forms k_new / v_new, which it awaits
// only after the cached keys; the next item's K/V rows are then requested only at the item's
// end (QA is chosen for batch 1, where the next item is always the next step), so one K/V
// register set serves as both cur and nxt.  Otherwise it awaits q, k_new and v_new from the
// Q team first.  Returns whether there is a next item.
template <int NE, bool QA>
__device__ __forceinline__ bool a_item(const RelayArgs& a, const Role& ro, int r, const floatx4* wr, const Lds<NE>& s,
                                       const LnPost& lp, Item it, int s1, bool prefetch, Poll<1, 64 * NE * 8>& px,
                                       Poll<QA ? 2 : 3, 64 * NE * 8>& pq, const KvRegs& cur, KvRegs& nxt,
                                       Meter& mt) {
    constexpr int C = 64 * NE, H = C / kHD;
    const int l = ro.layer, h = ro.idx;
    const int pos = a.pos0 + it.step;
    const uint32_t ep = epoch_of(a, it.step);
    const int lane = lane_id(), wave = wave_id(), o = thread_id();
    const int kk = lane >> 2, part = lane & 3;  // score lanes: key kk, dims part * 16 ..
    const int d4 = lane & 15, kq = lane >> 4;   // P.V lanes: dims 4 d4 .., keys kq + 4 i
    auto xsrc = [&](Item i) { return a.xw + ((size_t)l * a.B + i.b) * C; };
    // The Q team's words of head h: q (not under QA), k_new, v_new.
    auto qsrc = [&](Item i) { return a.qkvw + ((size_t)l * a.B + i.b) * 3 * C + (QA ? C : 0) + kHD * h; };
    stamp(a, r, it, 0);
    mt.start(a);
    Item nx;
    // QA (batch 1): one attention workgroup per head, every sequence.
    const int first = QA ? 0 : ro.sub, stride = QA ? 1 : a.nA;
    const bool more = next_item_of(a, it, s1, first, stride, nx);
    const bool same_step = !QA && more && nx.step == it.step;
    // Attention scratch in sv.  Each wave's 256 floats hold in turn its softmax weights (64),
    // its P.V partials (256, written after the weights are read) and its combine row (64 + 2,
    // written after the partials are read); all three are the wave's own, read in order.
    float* qs = s.sv;                 // q, k_new, v_new (3 x 64)
    float* wsc = qs + 3 * kHD;        // kWaves x 256
    float kn = 0.f, vn = 0.f;         // wave 0: the step's K/V cache row entries
    if constexpr (QA) {
        if (o < C) {
            poll_settle(px, s.flags, a.err);
            const float xv = ll_float(px.v[0]);
            s.xs[o] = xv;
            s.xn[o] = xv * lp.gx;
            if (prefetch && more) poll_issue(px, xsrc(nx), 8 * o, epoch_of(a, nx.step));
        }
    } else {
        if (wave == 0) {
            poll_settle(pq, s.flags, a.err);
            kn = ll_float(pq.v[1]);
            vn = ll_float(pq.v[2]);
            qs[lane] = ll_float(pq.v[0]);
            qs[kHD + lane] = kn;
            qs[2 * kHD + lane] = vn;
            if (prefetch && more) poll_issue(pq, qsrc(nx), 8 * lane, epoch_of(a, nx.step));
        }
        if (prefetch && same_step) kv_issue<NE>(a, l, h, nx, nxt);
    }
    lds_barrier();
    stamp(a, r, it, 1);
    mt.settled(a);
    if constexpr (QA) {
        float mean, inv_std;
        ln_stats<NE>(s.xs, mean, inv_std);
        gemv_regs<NE, kQaPasses>(wr + 2 * NE, s.xn, kHD,
                                 [&](int row, float v) { qs[row] = ln_apply(lp, v, mean, inv_std); });
        lds_barrier();
    }
    floatx4 qv[kNCK];
#pragma unroll
    for (int c = 0; c < kNCK; ++c) qv[c] = lds4(qs + part * 16 + 4 * c);
    // Cached keys 0..pos-1 (key pos is folded in below).
    float sc[kGroupsPerWave];
    float mx = -INFINITY;
#pragma unroll
    for (int gi = 0; gi < kGroupsPerWave; ++gi) {
        const int base = kKeyGroup * (wave + kWaves * gi);
        sc[gi] = -INFINITY;
        if (base < pos) {
            float sv2 = 0.f;
#pragma unroll
            for (int c = 0; c < kNCK; ++c) sv2 += dot4(qv[c], cur.k[gi][c]);
            sc[gi] = quad_sum(sv2) * a.scale;
            if (base + kk < pos) mx = fmaxf(mx, sc[gi]);
        }
    }
    const float m = wave_max(mx);  // -inf if this wave has no cached key
    float* pl = wsc + wave * 256;   // [group][4 (k % 4) + k / 4]
    float psum = 0.f;
#pragma unroll
    for (int gi = 0; gi < kGroupsPerWave; ++gi) {
        const int j = kKeyGroup * (wave + kWaves * gi) + kk;
        const float pv = j < pos ? __expf(sc[gi] - m) : 0.f;
        if (part == 0) {
            psum += pv;
            pl[16 * gi + 4 * (kk & 3) + (kk >> 2)] = pv;
        }
    }
    const float lsum = wave_sum(psum);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's softmax weights are in LDS
    float4 ov = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int gi = 0; gi < kGroupsPerWave; ++gi) {
        if (kKeyGroup * (wave + kWaves * gi) < pos) {
            const floatx4 pp = lds4(pl + 16 * gi + 4 * kq);
#pragma unroll
            for (int i = 0; i < 4; ++i) {  // key kq + 4 i of the group (rows from pos on read as zero)
                ov.x += pp[i] * cur.v[gi][i][0];
                ov.y += pp[i] * cur.v[gi][i][1];
                ov.z += pp[i] * cur.v[gi][i][2];
                ov.w += pp[i] * cur.v[gi][i][3];
            }
        }
    }
    float* ow = wsc + wave * 256;
    *reinterpret_cast<float4*>(ow + kq * 64 + 4 * d4) = ov;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const float osum = (ow[lane] + ow[64 + lane]) + (ow[128 + lane] + ow[192 + lane]);
    ow[2 + lane] = osum;
    if (lane == 0) {
        ow[0] = m;
        ow[1] = lsum;
    }
    // QA: k_new / v_new of key pos (the Q team's words), by wave 0.
    if constexpr (QA) {
        if (wave == 0) {
            poll_settle(pq, s.flags, a.err);
            kn = ll_float(pq.v[0]);
            vn = ll_float(pq.v[1]);
            qs[kHD + lane] = kn;
            qs[2 * kHD + lane] = vn;
            if (prefetch && more) poll_issue(pq, qsrc(nx), 8 * lane, epoch_of(a, nx.step));
        }
    }
    lds_barrier();
    // Every wave combines the waves' rows over the cached keys, then folds key pos in, into y_h
    // itself (same order, so the same y in each), in a row of its own in xs / xn (read no more
    // this item): no second barrier.  The rows are rewritten only after the item's last
    // barrier, when every wave has read them.
    static_assert(2 * C >= kWaves * kHD, "a y row per wave in xs and xn");
    float* ys = s.xs + wave * kHD;
    {
        float s_pos = 0.f;
#pragma unroll
        for (int c = 0; c < kNCK; ++c) s_pos += dot4(qv[c], lds4(qs + kHD + part * 16 + 4 * c));
        s_pos = quad_sum(s_pos) * a.scale;
        float M = wsc[0];
#pragma unroll
        for (int v = 1; v < kWaves; ++v) M = fmaxf(M, wsc[v * 256]);
        float od = 0.f, lt = 0.f;
#pragma unroll
        for (int v = 0; v < kWaves; ++v) {
            const float* cv = wsc + v * 256;
            const float wv = cv[0] == -INFINITY ? 0.f : __expf(cv[0] - M);
            od += wv * cv[2 + lane];
            lt += wv * cv[1];
        }
        const float Mn = fmaxf(M, s_pos);
        const float cold = M == -INFINITY ? 0.f : __expf(M - Mn), cnew = __expf(s_pos - Mn);
        od = od * cold + cnew * qs[2 * kHD + lane];
        lt = lt * cold + cnew;
        ys[lane] = od * __builtin_amdgcn_rcpf(lt);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's y row is in LDS
    stamp(a, r, it, 2);
    // dx1 partial of head h: output o = 128 p + 16 wave + lane / 4, dims 16 part ..
    const floatx4* y4 = reinterpret_cast<const floatx4*>(ys) + 4 * part;
    floatx4 yv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) yv[c] = y4[c];
    constexpr int PP = C / (16 * kWaves);
    static_assert(PP <= 4, "one pass per lane of a quad");
    float mine = 0.f;  // lane part == p keeps pass p's sum
#pragma unroll
    for (int p = 0; p < PP; ++p) {
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) acc = fma4(wr[4 * p + c], yv[c], acc);
        acc = quad_sum(acc);
        mine = part == p ? acc : mine;
    }
    uint64_t* dst = a.dx1w + (((size_t)l * a.B + it.b) * H + h) * C;
    if (part < PP) ll_put(&dst[part * 16 * kWaves + 16 * wave + (lane >> 2)], mine, ep);
    stamp(a, r, it, 3);
    if (wave == 0) {  // the step's cache row of this sequence
        const size_t slab = (((size_t)l * a.Bmax + it.b) * H + h) * (size_t)a.T * kHD;
        a.kc[slab + (size_t)pos * kHD + lane] = kn;
        a.vc[slab + (size_t)pos * kHD + lane] = vn;
        // The next step's K/V loads of this role (this WG) read the rows written in this step:
        // they are issued only after this wait and the barrier below.
        if (!same_step) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    lds_barrier();  // every wave is done with this item's LDS (and the cache rows are written)
    mt.end(a, r, it, stride);
    if (more) {
        if (!same_step || !prefetch) kv_issue<NE>(a, l, h, nx, nxt);
        if (!prefetch) {
            if (QA && o < C) poll_issue(px, xsrc(nx), 8 * o, epoch_of(a, nx.step));
            if (wave == 0) poll_issue(pq, qsrc(nx), 8 * lane, epoch_of(a, nx.step));
        }
    }
    return more;
}

template <int NE, bool QA>
__device__ __forceinline__ void loop_a(const RelayArgs& a, const Role& ro, int r, const floatx4* wr, float* lds,
                                       int s0, int s1, bool prefetch) {
    constexpr int C = 64 * NE;
    const Lds<NE> s(lds, a.V);
    const int l = ro.layer, h = ro.idx, o = thread_id();
    LnPost lp{0.f, 0.f, 0.f};
    if constexpr (QA) lp = ln_post_setup<NE, kQaPasses>(wr + 2 * NE, s.xn, a.layers[l].ln0g, a.layers[l].ln0b, kHD);
    Poll<1, C * 8> px;
    Poll<QA ? 2 : 3, C * 8> pq;
    KvRegs kv0, kv1;
    // Sequences ro.sub, ro.sub + a.nA, ... (a.nA attention workgroups per head; QA: one).
    const int first = QA ? 0 : ro.sub, stride = QA ? 1 : a.nA;
    if (first >= a.B) return;
    Item it{s0, first};
    kv_issue<NE>(a, ro.layer, ro.idx, it, kv0);
    if (QA && o < C) poll_issue(px, a.xw + ((size_t)l * a.B + it.b) * C, 8 * o, epoch_of(a, it.step));
    if (wave_id() == 0)
        poll_issue(pq, a.qkvw + ((size_t)l * a.B + it.b) * 3 * C + (QA ? C : 0) + kHD * h, 8 * lane_id(),
                   epoch_of(a, it.step));
    Meter mt;
    if constexpr (QA) {  // the next item's rows are requested after this item's last read: one set
        while (a_item<NE, QA>(a, ro, r, wr, s, lp, it, s1, prefetch, px, pq, kv0, kv0, mt)) {
            Item nx;
            next_item_of(a, it, s1, first, stride, nx);
            it = nx;
        }
        return;
    }
    // Two items per pass, so each register set is named at compile time.
    while (true) {
        Item nx;
        if (!a_item<NE, QA>(a, ro, r, wr, s, lp, it, s1, prefetch, px, pq, kv0, kv1, mt)) return;
        next_item_of(a, it, s1, first, stride, nx);
        it = nx;
        if (!a_item<NE, QA>(a, ro, r, wr, s, lp, it, s1, prefetch, px, pq, kv1, kv0, mt)) return;
        next_item_of(a, it, s1, first, stride, nx);
        it = nx;
    }
}

// ---- F: x_l + the heads' dx1 partials, LN1, rows of W_fc^T, GELU -> h; proj2 partial of
//      every output over the WG's 96 columns; then x_{l+1} for the WG's rows ---------------------

// The second phase of an F item: its R = C / nf rows of x_{l+1} = x' (kept rows, xk) + the nf
// partials of each row in team order (thread f R + i < nf R holds partial f of row i, polled
// into pp by poll_issue earlier).
template <int NE>
__device__ __forceinline__ void f_rows(const RelayArgs& a, const Role& ro, const Lds<NE>& s, Item it,
                                       Poll<1, 4 * 64 * NE / kRelayFRows * 64 * NE * 8>& pp, const float* xk) {
    constexpr int C = 64 * NE, NF = 4 * C / kRelayFRows, R = C / NF;
    const int tid = thread_id();
    float* ps = s.sv + kRelayFRows;  // [NF][R], after h
    if (tid < NF * R) {
        poll_settle(pp, s.flags, a.err);
        ps[tid] = ll_float(pp.v[0]);
    }
    lds_barrier();
    if (tid < R) {
        float dsum = ps[tid];
#pragma unroll
        for (int f = 1; f < NF; ++f) dsum += ps[f * R + tid];
        ll_put(&a.xw[((size_t)(ro.layer + 1) * a.B + it.b) * C + ro.idx * R + tid], xk[tid] + dsum,
               epoch_of(a, it.step));
    }
    lds_barrier();
}

// Items whose x_{l+1} rows still wait for their partials (at most the two before the current
// one, all of the current step).
struct FPending {
    int b1 = -1, b2 = -1;  // sequences of items gi - 1 and gi - 2 (-1: none pending)
};

// One F item (global item number gi of this role; pp_cur / pp_other: the partial polls of the
// items of gi's and the other parity).  With lag_rows the rows of an item are added up two items
// later, so the other F workgroups' partials have two items' time to arrive (more throughput
// for large batches, more latency per layer), except at the end of a step (the next step's items
// need them) or without prefetch; otherwise at once.  BIG: the row sums are the F2 team's; the
// item publishes its rows of x' for them instead.
template <int NE, bool BIG, int FR>
__device__ __forceinline__ bool f_item(const RelayArgs& a, const Role& ro, int r, const floatx4* wr, const Lds<NE>& s,
                                       const LnPost& lp, Item it, int gi, int s1, bool prefetch,
                                       Poll<1, 64 * NE * 8>& px, Poll<64 * NE / kHD, 64 * NE * 8>& pd,
                                       Poll<1, 4 * 64 * NE / FR * 64 * NE * 8>& pp_cur,
                                       Poll<1, 4 * 64 * NE / FR * 64 * NE * 8>& pp_other, FPending& pend,
                                       Meter& mt) {
    constexpr int C = 64 * NE, H = C / kHD, NF = 4 * C / FR, R = C / NF;
    constexpr int FP = FR / kRowsPerPass, FC4 = FR / 32;  // FC passes; float4 of proj2 columns per pass
    static_assert(FR == kRelayFRows || BIG, "the FC team's own row sums (f_rows) take kRelayFRows rows");
    static_assert(FR % 32 == 0 && FR + NF * R + 3 * R <= kScratch, "F scratch");
    const int l = ro.layer, r0 = ro.idx * R;
    float* hs = s.sv;                   // the WG's FR entries of h
    float* xkeep = s.sv + FR + NF * R;  // [3][R]: x' rows of the items gi % 3
    auto xsrc = [&](Item i) { return a.xw + ((size_t)l * a.B + i.b) * C; };
    auto dsrc = [&](Item i) { return a.dx1w + ((size_t)l * a.B + i.b) * H * C; };
    auto psrc = [&](Item i) { return a.partw + ((size_t)l * a.B + i.b) * NF * C + r0; };
    const int o = thread_id();
    stamp(a, r, it, 0);
    mt.start(a);
    Item nx;
    const bool more = next_item(a, it, s1, nx);
    const uint32_t ep = epoch_of(a, it.step);
    if (o < C) {
        poll_settle(px, s.flags, a.err);
        poll_settle(pd, s.flags, a.err);
        float d = ll_float(pd.v[0]);
#pragma unroll
        for (int hh = 1; hh < H; ++hh) d += ll_float(pd.v[hh]);
        const float xp = ll_float(px.v[0]) + d;
        s.xs[o] = xp;
        s.xn[o] = xp * lp.gx;
        if (o >= r0 && o < r0 + R) {
            if constexpr (BIG) ll_put(&a.xpw[((size_t)l * a.B + it.b) * C + o], xp, ep);
            else xkeep[(gi % 3) * R + (o - r0)] = xp;
        }
        if (more) {
            poll_issue(px, xsrc(nx), 8 * o, epoch_of(a, nx.step));
            poll_issue(pd, dsrc(nx), 8 * o, epoch_of(a, nx.step));
        }
    }
    lds_barrier();
    stamp(a, r, it, 1);
    mt.settled(a);
    if constexpr (FR == kRelayHRows) {  // the h cut: the WG's FR entries of h go out as words
        float mean, inv_std;
        ln_stats<NE>(s.xs, mean, inv_std);
        uint64_t* hw = a.partw + ((size_t)l * a.B + it.b) * NF * C + (size_t)ro.idx * FR;
        gemv_regs<NE, FP>(wr, s.xn, FR,
                          [&](int row, float v) { ll_put(&hw[row], gelu_ref(ln_apply(lp, v, mean, inv_std)), ep); });
        stamp(a, r, it, 2);
    } else {
        {
            float mean, inv_std;
            ln_stats<NE>(s.xs, mean, inv_std);
            gemv_regs<NE, FP>(wr, s.xn, FR,
                              [&](int row, float v) { hs[row] = gelu_ref(ln_apply(lp, v, mean, inv_std)); });
        }
        lds_barrier();
        stamp(a, r, it, 2);
        // Output o = 64 p + 8 wave + lane / 8: 8 lanes per row, 4 FC4 columns each.
        const int lane = lane_id(), wave = wave_id(), t8 = lane & 7;
        constexpr int PP = C / (8 * kWaves);
        static_assert(PP == NE && PP <= 8, "one pass per lane of an octet");
        floatx4 hq[FC4];
#pragma unroll
        for (int c = 0; c < FC4; ++c) hq[c] = lds4(hs + 4 * FC4 * t8 + 4 * c);
        float mine = 0.f;  // lane t8 == p keeps pass p's sum
#pragma unroll
        for (int p = 0; p < PP; ++p) {
            float acc = 0.f;
#pragma unroll
            for (int c = 0; c < FC4; ++c) acc = fma4(wr[FP * NE + FC4 * p + c], hq[c], acc);
            acc = oct_sum(acc);
            mine = t8 == p ? acc : mine;
        }
        uint64_t* part = a.partw + ((size_t)l * a.B + it.b) * NF * C;  // [NF][C] of this sequence
        if (t8 < PP) ll_put(&part[(size_t)ro.idx * C + 64 * t8 + 8 * wave + (lane >> 3)], mine, ep);
    }
    stamp(a, r, it, 3);
    if constexpr (!BIG) {
        if (pend.b2 >= 0) f_rows<NE>(a, ro, s, Item{it.step, pend.b2}, pp_cur, xkeep + ((gi + 1) % 3) * R);  // gi - 2
        if (o < NF * R) poll_issue(pp_cur, psrc(it), 8 * ((o / R) * C + o % R), ep);
        if (!prefetch || !a.lag_rows || !more || nx.step != it.step) {
            if (pend.b1 >= 0) f_rows<NE>(a, ro, s, Item{it.step, pend.b1}, pp_other, xkeep + ((gi + 2) % 3) * R);
            f_rows<NE>(a, ro, s, it, pp_cur, xkeep + (gi % 3) * R);
            pend.b1 = pend.b2 = -1;
        } else {
            pend.b2 = pend.b1;
            pend.b1 = it.b;
        }
    }
    stamp(a, r, it, 4);
    lds_barrier();
    mt.end(a, r, it);
    return more;
}

template <int NE, bool BIG, int FR>
__device__ __forceinline__ void loop_f(const RelayArgs& a, const Role& ro, int r, const floatx4* wr, float* lds,
                                       int s0, int s1, bool prefetch) {
    constexpr int C = 64 * NE, H = C / kHD, NF = 4 * C / FR;
    const Lds<NE> s(lds, a.V);
    const int l = ro.layer;
    const LnPost lp = ln_post_setup<NE, FR / kRowsPerPass>(wr, s.xn, a.layers[l].ln1g, a.layers[l].ln1b, FR);
    Poll<1, C * 8> px;
    Poll<H, C * 8> pd;
    Poll<1, NF * C * 8> pp0, pp1;
    const int o = thread_id();
    Item it{s0, 0};
    if (o < C) {
        poll_issue(px, a.xw + ((size_t)l * a.B + it.b) * C, 8 * o, epoch_of(a, it.step));
        poll_issue(pd, a.dx1w + ((size_t)l * a.B + it.b) * H * C, 8 * o, epoch_of(a, it.step));
    }
    FPending pend;
    Meter mt;
    // Two items per pass, so each partial poll is named at compile time.
    for (int gi = 0;; gi += 2) {
        Item nx;
        if (!f_item<NE, BIG, FR>(a, ro, r, wr, s, lp, it, gi, s1, prefetch, px, pd, pp0, pp1, pend, mt)) return;
        next_item(a, it, s1, nx);
        it = nx;
        if (!f_item<NE, BIG, FR>(a, ro, r, wr, s, lp, it, gi + 1, s1, prefetch, px, pd, pp1, pp0, pend, mt)) return;
        next_item(a, it, s1, nx);
        it = nx;
    }
}

// ---- F2 (big): the rows of x_{l+1} = x' + the FC team's partials in team order ---------------
// Workgroup k takes rows r0 = kRelayF2Rows k ..: thread t polls partials (t / kRelayF2Rows +
// 8 j, t % kRelayF2Rows) for j < J = nf kRelayF2Rows / kThreads and, for t < kRelayF2Rows,
// x'[r0 + t] (published by the FC workgroup holding that row); the sum is f_rows' (the same
// order, the same result).
template <int NE, int FR>
__device__ __forceinline__ void loop_f2(const RelayArgs& a, const Role& ro, int r, float* lds, int s0, int s1,
                                        bool prefetch) {
    constexpr int C = 64 * NE, NF = 4 * C / FR, R2 = kRelayF2Rows, J = NF * R2 / kThreads;
    static_assert(NF * R2 % kThreads == 0 && kThreads % R2 == 0, "whole partial words per thread");
    static_assert(NF * R2 + R2 <= kScratch, "F2 scratch");
    constexpr int kPStride = (kThreads / R2) * C * 8;  // bytes between a thread's partial words
    const Lds<NE> s(lds, a.V);
    const int l = ro.layer, r0 = ro.idx * R2, t = thread_id();
    float* ps = s.sv;            // [NF][R2]
    float* xk = s.sv + NF * R2;  // [R2]
    auto psrc = [&](Item i) { return a.partw + ((size_t)l * a.B + i.b) * NF * C + r0; };
    auto xsrc = [&](Item i) { return a.xpw + ((size_t)l * a.B + i.b) * C + r0; };
    const int poff = 8 * ((t / R2) * C + t % R2);
    Poll<J, kPStride> pp;
    Poll<1, C * 8> px;
    Item it{s0, 0};
    poll_issue(pp, psrc(it), poff, epoch_of(a, it.step));
    if (t < R2) poll_issue(px, xsrc(it), 8 * t, epoch_of(a, it.step));
    Meter mt;
    while (true) {
        stamp(a, r, it, 0);
        mt.start(a);
        Item nx;
        const bool more = next_item(a, it, s1, nx);
        poll_settle(pp, s.flags, a.err);
#pragma unroll
        for (int j = 0; j < J; ++j) ps[t + kThreads * j] = ll_float(pp.v[j]);
        if (t < R2) {
            poll_settle(px, s.flags, a.err);
            xk[t] = ll_float(px.v[0]);
        }
        if (prefetch && more) {
            poll_issue(pp, psrc(nx), poff, epoch_of(a, nx.step));
            if (t < R2) poll_issue(px, xsrc(nx), 8 * t, epoch_of(a, nx.step));
        }
        lds_barrier();
        stamp(a, r, it, 1);
        mt.settled(a);
        if (t < R2) {
            float dsum = ps[t];
#pragma unroll
            for (int f = 1; f < NF; ++f) dsum += ps[f * R2 + t];
            ll_put(&a.xw[((size_t)(l + 1) * a.B + it.b) * C + r0 + t], xk[t] + dsum, epoch_of(a, it.step));
        }
        stamp(a, r, it, 3);
        lds_barrier();  // every wave is done with this item's LDS before the next writes it
        mt.end(a, r, it);
        if (!more) return;
        if (!prefetch) {
            poll_issue(pp, psrc(nx), poff, epoch_of(a, nx.step));
            if (t < R2) poll_issue(px, xsrc(nx), 8 * t, epoch_of(a, nx.step));
        }
        it = nx;
    }
}

// ---- F2 (h cut): rows of x_{l+1} = x' + W_proj2 rows . h ---------------------------------------
// Workgroup k takes rows r0 = kRelayHF2Rows k ..: thread t polls h words t + kThreads j (the FC
// team's, all 4C of them) and, for t < kRelayHF2Rows, x'[r0 + t]; row r0 + 4 wave + g is the
// dot product of its W_proj2 row (registers) with h (LDS) over the 16 lanes of group g.
template <int NE>
__device__ __forceinline__ void loop_f2h(const RelayArgs& a, const Role& ro, int r, const floatx4* wr, float* lds,
                                         int s0, int s1, bool prefetch) {
    constexpr int C = 64 * NE, K = 4 * C, R2 = kRelayHF2Rows, J = K / kThreads;
    static_assert(K % kThreads == 0 && K + R2 <= kScratch && R2 == 4 * kWaves, "F2 (h cut) layout");
    const Lds<NE> s(lds, a.V);
    const int l = ro.layer, r0 = ro.idx * R2, t = thread_id();
    const int lane = lane_id(), wave = wave_id(), tl = lane & 15, g = lane >> 4;
    float* hs = s.sv;      // [4C]
    float* xk = s.sv + K;  // [R2]
    auto hsrc = [&](Item i) { return a.partw + ((size_t)l * a.B + i.b) * a.nf * C; };
    auto xsrc = [&](Item i) { return a.xpw + ((size_t)l * a.B + i.b) * C + r0; };
    Poll<J, kThreads * 8> ph;
    Poll<1, C * 8> px;
    Item it{s0, 0};
    poll_issue(ph, hsrc(it), 8 * t, epoch_of(a, it.step));
    if (t < R2) poll_issue(px, xsrc(it), 8 * t, epoch_of(a, it.step));
    Meter mt;
    while (true) {
        stamp(a, r, it, 0);
        mt.start(a);
        Item nx;
        const bool more = next_item(a, it, s1, nx);
        poll_settle(ph, s.flags, a.err);
#pragma unroll
        for (int j = 0; j < J; ++j) hs[t + kThreads * j] = ll_float(ph.v[j]);
        if (t < R2) {
            poll_settle(px, s.flags, a.err);
            xk[t] = ll_float(px.v[0]);
        }
        if (prefetch && more) {
            poll_issue(ph, hsrc(nx), 8 * t, epoch_of(a, nx.step));
            if (t < R2) poll_issue(px, xsrc(nx), 8 * t, epoch_of(a, nx.step));
        }
        lds_barrier();
        stamp(a, r, it, 1);
        mt.settled(a);
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4 * NE; ++j) acc = fma4(wr[j], lds4(hs + 4 * (tl + 16 * j)), acc);
        acc = row16_sum(acc);
        const int row = 4 * wave + g;
        if (tl == 0)
            ll_put(&a.xw[((size_t)(l + 1) * a.B + it.b) * C + r0 + row], xk[row] + acc, epoch_of(a, it.step));
        stamp(a, r, it, 3);
        lds_barrier();  // every wave is done with this item's LDS before the next writes it
        mt.end(a, r, it);
        if (!more) return;
        if (!prefetch) {
            poll_issue(ph, hsrc(nx), 8 * t, epoch_of(a, nx.step));
            if (t < R2) poll_issue(px, xsrc(nx), 8 * t, epoch_of(a, nx.step));
        }
        it = nx;
    }
}

// ---- lm: x_L, ln_f, logits, first maximum -> the token, and the next step's x_0 ---------------

// x_0 of sequence b for step `step`: the embedding of `token` plus position row `prow`
// (Embedding x2 + AddLayer; dropout p = 0), as exchange words.  Threads o < C.
template <int NE>
__device__ __forceinline__ void emit_x0(const RelayArgs& a, int b, int step, const float* tokrow, const float* prow) {
    constexpr int C = 64 * NE;
    const int o = thread_id();
    if (o < C) ll_put(&a.xw[(size_t)b * C + o], tokrow[o] + prow[o], epoch_of(a, step));
}

template <int NE>
__device__ __forceinline__ void loop_lm(const RelayArgs& a, const Role& ro, int r, const floatx4* wr, float* lds,
                                        int s0, int s1, bool prefetch, bool table) {
    constexpr int C = 64 * NE;
    const Lds<NE> s(lds, a.V);
    const int o = thread_id();
    // lm_head role ro.sub of a.nlm takes sequences ro.sub, ro.sub + a.nlm, ...
    const int first = ro.sub, stride = a.nlm;
    if (first >= a.B) return;
    // The token embeddings in LDS (table: a single-role WG, for the whole launch).
    if (table)
        for (int e = o; e < a.V * C; e += kThreads) s.tokt[e] = ld1(a.tok + e);
    auto src = [&](Item i) { return a.xw + ((size_t)a.L * a.B + i.b) * C; };
    Poll<1, C * 8> px;
    Item it{s0, first};
    if (o < C) poll_issue(px, src(it), 8 * o, epoch_of(a, it.step));
    const LnPost lp = ln_post_setup<NE, kPasses>(wr, s.xn, a.lnf_g, a.lnf_b, a.V);
    float* lg = s.sv;
    Meter mt;
    while (true) {
        stamp(a, r, it, 0);
        mt.start(a);
        Item nx;
        const bool more = next_item_of(a, it, s1, first, stride, nx);
        const int pos = a.pos0 + it.step;
        const bool emit = it.step + 1 < a.n_steps;  // the next step's x_0
        if (it.b == first && emit && o < C) s.posrow[o] = ld1(a.pos_emb + (size_t)(pos + 1) * C + o);
        if (o < C) {
            poll_settle(px, s.flags, a.err);
            const float xv = ll_float(px.v[0]);
            s.xs[o] = xv;
            s.xn[o] = xv * lp.gx;
            if (prefetch && more) poll_issue(px, src(nx), 8 * o, epoch_of(a, nx.step));
        }
        lds_barrier();
        stamp(a, r, it, 1);
        mt.settled(a);
        float mean, inv_std;
        ln_stats<NE>(s.xs, mean, inv_std);
        const bool keep = a.logit_hist && (size_t)(a.gen0 + it.step) < a.hist_slots;
        float* lrow = a.logits + (size_t)it.b * a.V;
        float* hrow = keep ? a.logit_hist + ((size_t)(a.gen0 + it.step) * a.B + it.b) * a.V : nullptr;
        gemv_regs<NE>(wr, s.xn, a.V, [&](int row, float v) {
            v = ln_apply(lp, v, mean, inv_std);
            lg[row] = v;
            lrow[row] = v;
            if (keep) hrow[row] = v;
        });
        lds_barrier();
        stamp(a, r, it, 2);
        if (wave_id() == 0) {
            const int lane = lane_id();
            float bv = -INFINITY;
            int bi = -1;
            for (int v = lane; v < a.V; v += 64) {
                if (bi < 0 || lg[v] > bv) {  // strict: the lower index keeps a tie
                    bv = lg[v];
                    bi = v;
                }
            }
            float best;
            const int t = wave_argmax(bv, bi, best);
            if (lane == 0) {
                const int tk = t < 0 ? 0 : t;
                a.hist[(size_t)it.b * a.HS + pos + 1] = tk;
                s.flags[1] = tk;
            }
        }
        lds_barrier();
        if (emit) {
            const int tk = s.flags[1];
            emit_x0<NE>(a, it.b, it.step + 1, table ? s.tokt + (size_t)tk * C : a.tok + (size_t)tk * C,
                        s.posrow);
        }
        stamp(a, r, it, 3);
        lds_barrier();
        mt.end(a, r, it, stride);
        if (!more) return;
        if (!prefetch && o < C) poll_issue(px, src(nx), 8 * o, epoch_of(a, nx.step));
        it = nx;
    }
}

// ---- role dispatch -----------------------------------------------------------------------------

// Items of steps [s0, s1) of role ro (kind K) with its weights in wr.
template <int NE, bool QA, bool BIG, int FR, int K>
__device__ __forceinline__ void run_items(const RelayArgs& a, const Role& ro, int r, const floatx4* wr, float* lds,
                                          int s0, int s1, bool single) {
    if constexpr (K == kQ) loop_q<NE, QA, BIG>(a, ro, r, wr, lds, s0, s1, single);
    else if constexpr (K == kA) loop_a<NE, QA>(a, ro, r, wr, lds, s0, s1, single);
    else if constexpr (K == kF) loop_f<NE, BIG, FR>(a, ro, r, wr, lds, s0, s1, single);
    else if constexpr (K == kF2 && FR == kRelayHRows) loop_f2h<NE>(a, ro, r, wr, lds, s0, s1, single);
    else if constexpr (K == kF2) loop_f2<NE, FR>(a, ro, r, lds, s0, s1, single);
    else loop_lm<NE>(a, ro, r, wr, lds, s0, s1, single, single);
}

// A workgroup with one role: its weights are loaded once, and it runs every item of the launch
// with the next item's inputs requested early (prefetch).
template <int NE, bool QA, bool BIG, int FR, int K>
__device__ __forceinline__ void run_single(const RelayArgs& a, const Role& ro, int r, float* lds) {
    floatx4 wr[wr_count<NE, K, QA, BIG, FR>()];
    load_weights<NE, K, QA, BIG, FR>(a, ro, wr);
    run_items<NE, QA, BIG, FR, K>(a, ro, r, wr, lds, 0, a.n_steps, true);
}

// One role of a workgroup with two, for one step: the role's weights are requested when it
// starts (its inputs come much later: the role before it in the step order is several layers
// back); its items run without prefetch.
template <int NE, bool QA, bool BIG, int FR, int K>
__device__ __forceinline__ void run_loaded(const RelayArgs& a, const Role& ro, int r, int step, float* lds) {
    floatx4 wr[wr_count<NE, K, QA, BIG, FR>()];
    load_weights<NE, K, QA, BIG, FR>(a, ro, wr);
    run_items<NE, QA, BIG, FR, K>(a, ro, r, wr, lds, step, step + 1, false);
}

// SPLIT (with BIG): two attention and two lm_head workgroups per head / model, each taking every
// other sequence, and at n_embed 384 FC slices of kRelaySplitFRows rows (to stay within 256
// workgroups for six layers); SPLIT 2 (n_embed 384), the h cut: FC slices of kRelayHRows rows
// that publish h, and the MLP projection's rows in the F2 team.
template <int NE, bool QA, bool BIG, int SPLIT>
__global__ __launch_bounds__(kThreads) void decode_relay_kernel(RelayArgs a) {
    constexpr int C = 64 * NE, H = C / kHD;
    constexpr int FR = SPLIT == 2 ? kRelayHRows : SPLIT && NE == 6 ? kRelaySplitFRows : kRelayFRows;
    static_assert(SPLIT != 2 || NE == 6, "the h cut is compiled for n_embed 384");
    static_assert(C % kHD == 0 && NE % 2 == 0, "heads");
    static_assert(!(QA && BIG) && (!SPLIT || BIG) && 4 * C % FR == 0, "one team cut");
    static_assert((QA ? 2 : 3) * C % (BIG ? kRelayBigTeamRows : kRelayTeamRows) == 0 && 4 * C % kRelayFRows == 0 &&
                      kHD % kRowsPerPass == 0 && (!BIG || C % kRelayF2Rows == 0),
                  "teams");
    extern __shared__ float lds[];
    const Lds<NE> s(lds, a.V);

    const int w = static_cast<int>(blockIdx.x), G = static_cast<int>(gridDim.x);
    if (thread_id() == 0) __hip_atomic_store(s.flags, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    // x_0 of the launch's first step, from the token history, by the lm_head role's workgroup
    // (before any of its roles waits for anything).
    if (w == (a.roles - 1) % G) {
        for (int b = 0; b < a.B; ++b) {
            const int t = a.hist[(size_t)b * a.HS + a.pos0];
            const int tk = t < 0 || t >= a.V ? 0 : t;  // a corrupt history must not index out of the table
            emit_x0<NE>(a, b, 0, a.tok + (size_t)tk * C, a.pos_emb + (size_t)a.pos0 * C);
        }
    }
    lds_barrier();
    const Role ro = role_of(a, H, w);
    if (w + G >= a.roles) {
        switch (ro.kind) {
            case kQ: run_single<NE, QA, BIG, FR, kQ>(a, ro, w, lds); break;
            case kA: run_single<NE, QA, BIG, FR, kA>(a, ro, w, lds); break;
            case kF: run_single<NE, QA, BIG, FR, kF>(a, ro, w, lds); break;
            case kF2:
                if constexpr (BIG) run_single<NE, QA, BIG, FR, kF2>(a, ro, w, lds);
                break;
            default: run_single<NE, QA, BIG, FR, kLm>(a, ro, w, lds); break;
        }
    } else {
        for (int step = 0; step < a.n_steps; ++step) {
            for (int r = w; r < a.roles; r += G) {
                const Role rr = role_of(a, H, r);
                switch (rr.kind) {
                    case kQ: run_loaded<NE, QA, BIG, FR, kQ>(a, rr, r, step, lds); break;
                    case kA: run_loaded<NE, QA, BIG, FR, kA>(a, rr, r, step, lds); break;
                    case kF: run_loaded<NE, QA, BIG, FR, kF>(a, rr, r, step, lds); break;
                    case kF2:
                        if constexpr (BIG) run_loaded<NE, QA, BIG, FR, kF2>(a, rr, r, step, lds);
                        break;
                    default: run_loaded<NE, QA, BIG, FR, kLm>(a, rr, r, step, lds); break;
                }
            }
        }
    }
    if (blockIdx.x == 0 && thread_id() == 0) {
        a.st_pos[0] = a.pos0 + a.n_steps;
        a.st_pos[1] = a.gen0 + a.n_steps;
    }
}

template <int NE, bool QA, bool BIG, int SPLIT>
int launch(const RelayArgs& a, const RelayPlan& p, hipStream_t s) {
    auto kern = decode_relay_kernel<NE, QA, BIG, SPLIT>;
    FMLH_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(p.smem)));
    if (inject_fault(kFaultLaunch))
        return set_error(FMLH_E_HIP, "decode_relay_kernel: launch failed (injected by FMLH_FAULT)");
    RelayArgs args = a;
    void* params[] = {&args};
    const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kern), dim3(p.G), dim3(kThreads),
                                                    params, static_cast<unsigned>(p.smem), s);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        set_error(FMLH_E_HIP, "relay decode: cooperative launch refused (%s)", hipGetErrorString(e));
        return kPersistRefused;
    }
    return FMLH_OK;
}

}  // namespace relay
}  // namespace fmlh
