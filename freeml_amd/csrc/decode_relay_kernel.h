// Relay decode kernel for one sequence (see decode_relay.h for the team layout).
//
// Step s of a launch decodes position pos = pos0 + s.  Every exchange word of the step carries
// epoch e(s) = epoch_base + s + 1 and every buffer is written once per step, so one epoch per
// step suffices.  Single buffers are safe because every consumer of a word reads it before it
// publishes its own outputs, and everything it publishes leads to the next step's token: a word
// is only rewritten (next step) after the token of this step exists, i.e. after all its
// consumers have read it.
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
// Attention (A): keys 0..pos of one head, 16-key groups w, w + 8 per wave w (block_size <= 256:
// at most two groups), K/V rows in registers through bounded buffer loads (rows from pos on
// read as zero) requested before q is polled; key pos comes from the polled words.  Then the
// head's share of the attention projection, and last the step's K/V cache rows (the only
// workgroup that reads them later is this one, the same role of later steps).
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
constexpr int kPasses = kRelayTeamRows / kRowsPerPass;           // 3
constexpr int kScratch = 3 * kHD + kWaves * 256;                 // attention scratch (floats)
constexpr int kRawBufferFlags = 0x00020000;  // raw buffer, 32-bit data: loads past the records read 0
static_assert(kRelayTeamRows % kRowsPerPass == 0 && kRelayMaxVocab <= kRelayTeamRows, "whole passes");

enum RoleKind : int { kQ = 0, kA = 1, kF = 2, kLm = 3 };

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
    int kind, layer, idx;
};

__device__ __forceinline__ Role role_of(const RelayArgs& a, int H, int r) {
    const int per = a.nq + H + a.nf;
    Role ro;
    ro.layer = r / per;
    int o = r - ro.layer * per;
    if (ro.layer >= a.L) return Role{kLm, a.L, 0};
    if (o < a.nq) return Role{kQ, ro.layer, o};
    o -= a.nq;
    if (o < H) return Role{kA, ro.layer, o};
    return Role{kF, ro.layer, o - H};
}

// Registers of a role kind's weights (float4): Q and lm kPasses NE rows of K = C; F those plus
// its proj2 columns (C / (8 kWaves) = NE passes of 3); A its share of W_proj, NE / 2 passes of 4.
template <int NE, int K>
constexpr int wr_count() {
    return K == kA ? 2 * NE : K == kF ? kPasses * NE + 3 * NE : kPasses * NE;
}

// Requests the weights of role ro (of kind K) into wr.  Nothing waits for them here.
template <int NE, int K>
__device__ __forceinline__ void load_weights(const RelayArgs& a, const Role& ro, floatx4 (&wr)[wr_count<NE, K>()]) {
    constexpr int C = 64 * NE;
    const int lane = lane_id(), wave = wave_id();
    if constexpr (K == kA) {
        const PersistLayer& lw = a.layers[ro.layer];
        const float* src = lw.wproj + (size_t)(16 * wave + (lane >> 2)) * C + kHD * ro.idx + 16 * (lane & 3);
#pragma unroll
        for (int p = 0; p < NE / 2; ++p)
#pragma unroll
            for (int c = 0; c < 4; ++c) wr[4 * p + c] = ld4(src + (size_t)p * 16 * kWaves * C + 4 * c);
    } else {
        const float* src;
        int rows;
        if constexpr (K == kLm) {
            src = a.lm;
            rows = a.V;
        } else {
            const PersistLayer& lw = a.layers[ro.layer];
            src = (K == kQ ? lw.wqkvT : lw.wfcT) + (size_t)ro.idx * kRelayTeamRows * C;
            rows = kRelayTeamRows;
            if constexpr (K == kF) {  // W_proj2^T[o][96 idx + 12 (lane % 8) ..], o = 64 p + 8 wave + lane / 8
                const float* w2 = lw.w2T + (size_t)(8 * wave + (lane >> 3)) * 4 * C + kRelayTeamRows * ro.idx +
                                  12 * (lane & 7);
                static_assert(C / (8 * kWaves) == NE && kPasses * NE + 3 * NE == wr_count<NE, K>(), "F registers");
#pragma unroll
                for (int p = 0; p < NE; ++p)
#pragma unroll
                    for (int c = 0; c < 3; ++c)
                        wr[kPasses * NE + 3 * p + c] = ld4(w2 + (size_t)p * 8 * kWaves * 4 * C + 4 * c);
            }
        }
        const int t = lane & 15, g = lane >> 4;
#pragma unroll
        for (int p = 0; p < kPasses; ++p) {
            const float* w = src + (size_t)min(kRowsPerPass * p + 4 * wave + g, rows - 1) * C + 4 * t;
#pragma unroll
            for (int j = 0; j < NE; ++j) wr[NE * p + j] = ld4(w + 64 * j);
        }
    }
}

// This step's token: hist at the launch's first step, then the lm_head role's word.
__device__ __forceinline__ int token_in(const RelayArgs& a, int step, uint32_t ep, int* tokslot, int* bail) {
    if (thread_id() == 0) {
        int t;
        if (step == 0) {
            t = a.hist[a.pos0];
        } else {
            const uint64_t* p[1] = {a.tokw};
            uint64_t v[1];
            ll_issue_n(p, v, ep);
            ll_settle_n(p, v, ep, bail, a.err);
            t = static_cast<int>(static_cast<uint32_t>(v[0]));
        }
        *tokslot = t;
    }
    lds_barrier();
    const int t = *tokslot;
    return t < 0 || t >= a.V ? 0 : t;  // a corrupt word must not index out of the embedding
}

// Polls N1 + N2 exchange words: word k < N1 at b1 + k kStride bytes, word N1 + k at
// b2 + k kStride, each plus the lane's `off` bytes, until every one carries `epoch`.  Buffer
// loads with sc1 (the agent-scope coherent load that ll_load is), so a word's address is an
// SGPR offset from the lane's and no 64-bit address is held per word.  First every word is
// loaded, then rounds load the stale words again (wave-uniform exit, as ll_settle_n); each
// round starts with a compiler memory barrier, so no load of a round is merged with or hoisted
// above an earlier one.
constexpr int kPollAux = 0x10;  // sc1
template <int N1, int N2, int kStride>
__device__ __forceinline__ void poll_words(const uint64_t* b1, const uint64_t* b2, int off, uint32_t epoch,
                                           uint64_t (&v)[N1 + N2], int* bail, unsigned* err) {
    const auto r1 = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(b1), 0, N1 * kStride, kRawBufferFlags);
    const auto r2 = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(b2), 0, N2 * kStride, kRawBufferFlags);
    auto load = [&](int k) -> uint64_t {
        if (k < N1) return __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(r1, off, k * kStride, kPollAux));
        return __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(r2, off, (k - N1) * kStride, kPollAux));
    };
#pragma unroll
    for (int k = 0; k < N1 + N2; ++k) v[k] = load(k);
    int it = 0;
    while (true) {
        bool stale = false;
#pragma unroll
        for (int k = 0; k < N1 + N2; ++k) stale |= !persist::ll_current(v[k], epoch);
        if (__builtin_amdgcn_ballot_w64(stale) == 0 || !persist::ll_keep_polling(it, bail, err)) return;
        asm volatile("" ::: "memory");
#pragma unroll
        for (int k = 0; k < N1 + N2; ++k) {
            const bool need = !persist::ll_current(v[k], epoch);
            uint64_t nv = v[k];
            if (need) nv = load(k);
            v[k] = need ? nv : v[k];
        }
    }
}

// x entering layer l into xs (thread o < C owns entry o): the embedding of this step's token
// (l = 0), else the F team's word of layer l - 1.  kDx1 (F roles): plus the sum of the H
// attention-projection partials of layer l, in head order.
template <int NE, bool kDx1>
__device__ __forceinline__ void x_in(const RelayArgs& a, int l, int step, int pos, uint32_t ep, float* xs,
                                     int* flags) {
    constexpr int C = 64 * NE, H = C / kHD;
    int* bail = flags;
    const int o = thread_id();
    const uint64_t* dx1 = a.dx1w + (size_t)l * H * C;
    float x, d = 0.f;
    if (l == 0) {
        const int token = token_in(a, step, ep, flags + 1, bail);
        if (o >= C) return;  // whole waves (C is a multiple of 64)
        x = a.tok[(size_t)token * C + o] + a.pos_emb[(size_t)pos * C + o];
        if constexpr (kDx1) {
            uint64_t v[H];
            poll_words<H, 0, C * 8>(dx1, nullptr, 8 * o, ep, v, bail, a.err);
            d = ll_float(v[0]);
#pragma unroll
            for (int hh = 1; hh < H; ++hh) d += ll_float(v[hh]);
        }
    } else {
        if (o >= C) return;
        uint64_t v[1];
        poll_words<1, 0, C * 8>(a.xw + (size_t)l * C, nullptr, 8 * o, ep, v, bail, a.err);
        x = ll_float(v[0]);
        if constexpr (kDx1) {  // the dx1 words come later (two hand-offs): polled only from now
            uint64_t u[H];
            poll_words<H, 0, C * 8>(dx1, nullptr, 8 * o, ep, u, bail, a.err);
            d = ll_float(u[0]);
#pragma unroll
            for (int hh = 1; hh < H; ++hh) d += ll_float(u[hh]);
        }
    }
    xs[o] = kDx1 ? x + d : x;
}

// LayerNorm parameters of lane l: elements l + 64 m.  Loaded when a role starts, before its
// inputs are polled, so their latency hides behind the wait.
template <int NE>
struct LnRegs {
    float g[NE], b[NE];
};
template <int NE>
__device__ __forceinline__ LnRegs<NE> ln_params(const float* g, const float* b) {
    LnRegs<NE> r;
    const int lane = lane_id();
#pragma unroll
    for (int m = 0; m < NE; ++m) {
        r.g[m] = ld1(g + lane + 64 * m);
        r.b[m] = b ? ld1(b + lane + 64 * m) : 0.f;
    }
    return r;
}

// LayerNorm of the C floats at xs into xn (wave 0; two-pass variance, layernorm_kernel's order).
template <int NE>
__device__ __forceinline__ void layer_norm(const float* xs, const LnRegs<NE>& p, float* xn) {
    constexpr int C = 64 * NE;
    if (wave_id() == 0) {
        const int lane = lane_id();
        float v[NE];
#pragma unroll
        for (int m = 0; m < NE; ++m) v[m] = xs[lane + 64 * m];
        float s = 0.f;
#pragma unroll
        for (int m = 0; m < NE; ++m) s += v[m];
        const float mean = wave_sum(s) * (1.0f / C);
        float q = 0.f;
#pragma unroll
        for (int m = 0; m < NE; ++m) {
            const float d = v[m] - mean;
            q += d * d;
        }
        const float inv_std = __builtin_amdgcn_rsqf(wave_sum(q) * (1.0f / C) + 1e-5f);  // v_rsq_f32: 1 ulp
#pragma unroll
        for (int m = 0; m < NE; ++m) xn[lane + 64 * m] = ((v[m] - mean) * inv_std) * p.g[m] + p.b[m];
    }
    lds_barrier();
}

// The role's rows (wr, layout above) times xn (LDS).  emit(row, value) runs once per row, after
// the last pass, in lane t == p of the row's 16 lanes (which keeps pass p's sum); rows >= `rows`
// emit nothing.
template <int NE, class Emit>
__device__ __forceinline__ void gemv_regs(const floatx4* wr, const float* xn, int rows, Emit emit) {
    const int lane = lane_id(), wave = wave_id();
    const int t = lane & 15, g = lane >> 4;
    floatx4 xq[NE];
#pragma unroll
    for (int j = 0; j < NE; ++j) xq[j] = lds4(xn + 4 * (16 * j + t));
    float mine = 0.f;
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < NE; ++j) acc = fma4(wr[NE * p + j], xq[j], acc);
        acc = row16_sum(acc);
        mine = t == p ? acc : mine;
    }
    const int row = kRowsPerPass * t + 4 * wave + g;
    if (t < kPasses && row < rows) emit(row, mine);
}

// One role of one step (kind K; weights in wr).
template <int NE, int K>
__device__ __forceinline__ void run_role(const RelayArgs& a, const Role& ro, int r, int step,
                                         const floatx4 (&wr)[wr_count<NE, K>()], float* lds) {
    constexpr int C = 64 * NE, H = C / kHD, NCK = kHD / 16;
    constexpr int NF = 4 * C / kRelayTeamRows;
    float* sv = lds;                              // kScratch floats: attention scratch (A), h and partials (F), logits (lm)
    float* xs = sv + kScratch;                    // x (C)
    float* xn = xs + C;                           // normalised x (C)
    int* flags = reinterpret_cast<int*>(xn + C);  // [0] bail, [1] token
    int* bail = flags;
    const int pos = a.pos0 + step;
    const uint32_t ep = a.epoch_base + static_cast<uint32_t>(step) + 1u;
    const int l = ro.layer;
    const int tid = thread_id(), lane = lane_id(), wave = wave_id();
    (void)NCK;
    (void)NF;
    auto stamp = [&](int point) {
        if (a.trace && tid == 0 && step < kRelayTraceSteps)
            a.trace[((size_t)step * a.roles + r) * kRelayTracePoints + point] = wall_clock64();
    };
    stamp(0);
    if constexpr (K == kQ) {
        // ---- x_l, LN0, rows of W_qkv^T -> q / k_new / v_new words --------------------
        const PersistLayer& lw = a.layers[l];
        const LnRegs<NE> ln = ln_params<NE>(lw.ln0g, lw.ln0b);
        x_in<NE, false>(a, l, step, pos, ep, xs, flags);
        lds_barrier();
        stamp(1);
        layer_norm<NE>(xs, ln, xn);
        stamp(2);
        uint64_t* dst = a.qkvw + (size_t)l * 3 * C + (size_t)ro.idx * kRelayTeamRows;
        gemv_regs<NE>(wr, xn, kRelayTeamRows, [&](int row, float v) { ll_put(&dst[row], v, ep); });
        stamp(3);
    } else if constexpr (K == kA) {
        // ---- attention of head h, then its attention-projection partial -------------
        const int h = ro.idx;
        const size_t slab_kv = (((size_t)l * a.Bmax) * H + h) * (size_t)a.T * kHD;
        float* kb = a.kc + slab_kv;
        float* vb = a.vc + slab_kv;
        const int nkeys = pos + 1;
        const int kk = lane >> 2, part = lane & 3;  // score lanes: key kk, dims part * 16 ..
        const int d4 = lane & 15, kq = lane >> 4;   // P.V lanes: dims 4 d4 .., keys kq + 4 i
        const int gp = pos >> 4;                    // the 16-key group holding key pos
        floatx4 kr[kGroupsPerWave][NCK], vr[kGroupsPerWave][4];
        {
            const int bytes = pos * kHD * static_cast<int>(sizeof(float));
            const auto rk = __builtin_amdgcn_make_buffer_rsrc(kb, 0, bytes, kRawBufferFlags);
            const auto rv = __builtin_amdgcn_make_buffer_rsrc(vb, 0, bytes, kRawBufferFlags);
#pragma unroll
            for (int gi = 0; gi < kGroupsPerWave; ++gi) {
                const int base = kKeyGroup * (wave + kWaves * gi);
                if (base < nkeys) {
#pragma unroll
                    for (int c = 0; c < NCK; ++c) kr[gi][c] = bload4(rk, (base + kk) * kHD + part * 16 + 4 * c);
#pragma unroll
                    for (int i = 0; i < 4; ++i) vr[gi][i] = bload4(rv, (base + kq + 4 * i) * kHD + 4 * d4);
                }
            }
        }
        // Attention scratch in sv.  Each wave's 256 floats hold in turn its softmax
        // weights (64), its P.V partials (256, written after the weights are read) and
        // its combine row (64 + 2, written after the partials are read); all three are
        // the wave's own, read in order.
        float* qs = sv;                   // q, k_new, v_new (3 x 64)
        float* wsc = qs + 3 * kHD;        // kWaves x 256
        float kn = 0.f, vn = 0.f;         // wave 0: the step's K/V cache row entries
        if (wave == 0) {
            const uint64_t* src = a.qkvw + (size_t)l * 3 * C + kHD * h + lane;
            const uint64_t* pw[3] = {src, src + C, src + 2 * C};
            uint64_t vw[3];
            ll_issue_n(pw, vw, ep);
            ll_settle_n(pw, vw, ep, bail, a.err);
            kn = ll_float(vw[1]);
            vn = ll_float(vw[2]);
            qs[lane] = ll_float(vw[0]);
            qs[kHD + lane] = kn;
            qs[2 * kHD + lane] = vn;
        }
        lds_barrier();
        stamp(1);
        floatx4 qv[NCK];
        float s_pos = 0.f;  // score of key pos (k_new), in every lane
#pragma unroll
        for (int c = 0; c < NCK; ++c) {
            qv[c] = lds4(qs + part * 16 + 4 * c);
            s_pos += dot4(qv[c], lds4(qs + kHD + part * 16 + 4 * c));
        }
        s_pos = quad_sum(s_pos) * a.scale;
        float sc[kGroupsPerWave];
        float mx = -INFINITY;
#pragma unroll
        for (int gi = 0; gi < kGroupsPerWave; ++gi) {
            const int base = kKeyGroup * (wave + kWaves * gi);
            sc[gi] = -INFINITY;
            if (base < nkeys) {
                float sv2 = 0.f;
#pragma unroll
                for (int c = 0; c < NCK; ++c) sv2 += dot4(qv[c], kr[gi][c]);
                const float t = quad_sum(sv2) * a.scale;
                sc[gi] = base + kk == pos ? s_pos : t;
                if (base + kk < nkeys) mx = fmaxf(mx, sc[gi]);
            }
        }
        const float m = wave_max(mx);  // -inf only if this wave has no key
        float* pl = wsc + wave * 256;   // [group][4 (k % 4) + k / 4]
        float psum = 0.f;
#pragma unroll
        for (int gi = 0; gi < kGroupsPerWave; ++gi) {
            const int j = kKeyGroup * (wave + kWaves * gi) + kk;
            const float pv = j < nkeys ? __expf(sc[gi] - m) : 0.f;
            if (part == 0) {
                psum += pv;
                pl[16 * gi + 4 * (kk & 3) + (kk >> 2)] = pv;
            }
        }
        const float lsum = wave_sum(psum);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's softmax weights are in LDS
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int gi = 0; gi < kGroupsPerWave; ++gi) {
            if (kKeyGroup * (wave + kWaves * gi) < nkeys) {
                const floatx4 pp = lds4(pl + 16 * gi + 4 * kq);
#pragma unroll
                for (int i = 0; i < 4; ++i) {  // key kq + 4 i of the group
                    o.x += pp[i] * vr[gi][i][0];
                    o.y += pp[i] * vr[gi][i][1];
                    o.z += pp[i] * vr[gi][i][2];
                    o.w += pp[i] * vr[gi][i][3];
                }
            }
        }
        {  // key pos: its V row read as zero above
            const float pm = wave == gp % kWaves && kq == (pos & 3) ? __expf(s_pos - m) : 0.f;
            const floatx4 t = lds4(qs + 2 * kHD + 4 * d4);
            o.x += pm * t[0];
            o.y += pm * t[1];
            o.z += pm * t[2];
            o.w += pm * t[3];
        }
        float* ow = wsc + wave * 256;
        *reinterpret_cast<float4*>(ow + kq * 64 + 4 * d4) = o;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        float* cw = wsc + wave * 256;
        const float osum = (ow[lane] + ow[64 + lane]) + (ow[128 + lane] + ow[192 + lane]);
        cw[2 + lane] = osum;
        if (lane == 0) {
            cw[0] = m;
            cw[1] = lsum;
        }
        lds_barrier();
        // Wave 0 combines the waves' rows into y_h (in xs, idle during attention).
        float* ys = xs;
        if (wave == 0) {
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
            ys[lane] = od * __builtin_amdgcn_rcpf(lt);
        }
        lds_barrier();
        stamp(2);
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
        uint64_t* dst = a.dx1w + ((size_t)l * H + h) * C;
        if (part < PP) ll_put(&dst[part * 16 * kWaves + 16 * wave + (lane >> 2)], mine, ep);
        stamp(3);
        if (wave == 0) {  // the cache row of this step
            kb[(size_t)pos * kHD + lane] = kn;
            vb[(size_t)pos * kHD + lane] = vn;
            // Written before the role ends: the next step's role (this WG) loads the row
            // right after the barrier below.
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
    } else if constexpr (K == kF) {
        // ---- x_l + sum of the heads' dx1 partials, LN1, rows of W_fc^T, GELU -> h;
        //      proj2 partial of every output over the WG's 96 columns ----------------
        const PersistLayer& lw = a.layers[l];
        const LnRegs<NE> ln = ln_params<NE>(lw.ln1g, lw.ln1b);
        x_in<NE, true>(a, l, step, pos, ep, xs, flags);
        lds_barrier();
        stamp(1);
        layer_norm<NE>(xs, ln, xn);
        float* hs = sv;  // the WG's 96 entries of h
        gemv_regs<NE>(wr, xn, kRelayTeamRows, [&](int row, float v) { hs[row] = gelu_ref(v); });
        lds_barrier();
        stamp(2);
        // Output o = 64 p + 8 wave + lane / 8: 8 lanes per row, 12 columns each.
        const int t8 = lane & 7;
        constexpr int PP = C / (8 * kWaves);
        static_assert(PP == NE && PP <= 8, "one pass per lane of an octet");
        floatx4 hq[3];
#pragma unroll
        for (int c = 0; c < 3; ++c) hq[c] = lds4(hs + 12 * t8 + 4 * c);
        float mine = 0.f;  // lane t8 == p keeps pass p's sum
#pragma unroll
        for (int p = 0; p < PP; ++p) {
            float acc = 0.f;
#pragma unroll
            for (int c = 0; c < 3; ++c) acc = fma4(wr[kPasses * NE + 3 * p + c], hq[c], acc);
            acc = oct_sum(acc);
            mine = t8 == p ? acc : mine;
        }
        if (t8 < PP) ll_put(&a.partw[((size_t)l * NF + ro.idx) * C + 64 * t8 + 8 * wave + (lane >> 3)], mine, ep);
        stamp(3);
        // x_{l+1} for rows 24 idx .. (C / NF rows): x' + the NF partials of each row, in team
        // order (thread f R + i < NF R polls partial f of row i).
        constexpr int R = C / NF;
        float* pp = sv + kRelayTeamRows;  // [NF][R], after h
        static_assert(kRelayTeamRows + NF * R <= kScratch, "F scratch");
        const int r0 = ro.idx * R;
        if (tid < NF * R) {
            const int f = tid / R, i = tid - f * R;
            uint64_t v[1];
            const uint64_t* base = a.partw + (size_t)l * NF * C + r0;
            poll_words<1, 0, NF * C * 8>(base, base, 8 * (f * C + i), ep, v, bail, a.err);
            pp[tid] = ll_float(v[0]);
        }
        lds_barrier();
        stamp(4);
        if (tid < R) {
            float dsum = pp[tid];
#pragma unroll
            for (int f = 1; f < NF; ++f) dsum += pp[f * R + tid];
            ll_put(&a.xw[(size_t)(l + 1) * C + r0 + tid], xs[r0 + tid] + dsum, ep);
        }
        stamp(5);
    } else {
        // ---- lm_head: ln_f, logits, first maximum -> the next token -----------------------
        const LnRegs<NE> ln = ln_params<NE>(a.lnf_g, a.lnf_b);
        x_in<NE, false>(a, a.L, step, pos, ep, xs, flags);
        lds_barrier();
        stamp(1);
        layer_norm<NE>(xs, ln, xn);
        float* lg = sv;
        const bool keep = a.logit_hist && (size_t)(a.gen0 + step) < a.hist_slots;
        gemv_regs<NE>(wr, xn, a.V, [&](int row, float v) {
            lg[row] = v;
            a.logits[row] = v;
            if (keep) a.logit_hist[(size_t)(a.gen0 + step) * a.V + row] = v;
        });
        lds_barrier();
        stamp(2);
        if (wave == 0) {
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
                a.hist[pos + 1] = tk;
                if (step + 1 < a.n_steps) ll_put_bits(a.tokw, static_cast<uint32_t>(tk), ep + 1u);
            }
        }
        stamp(3);
        }
}

// A workgroup with one role: its weights are loaded once, before the first step.
template <int NE, int K>
__device__ __forceinline__ void run_single(const RelayArgs& a, const Role& ro, int r, float* lds) {
    floatx4 wr[wr_count<NE, K>()];
    load_weights<NE, K>(a, ro, wr);
    for (int step = 0; step < a.n_steps; ++step) {
        run_role<NE, K>(a, ro, r, step, wr, lds);
        lds_barrier();  // every wave is done with this step's LDS before the next step writes it
    }
}

// One role of a workgroup with two: the role's weights are requested when it starts (its
// inputs come much later: the role before it in the step order is several layers back).
template <int NE, int K>
__device__ __forceinline__ void run_loaded(const RelayArgs& a, const Role& ro, int r, int step, float* lds) {
    floatx4 wr[wr_count<NE, K>()];
    load_weights<NE, K>(a, ro, wr);
    run_role<NE, K>(a, ro, r, step, wr, lds);
}

template <int NE>
__global__ __launch_bounds__(kThreads) void decode_relay_kernel(RelayArgs a) {
    constexpr int C = 64 * NE, H = C / kHD;
    static_assert(C % kHD == 0 && NE % 2 == 0, "heads");
    static_assert(3 * C % kRelayTeamRows == 0 && 4 * C % kRelayTeamRows == 0, "teams");
    extern __shared__ float lds[];
    int* bail = reinterpret_cast<int*>(lds + kScratch + 2 * C);

    const int w = static_cast<int>(blockIdx.x), G = static_cast<int>(gridDim.x);
    if (thread_id() == 0) __hip_atomic_store(bail, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    lds_barrier();
    const Role ro = role_of(a, H, w);
    if (w + G >= a.roles) {
        switch (ro.kind) {
            case kQ: run_single<NE, kQ>(a, ro, w, lds); break;
            case kA: run_single<NE, kA>(a, ro, w, lds); break;
            case kF: run_single<NE, kF>(a, ro, w, lds); break;
            default: run_single<NE, kLm>(a, ro, w, lds); break;
        }
    } else {
        for (int step = 0; step < a.n_steps; ++step) {
            for (int r = w; r < a.roles; r += G) {
                const Role rr = role_of(a, H, r);
                switch (rr.kind) {
                    case kQ: run_loaded<NE, kQ>(a, rr, r, step, lds); break;
                    case kA: run_loaded<NE, kA>(a, rr, r, step, lds); break;
                    case kF: run_loaded<NE, kF>(a, rr, r, step, lds); break;
                    default: run_loaded<NE, kLm>(a, rr, r, step, lds); break;
                }
                lds_barrier();  // every wave is done with this role's LDS before the next writes it
            }
        }
    }
    if (blockIdx.x == 0 && thread_id() == 0) {
        a.st_pos[0] = a.pos0 + a.n_steps;
        a.st_pos[1] = a.gen0 + a.n_steps;
    }
}

template <int NE>
int launch(const RelayArgs& a, const RelayPlan& p, hipStream_t s) {
    auto kern = decode_relay_kernel<NE>;
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
