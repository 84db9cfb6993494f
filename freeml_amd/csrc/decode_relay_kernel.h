// Relay decode kernel for one sequence (see decode_relay.h for the team layout).
//
// Step s of a launch decodes position pos = pos0 + s.  Every exchange word of the step carries
// epoch e(s) = epoch_base + s + 1 and every buffer is written once per step, so one epoch per
// step suffices.  Single buffers are safe because every consumer of a word reads it before it
// publishes its own outputs, and everything it publishes leads to the next step's token: a word
// is only rewritten (next step) after the token of this step exists, i.e. after all its
// consumers have read it.
//
// Eight waves per workgroup (two per SIMD).  Team products (VALU dot products from LDS, DPP
// reductions):
//   rows of K = C   (Q, F, lm): 16 lanes per row (one DPP row), four rows per wave at a time;
//                   lane t of a row holds x[4 (16 j + t) ..] for j < C / 64
//   rows of K = 4C  (P):        the same layout, each wave over its own 4C / 8 columns; the
//                   waves' partial sums meet in LDS
// A team's weight slice is copied to LDS (global_load_lds_dwordx4) before its inputs are
// polled, so it streams while the workgroup waits; a workgroup with one role keeps it for the
// whole launch.
//
// Attention (A): keys 0..pos of one head, 16-key groups w, w + 8 per wave w (block_size <= 256:
// at most two groups), K/V rows in registers through bounded buffer loads (rows from pos on
// read as zero) requested before q is polled; key pos comes from the polled words.  Then the
// head's share of the attention projection: dx1_h[o] = W_proj[o][64 h ..] . y_h for every
// output o, four lanes per output.
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
constexpr int kRawBufferFlags = 0x00020000;  // raw buffer, 32-bit data: loads past the records read 0

enum RoleKind : int { kQ = 0, kA = 1, kF = 2, kP = 3, kLm = 4 };

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
// Barrier after this wave's LDS copies have landed.
__device__ __forceinline__ void copies_landed() {
    asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
#pragma clang diagnostic pop

__device__ __forceinline__ floatx4 lds4(const float* p) { return *reinterpret_cast<const floatx4*>(p); }
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

// Sum over the 16 lanes of a DPP row, in every lane of the row (row_ror 8, 4, 2, 1).
template <int kCtrl>
__device__ __forceinline__ float row16_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += row16_move<0x128>(v);
    v += row16_move<0x124>(v);
    v += row16_move<0x122>(v);
    v += row16_move<0x121>(v);
    return v;
}

struct Role {
    int kind, layer, idx;
};


__device__ __forceinline__ Role role_of(const RelayArgs& a, int H, int r) {
    const int per = a.nq + H + a.nf + a.np;
    Role ro;
    ro.layer = r / per;
    int o = r - ro.layer * per;
    if (ro.layer >= a.L) return Role{kLm, a.L, 0};
    if (o < a.nq) return Role{kQ, ro.layer, o};
    o -= a.nq;
    if (o < H) return Role{kA, ro.layer, o};
    o -= H;
    if (o < a.nf) return Role{kF, ro.layer, o};
    return Role{kP, ro.layer, o - a.nf};
}

// Copies n floats (n a multiple of 4) from src to LDS dst, 1 KB per wave instruction.
__device__ __forceinline__ void copy_to_lds(float* dst, const float* src, int n) {
    const int lane = lane_id(), wave = wave_id();
    for (int c0 = 256 * wave; c0 < n; c0 += 256 * kWaves)
        if (c0 + 4 * lane < n) copy16_to_lds(dst + c0, src + c0 + 4 * lane);
}

// Requests the weight slice of role ro into LDS (wl).
template <int NE>
__device__ __forceinline__ void fetch_weights(const RelayArgs& a, Role ro, float* wl) {
    constexpr int C = 64 * NE;
    if (ro.kind == kLm) {
        copy_to_lds(wl, a.lm, a.V * C);
        return;
    }
    const PersistLayer& lw = a.layers[ro.layer];
    if (ro.kind == kQ) {
        const int R = 3 * C / a.nq;
        copy_to_lds(wl, lw.wqkvT + (size_t)ro.idx * R * C, R * C);
    } else if (ro.kind == kF) {
        const int R = 4 * C / a.nf;
        copy_to_lds(wl, lw.wfcT + (size_t)ro.idx * R * C, R * C);
    } else if (ro.kind == kP) {
        const int R = C / a.np;
        copy_to_lds(wl, lw.w2T + (size_t)ro.idx * R * 4 * C, R * 4 * C);
    } else {  // A: columns [64 h, 64 h + 64) of every W_proj row, as [C][64]
        const int lane = lane_id(), wave = wave_id();
        for (int o0 = 4 * wave; o0 < C; o0 += 4 * kWaves)
            copy16_to_lds(wl + o0 * kHD, lw.wproj + (size_t)(o0 + lane / 16) * C + kHD * ro.idx + 4 * (lane % 16));
    }
}

// Words src[0..N) into dst (LDS), all threads of the WG, every load in flight at once (one
// round trip when the words are already there).
template <int N>
__device__ __forceinline__ void gather_all(const uint64_t* src, uint32_t epoch, float* dst, int* bail,
                                           unsigned* err) {
    constexpr int K = (N + kThreads - 1) / kThreads;
    const int tid = thread_id();
    const uint64_t* p[K];
    uint64_t v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) p[k] = k * kThreads + tid < N ? src + k * kThreads + tid : nullptr;
    ll_issue_n(p, v, epoch);
    ll_settle_n(p, v, epoch, bail, err);
#pragma unroll
    for (int k = 0; k < K; ++k)
        if (p[k] != nullptr) dst[k * kThreads + tid] = ll_float(v[k]);
}

// x entering layer l, all C entries, into LDS xs: the embedding of this step's token (l = 0)
// or the P team's words of layer l - 1.
template <int NE>
__device__ __forceinline__ void x_in(const RelayArgs& a, int l, int token, int pos, uint32_t ep, float* xs,
                                     int* bail) {
    constexpr int C = 64 * NE;
    if (l == 0) {
        for (int c = thread_id(); c < C; c += kThreads)
            xs[c] = a.tok[(size_t)token * C + c] + a.pos_emb[(size_t)pos * C + c];
    } else {
        gather_all<C>(a.xw + (size_t)l * C, ep, xs, bail, a.err);
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
        r.g[m] = g[lane + 64 * m];
        r.b[m] = b ? b[lane + 64 * m] : 0.f;
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

// R rows of C weights in LDS times xn (LDS), 16 lanes per row, four rows per wave per pass
// (kRowsPerPass rows per pass of the workgroup); emit(row, value) in lane t == 0 of each row's
// lanes.  Rows past R read row R - 1 and emit nothing.  (lm_head: R = vocabulary.)
constexpr int kRowsPerPass = 4 * kWaves;
template <int NE, class Emit>
__device__ __forceinline__ void gemv16(const float* wl, int R, const float* xn, Emit emit) {
    constexpr int C = 64 * NE;
    const int lane = lane_id(), wave = wave_id();
    const int t = lane & 15, g = lane >> 4;
    floatx4 xq[NE];
#pragma unroll
    for (int j = 0; j < NE; ++j) xq[j] = lds4(xn + 4 * (16 * j + t));
    for (int r0 = 0; r0 < R; r0 += 2 * kRowsPerPass) {
        floatx4 wv[2][NE];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const float* w = wl + min(r0 + kRowsPerPass * b + 4 * wave + g, R - 1) * C + 4 * t;
#pragma unroll
            for (int j = 0; j < NE; ++j) wv[b][j] = lds4(w + 64 * j);
        }
        float acc[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            acc[b] = 0.f;
#pragma unroll
            for (int j = 0; j < NE; ++j) acc[b] = fma4(wv[b][j], xq[j], acc[b]);
            acc[b] = row16_sum(acc[b]);
        }
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int row = r0 + kRowsPerPass * b + 4 * wave + g;
            if (t == 0 && row < R) emit(row, acc[b]);
        }
    }
}

// The same for a compile-time R (a multiple of kRowsPerPass), fully unrolled and software-pipelined: the
// weights of pass p + 1 are requested before the products of pass p, and every lane of a row
// emits (the same value), so no branch separates a pass's reads from their use.
//
// kDeferred: emit runs once, after the last pass, in lanes t < P of each row's lanes (lane t
// holds pass t's row), so per-row work in emit (GELU) runs once per wave instead of per pass.
template <int NE, int R, bool kDeferred, class Emit>
__device__ __forceinline__ void gemv16_fixed(const float* wl, const float* xn, Emit emit) {
    constexpr int C = 64 * NE, P = R / kRowsPerPass;
    static_assert(R % kRowsPerPass == 0 && P <= 16, "whole passes");
    const int lane = lane_id(), wave = wave_id();
    const int t = lane & 15, g = lane >> 4;
    floatx4 xq[NE];
#pragma unroll
    for (int j = 0; j < NE; ++j) xq[j] = lds4(xn + 4 * (16 * j + t));
    const float* w0 = wl + (4 * wave + g) * C + 4 * t;
    floatx4 wv[2][NE];
#pragma unroll
    for (int j = 0; j < NE; ++j) wv[0][j] = lds4(w0 + 64 * j);
    float mine = 0.f;  // kDeferred: the sum of pass t
#pragma unroll
    for (int p = 0; p < P; ++p) {
        if (p + 1 < P) {
#pragma unroll
            for (int j = 0; j < NE; ++j) wv[(p + 1) & 1][j] = lds4(w0 + kRowsPerPass * (p + 1) * C + 64 * j);
        }
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < NE; ++j) acc = fma4(wv[p & 1][j], xq[j], acc);
        acc = row16_sum(acc);
        if constexpr (kDeferred)
            mine = t == p ? acc : mine;
        else
            emit(kRowsPerPass * p + 4 * wave + g, acc);
    }
    if constexpr (kDeferred) {
        if (t < P) emit(kRowsPerPass * t + 4 * wave + g, mine);
    }
}

template <int NE>
__global__ __launch_bounds__(kThreads) void decode_relay_kernel(RelayArgs a) {
    constexpr int C = 64 * NE, C4 = 4 * C, H = C / kHD, NCK = kHD / 16;
    static_assert(C % kHD == 0, "heads");
    extern __shared__ float lds[];
    float* wl = lds;                          // the role's weights
    float* sv = wl + kRelayWeightFloats;      // H x C floats: dx1 partials (F), h (P), attention scratch (A), logits (lm)
    float* xs = sv + H * C;                   // x (C)
    float* xn = xs + C;                       // normalised x (C); P: x' of its rows
    int* flags = reinterpret_cast<int*>(xn + C);  // [0] bail, [1] token
    int* bail = flags;

    const int w = static_cast<int>(blockIdx.x), G = static_cast<int>(gridDim.x);
    if (thread_id() == 0) __hip_atomic_store(bail, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const bool single = w + G >= a.roles;  // one role: its weights stay in LDS
    fetch_weights<NE>(a, role_of(a, H, w), wl);
    lds_barrier();

    for (int step = 0; step < a.n_steps; ++step) {
        const int pos = a.pos0 + step;
        const uint32_t ep = a.epoch_base + static_cast<uint32_t>(step) + 1u;
        for (int r = w; r < a.roles; r += G) {
            const Role ro = role_of(a, H, r);
            const int l = ro.layer;
            const int tid = thread_id(), lane = lane_id(), wave = wave_id();
            auto stamp = [&](int point) {
                if (a.trace && tid == 0 && step < kRelayTraceSteps)
                    a.trace[((size_t)step * a.roles + r) * kRelayTracePoints + point] = wall_clock64();
            };
            stamp(0);
            if (ro.kind == kQ) {
                // ---- x_l, LN0, rows of W_qkv^T -> q / k_new / v_new words --------------------
                const PersistLayer& lw = a.layers[l];
                const LnRegs<NE> ln = ln_params<NE>(lw.ln0g, lw.ln0b);
                const int token = l == 0 ? token_in(a, step, ep, flags + 1, bail) : 0;
                x_in<NE>(a, l, token, pos, ep, xs, bail);
                lds_barrier();
                stamp(1);
                layer_norm<NE>(xs, ln, xn);
                copies_landed();
                const int R = 3 * C / a.nq, r0 = ro.idx * R;
                uint64_t* dst = a.qkvw + (size_t)l * 3 * C + r0;
                gemv16_fixed<NE, kRelayTeamRows, false>(wl, xn, [&](int row, float v) { ll_put(&dst[row], v, ep); });
                stamp(2);
            } else if (ro.kind == kA) {
                // ---- attention of head h, then its attention-projection partial -------------
                const int h = ro.idx;
                const size_t slab = (((size_t)l * a.Bmax) * H + h) * (size_t)a.T * kHD;
                float* kb = a.kc + slab;
                float* vb = a.vc + slab;
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
                // attention scratch in sv
                // Each wave's 256 floats hold in turn its softmax weights (64), its P.V partials
                // (256, written after the weights are read) and its combine row (64 + 2, written
                // after the partials are read); all three are the wave's own, read in order.
                float* qs = sv;                   // q, k_new, v_new (3 x 64)
                float* wsc = qs + 3 * kHD;        // kWaves x 256
                static_assert(3 * kHD + kWaves * 256 <= H * C && kHD <= C, "attention scratch");
                if (wave == 0) {
                    const uint64_t* src = a.qkvw + (size_t)l * 3 * C + kHD * h + lane;
                    const uint64_t* pw[3] = {src, src + C, src + 2 * C};
                    uint64_t vw[3];
                    ll_issue_n(pw, vw, ep);
                    ll_settle_n(pw, vw, ep, bail, a.err);
                    const float kn = ll_float(vw[1]), vn = ll_float(vw[2]);
                    qs[lane] = ll_float(vw[0]);
                    qs[kHD + lane] = kn;
                    qs[2 * kHD + lane] = vn;
                    kb[(size_t)pos * kHD + lane] = kn;  // the cache row of this step
                    vb[(size_t)pos * kHD + lane] = vn;
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
                copies_landed();
                // dx1 partial of head h: output o = 64 p + 16 wave + lane / 4, dims 16 part ..
                const floatx4* y4 = reinterpret_cast<const floatx4*>(ys) + 4 * part;
                floatx4 yv[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) yv[c] = y4[c];
                uint64_t* dst = a.dx1w + ((size_t)l * H + h) * C;
                // Six passes of 16 outputs per wave, software-pipelined over two register buffers.
                constexpr int PP = C / (16 * kWaves);
                const float* w0 = wl + (size_t)(16 * wave + (lane >> 2)) * kHD + 16 * part;
                floatx4 wv[2][4];
#pragma unroll
                for (int c = 0; c < 4; ++c) wv[0][c] = lds4(w0 + 4 * c);
#pragma unroll
                for (int p = 0; p < PP; ++p) {
                    if (p + 1 < PP) {
#pragma unroll
                        for (int c = 0; c < 4; ++c) wv[(p + 1) & 1][c] = lds4(w0 + (p + 1) * 16 * kWaves * kHD + 4 * c);
                    }
                    float acc = 0.f;
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc = fma4(wv[p & 1][c], yv[c], acc);
                    acc = quad_sum(acc);
                    if (part == 0) ll_put(&dst[p * 16 * kWaves + 16 * wave + (lane >> 2)], acc, ep);
                }
                stamp(2);
            } else if (ro.kind == kF) {
                // ---- x_l + sum of the heads' dx1 partials, LN1, rows of W_fc^T, GELU -> h ------
                const PersistLayer& lw = a.layers[l];
                const LnRegs<NE> ln = ln_params<NE>(lw.ln1g, lw.ln1b);
                const int token = l == 0 ? token_in(a, step, ep, flags + 1, bail) : 0;
                x_in<NE>(a, l, token, pos, ep, xs, bail);
                gather_all<H * C>(a.dx1w + (size_t)l * H * C, ep, sv, bail, a.err);
                lds_barrier();
                stamp(1);
                for (int c = tid; c < C; c += kThreads) {
                    float d = sv[c];
#pragma unroll
                    for (int hh = 1; hh < H; ++hh) d += sv[hh * C + c];
                    xs[c] += d;
                }
                lds_barrier();
                layer_norm<NE>(xs, ln, xn);
                copies_landed();
                const int R = 4 * C / a.nf, r0 = ro.idx * R;
                uint64_t* dst = a.hw + (size_t)l * C4 + r0;
                gemv16_fixed<NE, kRelayTeamRows, false>(wl, xn, [&](int row, float v) { ll_put(&dst[row], gelu_ref(v), ep); });
                stamp(2);
            } else if (ro.kind == kP) {
                // ---- rows of W_proj2^T over h, plus x' of its rows -> x of layer l + 1 ---------
                constexpr int R = kRelayPRows;
                const int r0 = ro.idx * R;
                const int token = l == 0 ? token_in(a, step, ep, flags + 1, bail) : 0;
                // x' = x_l + sum of the dx1 partials, for rows r0 .. r0 + R (thread k R + i: k < H
                // partial k of row i, k = H the row of x_l)
                float* xr = xn;  // [H + 1][R]
                if (tid < (H + 1) * R) {
                    const int k = tid / R, i = tid - k * R;
                    if (k == H && l == 0) {
                        xr[tid] = a.tok[(size_t)token * C + r0 + i] + a.pos_emb[(size_t)pos * C + r0 + i];
                    } else {
                        const uint64_t* p[1] = {k < H ? a.dx1w + ((size_t)l * H + k) * C + r0 + i
                                                      : a.xw + (size_t)l * C + r0 + i};
                        uint64_t v[1];
                        ll_issue_n(p, v, ep);
                        ll_settle_n(p, v, ep, bail, a.err);
                        xr[tid] = ll_float(v[0]);
                    }
                }
                gather_all<C4>(a.hw + (size_t)l * C4, ep, sv, bail, a.err);
                copies_landed();
                stamp(1);
                // Wave w takes columns [K4 w, K4 w + K4) of all R rows (K4 = 4C / kWaves), 16
                // lanes per row and four rows per pass, as gemv16_fixed; the waves' partial
                // sums then meet in LDS, where thread i < R adds x' of row i (x_l plus the
                // heads' partials in head order).
                constexpr int K4 = C4 / kWaves, NJ = K4 / 64, PASSES = R / 4;
                static_assert(K4 % 64 == 0 && R % 4 == 0, "P layout");
                float* part = xr + (H + 1) * R;  // [kWaves][R]
                const int t = lane & 15, g = lane >> 4;
                floatx4 hq[NJ];
#pragma unroll
                for (int j = 0; j < NJ; ++j) hq[j] = lds4(sv + K4 * wave + 4 * (16 * j + t));
                const float* w0 = wl + g * C4 + K4 * wave + 4 * t;
                floatx4 wv[2][NJ];
#pragma unroll
                for (int j = 0; j < NJ; ++j) wv[0][j] = lds4(w0 + 64 * j);
#pragma unroll
                for (int q = 0; q < PASSES; ++q) {
                    if (q + 1 < PASSES) {
#pragma unroll
                        for (int j = 0; j < NJ; ++j) wv[(q + 1) & 1][j] = lds4(w0 + 4 * (q + 1) * C4 + 64 * j);
                    }
                    float acc = 0.f;
#pragma unroll
                    for (int j = 0; j < NJ; ++j) acc = fma4(wv[q & 1][j], hq[j], acc);
                    acc = row16_sum(acc);
                    if (t == 0) part[wave * R + 4 * q + g] = acc;
                }
                lds_barrier();
                uint64_t* dst = a.xw + (size_t)(l + 1) * C + r0;
                if (tid < R) {
                    float d = xr[tid];
#pragma unroll
                    for (int hh = 1; hh < H; ++hh) d += xr[hh * R + tid];
                    const float xp = xr[H * R + tid] + d;
                    float acc = part[tid];
#pragma unroll
                    for (int v = 1; v < kWaves; ++v) acc += part[v * R + tid];
                    ll_put(&dst[tid], xp + acc, ep);
                }
                stamp(2);
            } else {
                // ---- lm_head: ln_f, logits, first maximum -> the next token -----------------------
                const LnRegs<NE> ln = ln_params<NE>(a.lnf_g, a.lnf_b);
                gather_all<C>(a.xw + (size_t)a.L * C, ep, xs, bail, a.err);
                lds_barrier();
                stamp(1);
                layer_norm<NE>(xs, ln, xn);
                copies_landed();
                float* lg = sv;
                const bool keep = a.logit_hist && (size_t)(a.gen0 + step) < a.hist_slots;
                gemv16<NE>(wl, a.V, xn, [&](int row, float v) {
                    lg[row] = v;
                    a.logits[row] = v;
                    if (keep) a.logit_hist[(size_t)(a.gen0 + step) * a.V + row] = v;
                });
                lds_barrier();
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
                stamp(2);
            }
            // Every wave is done with this role's LDS before the next role (or step) writes it;
            // then the next role of this workgroup (possibly the first of the next step) gets its
            // weights.
            lds_barrier();
            if (!single && (r + G < a.roles || step + 1 < a.n_steps))
                fetch_weights<NE>(a, role_of(a, H, r + G < a.roles ? r + G : w), wl);
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
