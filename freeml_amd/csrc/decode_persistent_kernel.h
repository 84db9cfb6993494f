// Persistent decode kernel: many greedy decode steps of the NanoLLM token loop in one
// cooperative launch, for small batches (B <= 8).  Included by the per-head-dimension
// translation units decode_persistent_hd{16,32,64}.hip.
//
// Why: a decode step at batch 1 moves ~45 MB (c2-sized model) -- a few microseconds of HBM
// time -- but as ~60 separate kernels it costs ~540 us, almost all launch and dependency
// latency.  Here every workgroup (WG, one per CU) stays resident for the whole loop and the
// phases of a step exchange their outputs through global memory.
//
// Exchange protocol ("LL" words).  Every value passed between WGs is a 64-bit word
// {payload bits, epoch}, written with one agent-scope store and read with agent-scope loads
// (both bypass the per-XCD L2, so no cache maintenance is needed).  A consumer polls the
// words themselves until their epoch is the one it expects, so a hand-off costs one store and
// one load round trip instead of a grid barrier plus a load.  Epochs are unique per
// (launch, step, hop) and increase monotonically across launches.
//
// Why single buffers are safe: hops 3, 4 and 5 are all-to-all -- every WG publishes at least
// one word (G <= n_embed) and every WG waits for all words.  A WG can only rewrite a buffer
// after consuming an all-to-all hop whose words each WG publishes after its own read of that
// buffer, so no reader can still be waiting on the old contents.  (The lm_head hop's candidates
// come only from the WGs that own lm_head rows; the next step's hop 4 orders their reuse.)
//
// Residual stream: each WG keeps the whole x[B][C] in registers, row b in wave b % 4 (lane l
// holds elements 4(l + 64j) .. +3), and recomputes the LayerNorms redundantly, so only
// projection outputs travel.  The wave that owns a row also gathers that row's exchange words
// straight into registers.  Per layer and step:
//   hop 1: x += dx2 (previous layer), LN0, QKV rows          -> q, k_new, v_new
//   hop 2: attention items (sequence, head, 64-key chunk)     -> partial (max, sum, P.V)
//   hop 3: combine partials -> y, attention-proj rows         -> dx1
//   hop 4: x += dx1, LN1, FC rows, GELU                       -> h
//   hop 5: proj2 rows                                         -> dx2
// then x += dx2, ln_f, lm_head rows -> logits + per-WG (max, index); every WG reduces the G
// candidates itself (first maximum, NanoLLM.cpp:192-201), so the next token never leaves
// the device and the next step starts without another hand-off.
//
// Weights are read from engine-owned copies laid out one output per contiguous row
// (W_qkv^T, W_fc^T, W_proj2^T; W_proj and lm_head already are).  A WG's slice of a hop is
// DMA'd into LDS (global_load_lds) before the WG waits for the hop's inputs, into one of two
// buffers used alternately, so the loads of the next hop never race the reads of this one.
// Rows sit in LDS at a padded stride (a multiple of 256 floats) so every lane of a product
// reads the same number of float4 chunks; the padding of the activation rows is zero.
//
// Every wait is bounded: after ~1 s of polling a wait sets an error flag and the WG stops
// waiting for the rest of the launch, so a protocol error ends the kernel instead of hanging.
#pragma once

#include "decode_persistent.h"

namespace fmlh {
namespace persist {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kItemKeys = kPersistItemKeys;
constexpr int kWaveKeys = kItemKeys / kWaves;  // keys per wave inside an attention item
constexpr long kSpinLimit = 1L << 21;          // polls of ~0.5-1 us each: a few seconds at most
constexpr int kScratchPerWave = 512;           // q, k_new, v_new, p (64 each), P.V partials (256)

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x & 63); }
__device__ __forceinline__ int wave_id() {
    return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
}

// ---- exchange words -------------------------------------------------------------------------

__device__ __forceinline__ uint64_t ll_load(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_put_bits(uint64_t* p, uint32_t bits, uint32_t epoch) {
    __hip_atomic_store(p, (static_cast<uint64_t>(epoch) << 32) | bits, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_put(uint64_t* p, float v, uint32_t epoch) {
    ll_put_bits(p, __float_as_uint(v), epoch);
}
__device__ __forceinline__ bool ll_current(uint64_t v, uint32_t epoch) {
    return static_cast<uint32_t>(v >> 32) == epoch;
}

// Bookkeeping of a polling loop, looked at every 256 polls so a poll costs one load: false
// once the WG gave up (a timeout here or in another wave).  `bail` is an LDS flag.
__device__ __forceinline__ bool ll_keep_polling(int& it, int* bail, unsigned* err) {
    if ((++it & 255) != 0) return true;
    if (__hip_atomic_load(bail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) return false;
    if (it > kSpinLimit) {
        __hip_atomic_store(bail, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        atomicOr(err, 1u);
        return false;
    }
    return true;
}

// Completes the words p[k] (nullptr: none) whose first loads returned v[k]: while any is stale,
// loads all stale ones again together, so each round costs one round trip.
//
// The loop is wave-uniform: it ends when no active lane of the wave has a stale word (a
// ballot), so no lane leaves it early.  With a per-lane exit, hipcc (ROCm 7.2, gfx950) gave
// the bail-flag read inside the loop the register of a word that lanes with only other words
// stale still held; those lanes then wrote the flag (0) as the word's value with a current
// epoch.  Keeping every lane in the loop keeps the words live in every lane, and a word is
// replaced through a select.
template <int N>
__device__ __forceinline__ void ll_settle_n(const uint64_t* const (&p)[N], uint64_t (&v)[N], uint32_t epoch,
                                            int* bail, unsigned* err) {
    int it = 0;
    while (true) {
        bool stale = false;
#pragma unroll
        for (int k = 0; k < N; ++k) stale |= p[k] != nullptr && !ll_current(v[k], epoch);
        if (__builtin_amdgcn_ballot_w64(stale) == 0 || !ll_keep_polling(it, bail, err)) return;
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const bool need = p[k] != nullptr && !ll_current(v[k], epoch);
            uint64_t nv = v[k];
            if (need) nv = ll_load(p[k]);
            v[k] = need ? nv : v[k];
        }
    }
}

// Issues the first loads of words p[k] (nullptr: none; its v[k] is left current).
template <int N>
__device__ __forceinline__ void ll_issue_n(const uint64_t* const (&p)[N], uint64_t (&v)[N], uint32_t epoch) {
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = p[k] != nullptr ? ll_load(p[k]) : (static_cast<uint64_t>(epoch) << 32);
}

__device__ __forceinline__ float ll_float(uint64_t v) { return __uint_as_float(static_cast<uint32_t>(v)); }

// Register rows: lane l holds elements l + 64 m (m < NE) of a row, so the 64 lanes of each
// access touch consecutive words; elements at or beyond C are 0.

// Row of C exchange words into the calling wave's registers.  All loads are issued before the
// first check; only stale words are polled again.
template <int NE>
__device__ __forceinline__ void ll_row(const uint64_t* src, int C, uint32_t epoch, float (&out)[NE],
                                       int* bail, unsigned* err) {
    const int lane = lane_id();
    const uint64_t* p[NE];
    uint64_t v[NE];
#pragma unroll
    for (int m = 0; m < NE; ++m) p[m] = lane + 64 * m < C ? src + lane + 64 * m : nullptr;
    ll_issue_n(p, v, epoch);
    ll_settle_n(p, v, epoch, bail, err);
#pragma unroll
    for (int m = 0; m < NE; ++m) out[m] = p[m] != nullptr ? ll_float(v[m]) : 0.f;
}

// Words src[0..n) into dst (LDS), all threads of the WG; loads go out in batches of 8 per
// thread before their epochs are checked.
__device__ __forceinline__ void ll_gather(const uint64_t* src, int n, uint32_t epoch, float* dst,
                                          int* bail, unsigned* err) {
    constexpr int kBatch = 8;
    for (int base = 0; base < n; base += kBatch * kThreads) {
        const uint64_t* p[kBatch];
        uint64_t v[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int i = base + k * kThreads + static_cast<int>(threadIdx.x);
            p[k] = i < n ? src + i : nullptr;
        }
        ll_issue_n(p, v, epoch);
        ll_settle_n(p, v, epoch, bail, err);
#pragma unroll
        for (int k = 0; k < kBatch; ++k)
            if (p[k] != nullptr) dst[base + k * kThreads + static_cast<int>(threadIdx.x)] = ll_float(v[k]);
    }
}

// `rows` rows of K words (row stride K in src) into LDS rows of stride KP (>= K, multiple of
// 4), zero-filling columns K..KP.
__device__ __forceinline__ void ll_gather_rows(const uint64_t* src, int rows, int K, int KP,
                                               uint32_t epoch, float* dst, int* bail, unsigned* err) {
    const int per_row = KP / 4;
    const int n = rows * per_row;
    for (int base = 0; base < n; base += 2 * kThreads) {
        const uint64_t* p[8];
        uint64_t v[8];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int s = base + u * kThreads + static_cast<int>(threadIdx.x);
            const int r = s / per_row, e = 4 * (s - r * per_row);
            const bool in = s < n && e < K;
#pragma unroll
            for (int t = 0; t < 4; ++t) p[4 * u + t] = in ? src + (size_t)r * K + e + t : nullptr;
        }
        ll_issue_n(p, v, epoch);
        ll_settle_n(p, v, epoch, bail, err);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int s = base + u * kThreads + static_cast<int>(threadIdx.x);
            if (s < n) {
                const int r = s / per_row, e = 4 * (s - r * per_row);
                float f[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) f[t] = p[4 * u + t] != nullptr ? ll_float(v[4 * u + t]) : 0.f;
                *reinterpret_cast<float4*>(dst + (size_t)r * KP + e) = make_float4(f[0], f[1], f[2], f[3]);
            }
        }
    }
}

// ---- wave reductions ------------------------------------------------------------------------

// DPP scan leaving the wave total in lane 63 only (wave_reduce without the broadcast).
template <class Op>
__device__ __forceinline__ float wave_total_last(float v, float identity, Op op) {
    v = op(v, dpp_move<0x111, 0xf>(identity, v));  // row_shr:1
    v = op(v, dpp_move<0x112, 0xf>(identity, v));  // row_shr:2
    v = op(v, dpp_move<0x114, 0xf>(identity, v));  // row_shr:4
    v = op(v, dpp_move<0x118, 0xf>(identity, v));  // row_shr:8
    v = op(v, dpp_move<0x142, 0xa>(identity, v));  // row_bcast:15
    v = op(v, dpp_move<0x143, 0xc>(identity, v));  // row_bcast:31
    return v;
}
__device__ __forceinline__ float wave_sum_last(float v) {
    return wave_total_last(v, 0.0f, [](float a, float b) { return a + b; });
}

// Sum over the 4 lanes of each quad, in every lane of the quad.
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp_move<0xb1, 0xf>(0.0f, v);  // quad_perm [1,0,3,2]
    v += dpp_move<0x4e, 0xf>(0.0f, v);  // quad_perm [2,3,0,1]
    return v;
}

// First maximum over the wave: the largest value, lowest index among equal values; entries
// with idx < 0 take no part.  Returns the index (-1 if none) and the value, wave-uniform.
__device__ __forceinline__ int wave_argmax(float v, int idx, float& best) {
    const float vv = idx >= 0 ? v : -INFINITY;
    best = wave_max(vv);
    const float cand = (idx >= 0 && vv == best) ? static_cast<float>(idx) : 3.0e38f;
    const float lowest = -wave_max(-cand);
    return lowest >= 3.0e38f ? -1 : static_cast<int>(lowest);
}

// ---- LDS staging ----------------------------------------------------------------------------

__device__ __forceinline__ void dma16(float* lds_wave_base, const float* src_lane) {
    __builtin_amdgcn_global_load_lds(static_cast<const void*>(src_lane),
                                     (__attribute__((address_space(3))) void*)(lds_wave_base), 16, 0, 0);
}

// Rows [0, nrows) of src (row length K floats) into LDS rows of stride KP (multiple of 256);
// columns K..KP are not written.  Complete after s_waitcnt vmcnt(0) + a barrier.
__device__ __forceinline__ void dma_rows(float* lds, const float* src, int nrows, int K, int KP) {
    const int lane = lane_id(), wave = wave_id();
    const int per_row = KP / 256;
    const int n = nrows * per_row;
    for (int i = wave; i < n; i += kWaves) {
        const int r = i / per_row, j = i - r * per_row;
        const int e = 256 * j + 4 * lane;
        if (e < K) dma16(lds + (size_t)r * KP + 256 * j, src + (size_t)r * K + e);
    }
}

// nfloats (multiple of 4) contiguous floats into LDS.
__device__ __forceinline__ void dma_block(float* lds, const float* src, int nfloats) {
    const int lane = lane_id(), wave = wave_id();
    const int n = (nfloats + 255) / 256;
    for (int i = wave; i < n; i += kWaves) {
        const int e = 256 * i + 4 * lane;
        if (e < nfloats) dma16(lds + 256 * i, src + e);
    }
}

__device__ __forceinline__ void wait_dma() { __builtin_amdgcn_s_waitcnt(0); }

// ---- arithmetic on register rows -----------------------------------------------------------

// Row of a global array (p may be null: zeros).  The pointer is taken as global memory
// explicitly: pointers read from the layer table would otherwise become flat accesses, which
// also count against the LDS wait counter.
template <int NE>
__device__ __forceinline__ void load_row(const float* p, int C, float (&out)[NE]) {
    const int lane = lane_id();
    const __attribute__((address_space(1))) float* gp = (const __attribute__((address_space(1))) float*)p;
#pragma unroll
    for (int m = 0; m < NE; ++m) {
        const int e = lane + 64 * m;
        out[m] = (p && e < C) ? gp[e] : 0.f;
    }
}

// LayerNormOp (MatrixBase_Functions.h:481-549) of one register row: mean = sum * (1/C),
// var = sum((x - mean)^2) * (1/C), out = (x - mean) * (1 / sqrt(var + 1e-5)) * g + b; written
// to LDS row `dst` (64 * NE floats, padding columns 0).
template <int NE>
__device__ __forceinline__ void ln_row_to_lds(const float (&x)[NE], const float (&g)[NE],
                                              const float (&bt)[NE], int C, float* dst) {
    const int lane = lane_id();
    const float inv_cols = 1.0f / static_cast<float>(C);
    float s = 0.f;
#pragma unroll
    for (int m = 0; m < NE; ++m) s += x[m];
    const float mean = wave_sum(s) * inv_cols;
    float v = 0.f;
#pragma unroll
    for (int m = 0; m < NE; ++m) {
        const float d = x[m] - mean;
        if (lane + 64 * m < C) v += d * d;
    }
    const float inv_std = 1.0f / sqrtf(wave_sum(v) * inv_cols + 1e-5f);
#pragma unroll
    for (int m = 0; m < NE; ++m) {
        const int e = lane + 64 * m;
        dst[e] = e < C ? (x[m] - mean) * inv_std * g[m] + bt[m] : 0.f;
    }
}

__device__ __forceinline__ float gelu_ref(float x) { return 0.5f * x * (1.0f + erff(x / 1.41421354f)); }

// ---- products from LDS ---------------------------------------------------------------------

__device__ __forceinline__ float dot4(float4 a, float4 b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

// out(r, b) = sum_k w[r][k] * act[b][k] for rows r < cnt of w (stride KP = 256 * NQ) and the
// BT act rows (stride KP, zero padding).  Wave v takes rows v, v + 4, ... RB at a time (rows
// past cnt repeat the last row and are dropped); every lane reads NQ float4 chunks per row.
// Lane 63 hands each result to emit(r, b, v) for b < B.
template <int BT, int NQ, int RB, class Emit>
__device__ __forceinline__ void gemv_lds(const float* w, int cnt, const float* act, int B, Emit emit) {
    constexpr int KP = 256 * NQ;
    const int lane = lane_id(), wave = wave_id();
    for (int r0 = wave; r0 < cnt; r0 += kWaves * RB) {
        float acc[RB][BT];
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int b = 0; b < BT; ++b) acc[i][b] = 0.f;
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
            float4 wv[RB];
#pragma unroll
            for (int i = 0; i < RB; ++i) {
                const int r = min(r0 + kWaves * i, cnt - 1);
                wv[i] = *reinterpret_cast<const float4*>(w + r * KP + 256 * j + 4 * lane);
            }
#pragma unroll
            for (int b = 0; b < BT; ++b) {
                const float4 av = *reinterpret_cast<const float4*>(act + b * KP + 256 * j + 4 * lane);
#pragma unroll
                for (int i = 0; i < RB; ++i) acc[i][b] += dot4(wv[i], av);
            }
        }
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int b = 0; b < BT; ++b) acc[i][b] = wave_sum_last(acc[i][b]);
        if (lane == 63) {
#pragma unroll
            for (int i = 0; i < RB; ++i)
#pragma unroll
                for (int b = 0; b < BT; ++b)
                    if (r0 + kWaves * i < cnt && b < B) emit(r0 + kWaves * i, b, acc[i][b]);
        }
    }
}

// The same for rows of runtime length KP = 256 * nq (nq even), two chunks per pass.
template <int BT, class Emit>
__device__ __forceinline__ void gemv_lds_long(const float* w, int cnt, const float* act, int B, int nq,
                                              Emit emit) {
    const int KP = 256 * nq;
    const int lane = lane_id(), wave = wave_id();
    for (int r = wave; r < cnt; r += kWaves) {
        float acc[BT];
#pragma unroll
        for (int b = 0; b < BT; ++b) acc[b] = 0.f;
        for (int j = 0; j < nq; j += 2) {
            const float4 w0 = *reinterpret_cast<const float4*>(w + r * KP + 256 * j + 4 * lane);
            const float4 w1 = *reinterpret_cast<const float4*>(w + r * KP + 256 * (j + 1) + 4 * lane);
#pragma unroll
            for (int b = 0; b < BT; ++b) {
                const float4 a0 = *reinterpret_cast<const float4*>(act + b * KP + 256 * j + 4 * lane);
                const float4 a1 = *reinterpret_cast<const float4*>(act + b * KP + 256 * (j + 1) + 4 * lane);
                acc[b] += dot4(w0, a0) + dot4(w1, a1);
            }
        }
#pragma unroll
        for (int b = 0; b < BT; ++b) acc[b] = wave_sum_last(acc[b]);
        if (lane == 63) {
#pragma unroll
            for (int b = 0; b < BT; ++b)
                if (b < B) emit(r, b, acc[b]);
        }
    }
}

// Balanced split of n outputs over G WGs.
__device__ __forceinline__ void my_range(int n, int G, int w, int& lo, int& hi) {
    lo = static_cast<int>((static_cast<long>(n) * w) / G);
    hi = static_cast<int>((static_cast<long>(n) * (w + 1)) / G);
}

// ---- the kernel -----------------------------------------------------------------------------

template <int HD, int BT, int NQC, bool GRP>
__global__ __launch_bounds__(kThreads) void decode_persistent_kernel(PersistArgs a) {
    extern __shared__ float smem_f[];
    constexpr int CP = 256 * NQC;                  // LDS stride of C-long rows
    constexpr int RPW = (BT + kWaves - 1) / kWaves;  // residual rows per wave
    constexpr int NE = CP / 64;                     // row elements per lane
    static_assert(HD == 16 || HD == 32 || HD == 64, "head_dim");
    const int C = a.C, H = a.H, L = a.L, V = a.V;
    const int G = GRP ? static_cast<int>(gridDim.x) / a.groups : static_cast<int>(gridDim.x);
    const int grp = GRP ? static_cast<int>(blockIdx.x) / G : 0;
    const int w = static_cast<int>(blockIdx.x) - grp * G;
    const int s0 = grp * a.Bg;
    const int B = GRP ? min(a.Bg, a.B - s0) : a.B;
#define hist (a.hist + (size_t)s0 * a.HS)
#define logits (a.logits + (size_t)s0 * V)
#define xq (a.q + grp * a.gw_qkv)
#define xkn (a.kn + grp * a.gw_qkv)
#define xvn (a.vn + grp * a.gw_qkv)
#define xatt (a.att + grp * a.gw_att)
#define xdx1 (a.dx1 + grp * a.gw_c)
#define xdx2 (a.dx2 + grp * a.gw_c)
#define xhb (a.hb + grp * a.gw_h4)
#define xam (a.am + grp * a.gw_am)
    const int tid = static_cast<int>(threadIdx.x), lane = lane_id(), wave = wave_id();
    const int C4 = 4 * C, H4P = a.h4p, nq4 = H4P / 256;

    float* wbuf[2] = {smem_f, smem_f + a.wcap};
    float* actA = smem_f + 2 * a.wcap;
    float* actB = actA + BT * CP;
    float* U = actB + BT * CP;  // [K/V rows |] partials | h rows | lm values, by hop
    // K/V rows of an attention item: their own region when the plan has room for it (then the
    // first item's rows are fetched at the start of the layer), else the start of U.
    float* kvr = a.kv_sep ? U + a.ufloats : U;
    float* scr = U + a.ufloats + (a.kv_sep ? 2 * kItemKeys * HD : 0);  // kScratchPerWave per wave
    float* comb = scr + kWaves * kScratchPerWave;  // kWaves x (HD + 2)
    int* bail = reinterpret_cast<int*>(comb + kWaves * (HD + 2));

    // Zero the weight buffers (their padding columns must be finite) and the activation rows
    // (padding columns and rows past B are read as 0).
    for (int e = tid; e < 2 * a.wcap + 2 * BT * CP; e += kThreads) smem_f[e] = 0.f;
    if (tid == 0) __hip_atomic_store(bail, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);

    const int hops = 5 * L + 1;
    const float scale = a.scale;

    // Optional timeline of every WG for the first kTraceSteps steps (development aid,
    // FMLH_PERSIST_TRACE): slot 0 = step start, 1 + 12 l + k = point k of layer l, then the
    // lm_head points.
    auto stamp = [&](int step, int slot) {
        if (a.trace && tid == 0 && step < kTraceSteps && slot < kTracePoints)
            a.trace[((size_t)step * kMaxPersistG + blockIdx.x) * kTracePoints + slot] = wall_clock64();
    };

    // Residual rows of this wave: b = wave + 4k.
    float x[RPW][NE];
    int tok[RPW];
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
        const int b = wave + kWaves * k;
        tok[k] = b < B ? hist[(size_t)b * a.HS + a.pos0] : 0;  // last token of the history
    }
    __syncthreads();

    for (int step = 0; step < a.n_steps; ++step) {
        const int pos = a.pos0 + step;
        const uint32_t ep0 = a.epoch_base + static_cast<uint32_t>(step) * hops;
        stamp(step, 0);
        int lo, hi;
        my_range(3 * C, G, w, lo, hi);
        dma_rows(wbuf[0], a.layers[0].wqkvT + (size_t)lo * C, hi - lo, C, CP);
        // Embedding x = tok[token] + pos_emb[pos] (Embedding x2 + AddLayer; dropout p = 0).
#pragma unroll
        for (int k = 0; k < RPW; ++k) {
            const int b = wave + kWaves * k;
            if (b < B) {
                float te[NE], pe[NE];
                load_row(a.tok + (size_t)tok[k] * C, C, te);
                load_row(a.pos_emb + (size_t)pos * C, C, pe);
#pragma unroll
                for (int m = 0; m < NE; ++m) x[k][m] = te[m] + pe[m];
            }
        }

        for (int l = 0; l < L; ++l) {
            const PersistLayer& lw = a.layers[l];
            const uint32_t ep = ep0 + 5u * l;
            float* kc = a.kc + ((size_t)l * a.Bmax + s0) * H * a.T * HD;
            float* vc = a.vc + ((size_t)l * a.Bmax + s0) * H * a.T * HD;

            // ---- hop 1: x += dx2 (layer l-1), LN0, QKV rows -> q / k_new / v_new ------------
            if (l > 0) {
                my_range(3 * C, G, w, lo, hi);
                dma_rows(wbuf[0], lw.wqkvT + (size_t)lo * C, hi - lo, C, CP);
            }
            // Cached K/V rows of this WG's first attention item, a whole layer ahead (nothing
            // in the layer writes them; the region was last read by the previous layer's
            // attention, several barriers ago).
            const int n_items = (pos / kItemKeys + 1) * B * H;
            if (a.kv_sep && w < n_items) {
                const int ch = w / (B * H), bh = w - ch * (B * H);
                const int j0 = ch * kItemKeys;
                const int nold = min(j0 + kItemKeys, pos + 1) == pos + 1 ? pos - j0 : kItemKeys;
                dma_block(kvr, kc + ((size_t)bh * a.T + j0) * HD, nold * HD);
                dma_block(kvr + kItemKeys * HD, vc + ((size_t)bh * a.T + j0) * HD, nold * HD);
            }
            {
                float g[NE], bt[NE];
                load_row(lw.ln0g, C, g);
                load_row(lw.ln0b, C, bt);
#pragma unroll
                for (int k = 0; k < RPW; ++k) {
                    const int b = wave + kWaves * k;
                    if (b < B) {
                        if (l > 0) {  // dx2 of layer l-1 was published at epoch ep0 + 5(l-1) + 5 = ep
                            float d[NE];
                            ll_row(xdx2 + (size_t)b * C, C, ep, d, bail, a.err);
#pragma unroll
                            for (int m = 0; m < NE; ++m) x[k][m] += d[m];
                        }
                        ln_row_to_lds(x[k], g, bt, C, actA + b * CP);
                    }
                }
            }
            stamp(step, 1 + 12 * l + 0);
            wait_dma();
            __syncthreads();
            stamp(step, 1 + 12 * l + 1);
            gemv_lds<BT, NQC, 3>(wbuf[0], hi - lo, actA, B, [&](int r, int b, float v) {
                const int n = lo + r;
                uint64_t* dst = n < C ? xq : (n < 2 * C ? xkn : xvn);
                ll_put(&dst[b * C + n % C], v, ep + 1);
            });
            stamp(step, 1 + 12 * l + 2);

            // ---- hop 2: attention partials (sequence, head, key chunk) ---------------------
            // Item (chunk ch, pair bh) always runs on WG (ch * B * H + bh) % G, so the WG that
            // writes a new K/V row (the owner of the chunk holding pos) is the only one that
            // reads it later in the launch, through the same CU.  Each wave takes 16 keys.
            {
                const int nch = pos / kItemKeys + 1;
                const int pairs = B * H;
                float* kbuf = kvr;
                float* vbuf = kvr + kItemKeys * HD;
                float* ws = scr + wave * kScratchPerWave;
                float* ws_q = ws;
                float* ws_k = ws + 64;
                float* ws_v = ws + 128;
                float* ws_p = ws + 192;
                float* ws_o = ws + 256;
                for (int item = w; item < nch * pairs; item += G) {
                    const int ch = item / pairs, bh = item - ch * pairs;
                    const int b = bh / H, hh = bh - b * H;
                    const int j0 = ch * kItemKeys, j1 = min(j0 + kItemKeys, pos + 1);
                    const bool has_new = j1 == pos + 1;
                    const int n = j1 - j0;
                    const int nold = has_new ? n - 1 : n;  // cached rows in the chunk
                    float* kb = kc + (size_t)bh * a.T * HD;
                    float* vb = vc + (size_t)bh * a.T * HD;
                    if (!a.kv_sep || item != w) {  // else fetched at the start of the layer
                        dma_block(kbuf, kb + (size_t)j0 * HD, nold * HD);
                        dma_block(vbuf, vb + (size_t)j0 * HD, nold * HD);
                    }
                    if (lane < HD) {
                        const size_t o = (size_t)b * C + hh * HD + lane;
                        const uint64_t* pw[3] = {&xq[o], has_new ? &xkn[o] : nullptr,
                                                 has_new ? &xvn[o] : nullptr};
                        uint64_t vw[3];
                        ll_issue_n(pw, vw, ep + 1);
                        ll_settle_n(pw, vw, ep + 1, bail, a.err);
                        ws_q[lane] = ll_float(vw[0]);
                        if (has_new) {
                            const float kv = ll_float(vw[1]);
                            const float vv = ll_float(vw[2]);
                            ws_k[lane] = kv;
                            ws_v[lane] = vv;
                            if (wave == 0) {  // the cache row of this step
                                kb[(size_t)pos * HD + lane] = kv;
                                vb[(size_t)pos * HD + lane] = vv;
                            }
                        }
                    }
                    stamp(step, 1 + 12 * l + 3);
                    wait_dma();
                    __syncthreads();
                    // scores: 4 lanes per key, HD/4 dims each, chunk order rotated per key
                    constexpr int NC = HD / 16;  // float4 chunks per lane
                    const int kk = lane >> 2, part = lane & 3;
                    const int jj = kWaveKeys * wave + kk;
                    const bool valid = jj < n;
                    const float* kr = jj < nold ? kbuf + jj * HD : (valid ? ws_k : kbuf);
                    float s = 0.f;
#pragma unroll
                    for (int t = 0; t < NC; ++t) {
                        const int c = part + 4 * ((t + kk) % NC);
                        s += dot4(*reinterpret_cast<const float4*>(ws_q + 4 * c),
                                  *reinterpret_cast<const float4*>(kr + 4 * c));
                    }
                    s = quad_sum(s) * scale;
                    const float m = wave_max(valid ? s : -INFINITY);
                    const float p = valid ? expf(s - m) : 0.f;
                    const float lsum = wave_sum(part == 0 ? p : 0.f);
                    if (part == 0) ws_p[kk] = p;
                    // P.V: lane (d4, kg) sums keys kg, kg + 4, ... over dims 4 d4 .. +3
                    const int d4 = lane & 15, kg = lane >> 4;
                    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (4 * d4 < HD) {
#pragma unroll
                        for (int i = 0; i < kWaveKeys / 4; ++i) {
                            const int k2 = kg + 4 * i, j2 = kWaveKeys * wave + k2;
                            if (j2 < n) {
                                const float* vr = j2 < nold ? vbuf + j2 * HD : ws_v;
                                const float4 vv = *reinterpret_cast<const float4*>(vr + 4 * d4);
                                const float pp = ws_p[k2];
                                o.x += pp * vv.x;
                                o.y += pp * vv.y;
                                o.z += pp * vv.z;
                                o.w += pp * vv.w;
                            }
                        }
                        *reinterpret_cast<float4*>(ws_o + kg * 64 + 4 * d4) = o;
                    }
                    float* cw = comb + wave * (HD + 2);
                    if (lane < HD) cw[2 + lane] = (ws_o[lane] + ws_o[64 + lane]) + (ws_o[128 + lane] + ws_o[192 + lane]);
                    if (lane == 0) {
                        cw[0] = m;
                        cw[1] = lsum;
                    }
                    __syncthreads();
                    if (wave == 0) {
                        // partials laid out [chunk][sequence * H + head][HD + 2]: the words of a
                        // layer are one contiguous range
                        uint64_t* slot = xatt + ((size_t)ch * pairs + bh) * (HD + 2);
                        float M = comb[0];
#pragma unroll
                        for (int v = 1; v < kWaves; ++v) M = fmaxf(M, comb[v * (HD + 2)]);
                        float wgt[kWaves];
#pragma unroll
                        for (int v = 0; v < kWaves; ++v) wgt[v] = expf(comb[v * (HD + 2)] - M);
                        if (lane < HD) {
                            float od = 0.f;
#pragma unroll
                            for (int v = 0; v < kWaves; ++v) od += wgt[v] * comb[v * (HD + 2) + 2 + lane];
                            ll_put(&slot[2 + lane], od, ep + 2);
                        }
                        if (lane == 0) {
                            float lt = 0.f;
#pragma unroll
                            for (int v = 0; v < kWaves; ++v) lt += wgt[v] * comb[v * (HD + 2) + 1];
                            ll_put(&slot[0], M, ep + 2);
                            ll_put(&slot[1], lt, ep + 2);
                        }
                    }
                }
            }
            stamp(step, 1 + 12 * l + 4);

            // ---- hop 3: combine -> y, attention proj -> dx1 -----------------------------
            {
                my_range(C, G, w, lo, hi);
                dma_rows(wbuf[1], lw.wproj + (size_t)lo * C, hi - lo, C, CP);
                const int nch = pos / kItemKeys + 1;
                const int pstride = B * H * (HD + 2);  // words per chunk
                float* part = U;
                ll_gather(xatt, nch * pstride, ep + 2, part, bail, a.err);
                __syncthreads();
                stamp(step, 1 + 12 * l + 5);
                for (int e = tid; e < B * C; e += kThreads) {
                    const int b = e / C, c = e - b * C, hh = c / HD, d = c - hh * HD;
                    const float* pp = part + (size_t)(b * H + hh) * (HD + 2);
                    float m = -INFINITY;
                    for (int ch = 0; ch < nch; ++ch) m = fmaxf(m, pp[ch * pstride]);
                    float lsum = 0.f, o = 0.f;
                    for (int ch = 0; ch < nch; ++ch) {
                        const float wgt = expf(pp[ch * pstride] - m);
                        lsum += wgt * pp[ch * pstride + 1];
                        o += wgt * pp[ch * pstride + 2 + d];
                    }
                    actB[b * CP + c] = o / lsum;
                }
                wait_dma();
                __syncthreads();
                gemv_lds<BT, NQC, 1>(wbuf[1], hi - lo, actB, B, [&](int r, int b, float v) {
                    ll_put(&xdx1[b * C + lo + r], v, ep + 3);
                });
            }
            stamp(step, 1 + 12 * l + 6);

            // ---- hop 4: x += dx1, LN1, FC rows + GELU -> h -------------------------------
            my_range(C4, G, w, lo, hi);
            dma_rows(wbuf[0], lw.wfcT + (size_t)lo * C, hi - lo, C, CP);
            {
                float g[NE], bt[NE];
                load_row(lw.ln1g, C, g);
                load_row(lw.ln1b, C, bt);
#pragma unroll
                for (int k = 0; k < RPW; ++k) {
                    const int b = wave + kWaves * k;
                    if (b < B) {
                        float d[NE];
                        ll_row(xdx1 + (size_t)b * C, C, ep + 3, d, bail, a.err);
#pragma unroll
                        for (int m = 0; m < NE; ++m) x[k][m] += d[m];
                        ln_row_to_lds(x[k], g, bt, C, actA + b * CP);
                    }
                }
            }
            stamp(step, 1 + 12 * l + 7);
            wait_dma();
            __syncthreads();
            gemv_lds<BT, NQC, 3>(wbuf[0], hi - lo, actA, B, [&](int r, int b, float v) {
                ll_put(&xhb[b * C4 + lo + r], gelu_ref(v), ep + 4);
            });
            stamp(step, 1 + 12 * l + 8);

            // ---- hop 5: proj2 rows -> dx2 -------------------------------------------------
            my_range(C, G, w, lo, hi);
            dma_rows(wbuf[1], lw.w2T + (size_t)lo * C4, hi - lo, C4, H4P);
            ll_gather_rows(xhb, B, C4, H4P, ep + 4, U, bail, a.err);
            stamp(step, 1 + 12 * l + 9);
            wait_dma();
            __syncthreads();
            gemv_lds_long<BT>(wbuf[1], hi - lo, U, B, nq4, [&](int r, int b, float v) {
                ll_put(&xdx2[b * C + lo + r], v, ep + 5);
            });
            stamp(step, 1 + 12 * l + 10);
        }

        // ---- lm_head hop: x += dx2, ln_f, logits, per-WG candidates ----------------------
        const uint32_t ep_lm = ep0 + 5u * L + 1u;
        my_range(V, G, w, lo, hi);
        const int cnt = hi - lo;
        dma_rows(wbuf[0], a.lm + (size_t)lo * C, cnt, C, CP);
        {
            float g[NE], bt[NE];
            load_row(a.lnf_g, C, g);
            load_row(a.lnf_b, C, bt);
#pragma unroll
            for (int k = 0; k < RPW; ++k) {
                const int b = wave + kWaves * k;
                if (b < B) {
                    float d[NE];
                    ll_row(xdx2 + (size_t)b * C, C, ep_lm - 1, d, bail, a.err);
#pragma unroll
                    for (int m = 0; m < NE; ++m) x[k][m] += d[m];
                    ln_row_to_lds(x[k], g, bt, C, actA + b * CP);
                }
            }
        }
        stamp(step, 1 + 12 * L + 0);
        wait_dma();
        __syncthreads();
        float* lgs = U;  // this WG's logits [row][BT]
        const bool keep = a.logit_hist && (size_t)(a.gen0 + step) < a.hist_slots;
        gemv_lds<BT, NQC, 1>(wbuf[0], cnt, actA, B, [&](int r, int b, float v) {
            const int n = lo + r;
            logits[(size_t)b * V + n] = v;
            if (keep) a.logit_hist[((size_t)(a.gen0 + step) * a.B + s0 + b) * V + n] = v;
            lgs[r * BT + b] = v;
        });
        __syncthreads();
        stamp(step, 1 + 12 * L + 1);
        // Per-WG first maximum of each row over its slice (WGs with empty slices publish nothing),
        // then every WG gathers the G candidates of its rows and reduces them: the lowest
        // index wins ties (first maximum).
        // Only WGs that own lm_head rows publish candidates (V < G leaves the others empty).
#pragma unroll
        for (int k = 0; k < RPW; ++k) {
            const int b = wave + kWaves * k;
            if (b < B && cnt > 0) {
                float bv = -INFINITY;
                int bi = -1;
                for (int i = lane; i < cnt; i += 64) {
                    const float v = lgs[i * BT + b];
                    if (bi < 0 || v > bv) { bv = v; bi = lo + i; }
                }
                float best;
                const int idx = wave_argmax(bv, bi, best);
                if (lane == 0) {
                    ll_put(&xam[((size_t)w * B + b) * 2], best, ep_lm);
                    ll_put_bits(&xam[((size_t)w * B + b) * 2 + 1], static_cast<uint32_t>(idx), ep_lm);
                }
            }
        }
        stamp(step, 1 + 12 * L + 2);
#pragma unroll
        for (int k = 0; k < RPW; ++k) {
            const int b = wave + kWaves * k;
            if (b < B) {
                float bv = -INFINITY;
                int bi = -1;
                constexpr int NU = kMaxPersistG / 64;
                const uint64_t* pa[2 * NU];
                uint64_t va[2 * NU];
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    const int g = lane + 64 * u;
                    // WG g owns lm_head rows [V g / G, V (g + 1) / G) (my_range)
                    const bool owns = g < G && (static_cast<long>(V) * (g + 1)) / G > (static_cast<long>(V) * g) / G;
                    pa[2 * u] = owns ? &xam[((size_t)g * B + b) * 2] : nullptr;
                    pa[2 * u + 1] = owns ? &xam[((size_t)g * B + b) * 2 + 1] : nullptr;
                }
                ll_issue_n(pa, va, ep_lm);
                ll_settle_n(pa, va, ep_lm, bail, a.err);
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    if (pa[2 * u] != nullptr) {
                        const float v = ll_float(va[2 * u]);
                        const int idx = static_cast<int>(static_cast<uint32_t>(va[2 * u + 1]));
                        if (idx >= 0 && (bi < 0 || v > bv || (v == bv && idx < bi))) { bv = v; bi = idx; }
                    }
                }
                float best;
                const int t = wave_argmax(bv, bi, best);
                tok[k] = t < 0 ? 0 : t;
                if (w == 0 && lane == 0) hist[(size_t)b * a.HS + pos + 1] = tok[k];
            }
        }
        stamp(step, 1 + 12 * L + 3);
    }
    if (blockIdx.x == 0 && tid == 0) {
        a.st_pos[0] = a.pos0 + a.n_steps;
        a.st_pos[1] = a.gen0 + a.n_steps;
    }
}

#undef hist
#undef logits
#undef xq
#undef xkn
#undef xvn
#undef xatt
#undef xdx1
#undef xdx2
#undef xhb
#undef xam

template <int HD, int BT, int NQC, bool GRP = false>
int launch(const PersistArgs& a, const PersistPlan& p, hipStream_t s) {
    auto kern = decode_persistent_kernel<HD, BT, NQC, GRP>;
    FMLH_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(p.smem)));
    if (inject_fault(kFaultLaunch))
        return set_error(FMLH_E_HIP, "decode_persistent_kernel: launch failed (injected by FMLH_FAULT)");
    PersistArgs args = a;
    void* params[] = {&args};
    const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kern), dim3(p.G * p.groups),
                                                    dim3(kThreads), params, static_cast<unsigned>(p.smem), s);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        set_error(FMLH_E_HIP, "persistent decode: cooperative launch refused (%s)", hipGetErrorString(e));
        return kPersistRefused;
    }
    return FMLH_OK;
}

template <int HD>
int launch_hd(const PersistArgs& a, const PersistPlan& p, hipStream_t s) {
    if (p.groups > 1)
        return p.nqc == 1 ? launch<HD, 8, 1, true>(a, p, s) : launch<HD, 8, 2, true>(a, p, s);
    const int sel = p.bt * 10 + p.nqc;
    switch (sel) {
        case 11: return launch<HD, 1, 1>(a, p, s);
        case 12: return launch<HD, 1, 2>(a, p, s);
        case 21: return launch<HD, 2, 1>(a, p, s);
        case 22: return launch<HD, 2, 2>(a, p, s);
        case 41: return launch<HD, 4, 1>(a, p, s);
        case 42: return launch<HD, 4, 2>(a, p, s);
        case 81: return launch<HD, 8, 1>(a, p, s);
        case 82: return launch<HD, 8, 2>(a, p, s);
        default: return set_error(FMLH_E_INVALID, "persistent decode: no kernel for batch tile %d, %d-chunk rows",
                                  p.bt, p.nqc);
    }
}

}  // namespace persist
}  // namespace fmlh
