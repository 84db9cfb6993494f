// Grouped persistent decode kernel: many greedy decode steps of up to kMaxGroups groups of up
// to kGroupBatch sequences in one cooperative launch.  Included by decode_grouped.hip.
//
// Why a second persistent kernel: with 8 sequences per group the products are 8-column matrix
// products, not dot products.  The batch-1 kernel (decode_persistent_kernel.h) reduces every
// (row, sequence) dot product across a wave with DPP steps, which at 8 sequences costs more than
// the exchange itself; here the products run on the matrix cores (v_mfma_f32_16x16x4f32: 16
// weight rows x 16 batch columns, 8 of them used), which accumulate over k without any
// cross-lane reduction.
//
// Layout of the work.  Group k runs on the workgroups (WGs) b with b % groups == k: one WG per
// CU, and with the round-robin dispatch of WGs over the 8 XCDs each group of an 8-group launch
// sits on one XCD (the exchange words are device-scope either way; a group that stays on one
// XCD measured the cheapest hand-offs).  Groups never talk to each other.  Within a group the
// hops of a step are those of the batch-1 kernel, exchanged through the same {payload, epoch}
// words (decode_persistent_kernel.h describes the protocol and why single buffers are safe: it
// needs every WG to publish in each all-to-all hop, hence G <= C):
//   hop 1: x += dx2 (previous layer), LN0, QKV rows                -> q, k_new, v_new
//   hop 2: attention, one item per (sequence, head) over all keys   -> y (normalised)
//   hop 3: gather y, attention-proj rows                             -> dx1
//   hop 4: x += dx1, LN1, FC rows + GELU                             -> h
//   hop 5: gather h, proj2 rows                                      -> dx2
// then x += dx2, ln_f, lm_head rows -> logits + per-WG first maximum per sequence, and every WG
// reduces the candidates itself.
//
// Products.  A WG's weight rows of a hop are loaded from global memory straight into the MFMA
// A-operand registers before the WG waits for the hop's inputs (no LDS staging): wave v takes
// the 16-wide k blocks j = v, v + 4, ..., and lane (r = lane % 16, g = lane / 16) holds
// W[row0 + 16 t + r][16 j + 4 g .. + 3] of tile t, one float4 feeding four MFMA steps.  The
// summation order over k is thereby permuted identically for both operands.  The activations
// (LayerNorm outputs, y, h) sit in LDS, row b holding float4 chunk q at position q ^ (b & 7)
// (conflict-free reads of the 8 rows at one chunk).  Each wave's partial 16 x 16 tiles are
// added across the four waves in LDS in wave order, then emitted.
//
// Attention.  Item (sequence, head) covers keys 0..pos: the four waves take 16-key groups
// v, v + 4, ... (at most 4 each for block_size <= 256), load all their K and V rows into
// registers before waiting for q (the cached rows do not depend on this step), run an online
// softmax over their groups, and combine in LDS.  The key at pos comes from the exchange words
// (k_new, v_new); wave 0 also writes it to the cache.  Item (b, h) always runs on the same WG,
// so that WG is the only reader of the rows it writes.
#pragma once

#include "decode_grouped.h"
#include "decode_persistent_kernel.h"

namespace fmlh {
namespace grouped {

using persist::kThreads;
using persist::kWaves;
using persist::ll_float;
using persist::ll_issue_n;
using persist::ll_put;
using persist::ll_put_bits;
using persist::ll_row;
using persist::ll_settle_n;
using persist::my_range;
using persist::quad_sum;
using persist::wave_argmax;

// Thread, lane and wave ids read through an empty asm statement at each use.  The compiler
// then computes per-lane LDS and exchange addresses where they are used instead of hoisting
// them out of the layer loop, where they would hold registers that the weight tiles need (and
// spill to scratch, whose reloads wait behind the weight loads in flight).
__device__ __forceinline__ int thread_id() {
    int t = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(t));
    return t;
}
__device__ __forceinline__ int lane_id() { return thread_id() & 63; }
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(thread_id() >> 6); }

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) float gfloat;
typedef const __attribute__((address_space(1))) floatx4 gfloatx4;

// 16 bytes of global memory (p 16-byte aligned).
__device__ __forceinline__ floatx4 gload4(gfloat* p) { return *(gfloatx4*)p; }

constexpr int kTile = 16;
constexpr int kKeyGroup = 16;        // keys per wave pass of an attention item
constexpr int kMaxGroupsPerWave = kGroupedMaxT / kKeyGroup / kWaves;  // 4

// Work-group barrier for LDS data: waits for this wave's LDS accesses, not for its global loads.
// __syncthreads() also waits for every outstanding global load (its release fence), which
// would turn the weight loads issued for the next hop into a stall at the next barrier.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
#pragma clang diagnostic pop

// Keeps the loads issued above it from being moved below it: the compiler would otherwise sink
// early (prefetch) loads to their first use, exposing their latency there.
__device__ __forceinline__ void issue_here() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ int swz(int q, int b) { return q ^ (b & 7); }

// Element e of row b (row length K) of a swizzled LDS operand.
__device__ __forceinline__ int swz_at(int b, int e, int K) { return b * K + (swz(e >> 2, b) << 2) + (e & 3); }

// LayerNormOp (MatrixBase_Functions.h:481-549) of a register row (lane l holds elements
// l + 64 m), written to row b of the swizzled operand: mean = sum * (1/C), two-pass variance,
// out = (x - mean) * (1 / sqrt(var + 1e-5)) * g + beta.
template <int NE>
__device__ __forceinline__ void ln_row_swz(const float (&x)[NE], const float (&gm)[NE], const float (&bt)[NE],
                                           float* act, int b) {
    constexpr int C = 64 * NE;
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
        v += d * d;
    }
    const float inv_std = 1.0f / sqrtf(wave_sum(v) * inv_cols + 1e-5f);
#pragma unroll
    for (int m = 0; m < NE; ++m) act[swz_at(b, lane + 64 * m, C)] = (x[m] - mean) * inv_std * gm[m] + bt[m];
}

// Weight rows [row0, row0 + n) (n >= 1, row length K = 64 NJ) into the A-operand registers of
// T tiles; rows past n repeat the last row (their results are dropped).
template <int T, int NJ>
__device__ __forceinline__ void load_w(floatx4 (&wr)[T][NJ], const float* W, int row0, int n) {
    constexpr int K = 64 * NJ;
    const int lane = lane_id(), wave = wave_id(), r = lane & 15, g = lane >> 4;
    gfloat* gw = (gfloat*)W;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int row = row0 + min(kTile * t + r, n - 1);
#pragma unroll
        for (int jj = 0; jj < NJ; ++jj) {
            const int k = 16 * (wave + 4 * jj) + 4 * g;
            wr[t][jj] = gload4(gw + (size_t)row * K + k);
        }
    }
}

// acc[t] (+)= W_tile_t * act^T over this wave's k blocks jj in [J0, J1) (zeroed first when
// `init`); act rows b >= Bl read as zero.  The k blocks jj < NJ/2 cover the first half of K.
template <int T, int NJ, int J0, int J1>
__device__ __forceinline__ void mfma_rows_part(const floatx4 (&wr)[T][NJ], const float* act, int Bl, floatx4 (&acc)[T],
                                               bool init) {
    constexpr int K = 64 * NJ;
    const int lane = lane_id(), wave = wave_id(), r = lane & 15, g = lane >> 4;
    if (init) {
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int jj = J0; jj < J1; ++jj) {
        const int q = 4 * (wave + 4 * jj) + g;
        float4 xv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < Bl) xv = *reinterpret_cast<const float4*>(act + r * K + (swz(q, r) << 2));
#pragma unroll
        for (int t = 0; t < T; ++t) {
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(wr[t][jj][0], xv.x, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(wr[t][jj][1], xv.y, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(wr[t][jj][2], xv.z, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(wr[t][jj][3], xv.w, acc[t], 0, 0, 0);
        }
    }
}

template <int T, int NJ>
__device__ __forceinline__ void mfma_rows(const floatx4 (&wr)[T][NJ], const float* act, int Bl, floatx4 (&acc)[T]) {
    mfma_rows_part<T, NJ, 0, NJ>(wr, act, Bl, acc, true);
}

// Raw buffer resource word 3 (32-bit data format): loads past the record count read as zero.
constexpr int kRawBufferFlags = 0x00020000;
__device__ __forceinline__ floatx4 bload4(__amdgpu_buffer_rsrc_t r, int e) {
    return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, e * 4, 0, 0));
}

// LDS floats before region U: attention scratch, lm values, bail flag (rounded to 16 B).
constexpr int grouped_scratch_floats(int hd) {
    return (6 * hd + 4 * 256 + 4 * 64 + 8 * (hd + 2) + kTile * 8 + 4 + 3) / 4 * 4;
}

// LDS row length of a WG's own h slice (16 tq floats, rounded up to whole 8-chunk swizzle
// blocks; the padding stays zero).
constexpr int h_row(int tq) { return (16 * tq + 31) / 32 * 32; }

// The proj2 partial of this WG's FC rows: acc[i] = W2T[c][f0 + k] h[b][k] summed over the
// WG's nf FC rows k, for the 16-row tiles t = wave + 4 i of all C outputs (NT = C / 64 tiles
// per wave, TQ k blocks of 16).  Waves split the output tiles, so no cross-wave sum is needed.
template <int NT, int TQ>
__device__ __forceinline__ void load_w2_part(floatx4 (&w2)[NT][TQ], const float* W2T, int C4, int f0, int nf) {
    const int lane = lane_id(), wave = wave_id(), r = lane & 15, g = lane >> 4;
    gfloat* gw = (gfloat*)W2T;
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int c = kTile * (wave + 4 * i) + r;
#pragma unroll
        for (int jj = 0; jj < TQ; ++jj) {
            const int k = kTile * jj + 4 * g;
            w2[i][jj] = k < nf ? gload4(gw + (size_t)c * C4 + f0 + k) : floatx4{0.f, 0.f, 0.f, 0.f};
        }
    }
}

template <int NT, int TQ>
__device__ __forceinline__ void mfma_w2_part(const floatx4 (&w2)[NT][TQ], const float* hl, int Bl, floatx4 (&acc)[NT]) {
    constexpr int KR = h_row(TQ);
    const int lane = lane_id(), r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int i = 0; i < NT; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jj = 0; jj < TQ; ++jj) {
        const int q = 4 * jj + g;
        float4 xv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < Bl) xv = *reinterpret_cast<const float4*>(hl + r * KR + (q ^ (r & 7)) * 4);
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(w2[i][jj][0], xv.x, acc[i], 0, 0, 0);
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(w2[i][jj][1], xv.y, acc[i], 0, 0, 0);
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(w2[i][jj][2], xv.z, acc[i], 0, 0, 0);
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(w2[i][jj][3], xv.w, acc[i], 0, 0, 0);
        }
    }
}

// Adds the four waves' partial tiles (wave order) and hands out(row, b) = value to emit for rows
// < n and sequences < Bl.  Thread t takes sequence t / 16 and row t % 16 of each tile, so that
// consecutive threads emit consecutive rows of one sequence (contiguous exchange words).
// red: kWaves * T * 256 floats.  Ends with a barrier (red is reused).
template <int T, class Emit>
__device__ __forceinline__ void reduce_emit(const floatx4 (&acc)[T], float* red, int n, int Bl, Emit emit) {
    const int lane = lane_id(), wave = wave_id(), tid = thread_id();
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[((wave * T + t) << 8) + (i << 6) + lane] = acc[t][i];
    lds_barrier();
    // element 64 i + l of a tile holds D[4 (l / 16) + i][l % 16]
    const int b = tid >> 4, rr = tid & 15;
    const int e = ((rr & 3) << 6) + ((rr >> 2) << 4) + b;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        const int row = kTile * t + rr;
        if (row < n && b < Bl) {
            float s = red[((0 * T + t) << 8) + e];
#pragma unroll
            for (int v = 1; v < kWaves; ++v) s += red[((v * T + t) << 8) + e];
            emit(row, b, s);
        }
    }
    lds_barrier();
}

// Columns [col0, col0 + LEN) of Bl rows of exchange words (row stride STRIDE in src) into the
// swizzled operand (row length STRIDE).  Thread t takes row t / 32 and columns t % 32 + 32 k:
// its LEN / 32 words are in flight at once, at constant offsets from one address, so a word
// costs two registers and the loops unroll fully.
template <int LEN, int STRIDE>
__device__ __forceinline__ void gather_swz(const uint64_t* src, int Bl, int col0, uint32_t epoch, float* act,
                                           int* bail, unsigned* err) {
    static_assert(LEN % 32 == 0 && kThreads == 32 * kGroupBatch, "one row per 32 threads");
    constexpr int NW = LEN / 32;
    const int tid = thread_id(), b = tid >> 5, c = tid & 31;
    if (b >= Bl) return;
    const uint64_t* p = src + (size_t)b * STRIDE + col0 + c;
    uint64_t v[NW];
#pragma unroll
    for (int k = 0; k < NW; ++k) v[k] = persist::ll_load(p + 32 * k);
    int it = 0;
    while (true) {  // wave-uniform, as persist::ll_settle_n (no lane leaves early)
        bool stale = false;
#pragma unroll
        for (int k = 0; k < NW; ++k) stale |= !persist::ll_current(v[k], epoch);
        if (__builtin_amdgcn_ballot_w64(stale) == 0 || !persist::ll_keep_polling(it, bail, err)) break;
#pragma unroll
        for (int k = 0; k < NW; ++k) {
            const bool need = !persist::ll_current(v[k], epoch);
            uint64_t nv = v[k];
            if (need) nv = persist::ll_load(p + 32 * k);
            v[k] = need ? nv : v[k];
        }
    }
#pragma unroll
    for (int k = 0; k < NW; ++k) act[swz_at(b, col0 + c + 32 * k, STRIDE)] = ll_float(v[k]);
}

template <int NE>
__device__ __forceinline__ void load_vec(const float* p, float (&out)[NE]) {
    persist::load_row(p, 64 * NE, out);
}

template <int HD, int NE, int TQ>
__global__ __launch_bounds__(kThreads) void decode_grouped_kernel(GroupedArgs a) {
    constexpr int C = 64 * NE, C4 = 4 * C, H = C / HD;
    constexpr int NCK = HD / 16;  // float4 of a key row per lane (4 lanes per key)
    static_assert(HD == 16 || HD == 32 || HD == 64, "head_dim");
    static_assert(kGroupBatch == 8, "two residual rows per wave");
    extern __shared__ float smem_f[];
    const int L = a.L, V = a.V;
    const int groups = a.groups;
    const int grp = static_cast<int>(blockIdx.x) % groups;
    const int w = static_cast<int>(blockIdx.x) / groups;
    const int G = static_cast<int>(gridDim.x) / groups;
    const int s0 = grp * a.Bg;
    const int Bl = min(a.Bg, a.B - s0);
    int32_t* hist = a.hist + (size_t)s0 * a.HS;
    float* logits = a.logits + (size_t)s0 * V;
    uint64_t* xq = a.q + grp * a.gw_c;
    uint64_t* xkn = xq + a.qkv_stride;
    uint64_t* xvn = xq + 2 * a.qkv_stride;
    uint64_t* xy = a.y + grp * a.gw_c;
    uint64_t* xdx1 = a.dx1 + grp * a.gw_c;
    uint64_t* xdx2 = a.dx2 + grp * a.gw_c;
    uint64_t* xpart = a.part + (size_t)grp * G * kGroupBatch * C;  // [wg][8][C] of this group
    uint64_t* xam = a.am + grp * a.gw_am;
    const int tid = thread_id(), lane = lane_id(), wave = wave_id();

    // LDS: attention scratch (q, k_new, v_new of two items, per-wave P.V partials, per-wave
    // (max, sum, o)) | lm values | bail | region U.  U holds, by hop: act (8 x C, swizzled), hl
    // (this WG's h slice, 8 x h_row(TQ), swizzled), pg (proj2 partials of this WG's outputs,
    // 8 x C), red (4 x TQ x 256); during hop 2 it holds instead the cached K and V rows of a
    // WG's second attention item (2 x T x HD).
    constexpr int KR = h_row(TQ);
    float* qs = smem_f;                     // [2][HD]
    float* kns = qs + 2 * HD;               // [2][HD]
    float* vns = kns + 2 * HD;              // [2][HD]
    float* ows = vns + 2 * HD;                  // kWaves x 256: P.V partials (key lane groups)
    float* pls = ows + kWaves * 256;            // kWaves x 64: softmax numerators
    float* comb = pls + kWaves * 64;            // [item of the pair][wave][max, sum, o (HD)]
    float* lgs = comb + 2 * kWaves * (HD + 2);  // lm values [row][b], 16 x 8
    int* bail = reinterpret_cast<int*>(lgs + kTile * kGroupBatch);
    float* act = smem_f + grouped_scratch_floats(HD);
    float* hl = act + kGroupBatch * C;
    float* pg = hl + kGroupBatch * KR;
    float* red = pg + kGroupBatch * C;
    float* kvl = act;  // [K: T x HD][V: T x HD], hop 2 only

    for (int e = tid; e < kGroupBatch * (C + KR); e += kThreads) act[e] = 0.f;
    if (tid == 0) __hip_atomic_store(bail, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);

    const int hops = 5 * L + 1;
    // Timeline: slot 0 = step start, 1 + 16 l + k = point k of layer l, 1 + 16 L + k = lm points.
    auto stamp = [&](int step, int slot) {
        if (a.trace && tid == 0 && step < kGroupedTraceSteps && slot < kGroupedTracePoints &&
            blockIdx.x < kGroupedTraceWGs)
            a.trace[((size_t)step * kGroupedTraceWGs + blockIdx.x) * kGroupedTracePoints + slot] = wall_clock64();
    };
    float x[2][NE];
    int tok[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int b = wave + kWaves * k;
        tok[k] = b < Bl ? hist[(size_t)b * a.HS + a.pos0] : 0;
    }
    // This WG's rows of each product (the same in every layer).
    int lo_q, hi_q, lo_p, hi_p, lo_f, hi_f, lo_l, hi_l;
    my_range(3 * C, G, w, lo_q, hi_q);
    my_range(C, G, w, lo_p, hi_p);  // attention proj and proj2
    my_range(C4, G, w, lo_f, hi_f);
    my_range(V, G, w, lo_l, hi_l);
    const int cnt = hi_l - lo_l;
    // Weight registers.  Each hop's weights are requested right after the previous hop has
    // published its outputs: they then stream in while the WG waits for the next inputs, and no
    // publish queues behind them (a CU's memory requests are served in order).
    constexpr int NT2 = C / 64;  // proj2 output tiles per wave
    floatx4 wq[TQ][NE], wp[1][NE], wf[TQ][NE], w2[NT2][TQ], wl[1][NE];
    load_w<TQ, NE>(wq, a.layers[0].wqkvT, lo_q, hi_q - lo_q); issue_here();
    lds_barrier();

    for (int step = 0; step < a.n_steps; ++step) {
        const int pos = a.pos0 + step;
        const uint32_t ep0 = a.epoch_base + static_cast<uint32_t>(step) * hops;
        stamp(step, 0);
        // Embedding x = tok[token] + pos_emb[pos] (Embedding x2 + AddLayer; dropout p = 0).
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int b = wave + kWaves * k;
            if (b < Bl) {
                float te[NE], pe[NE];
                load_vec(a.tok + (size_t)tok[k] * C, te);
                load_vec(a.pos_emb + (size_t)pos * C, pe);
#pragma unroll
                for (int m = 0; m < NE; ++m) x[k][m] = te[m] + pe[m];
            }
        }

        for (int l = 0; l < L; ++l) {
            const int tid = thread_id(), lane = lane_id(), wave = wave_id();  // not hoisted (see thread_id)
            const PersistLayer& lw = a.layers[l];
            const uint32_t ep = ep0 + 5u * l;
            float* kc = a.kc + ((size_t)l * a.Bmax + s0) * H * a.T * HD;
            float* vc = a.vc + ((size_t)l * a.Bmax + s0) * H * a.T * HD;

            // ---- hop 1: x += dx2 (layer l-1), LN0, QKV rows -> q / k_new / v_new -----------
            {
                float gm[NE], bt[NE];
                load_vec(lw.ln0g, gm);
                load_vec(lw.ln0b, bt);
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int b = wave + kWaves * k;
                    if (b < Bl) {
                        if (l > 0) {  // dx2 of layer l-1, published at epoch ep0 + 5 (l - 1) + 5 = ep
                            float d[NE];
                            ll_row(xdx2 + (size_t)b * C, C, ep, d, bail, a.err);
#pragma unroll
                            for (int m = 0; m < NE; ++m) x[k][m] += d[m];
                        }
                        ln_row_swz(x[k], gm, bt, act, b);
                    }
                }
                lds_barrier();
                stamp(step, 1 + 16 * l + 0);
                floatx4 acc[TQ];
                mfma_rows(wq, act, Bl, acc);
                stamp(step, 1 + 16 * l + 1);
                reduce_emit<TQ>(acc, red, hi_q - lo_q, Bl, [&](int r, int b, float v) {
                    const int n = lo_q + r, part = n / C;  // 0 q, 1 k_new, 2 v_new
                    ll_put(&xq[part * a.qkv_stride + b * C + (n - part * C)], v, ep + 1);
                });
                load_w<1, NE>(wp, lw.wproj, lo_p, hi_p - lo_p); issue_here();
            }

            // ---- hop 2: attention items (sequence, head) over keys 0..pos -> y -------------
            // A WG takes items w, w + G, ... in pairs: the cached K/V rows of the first item of a
            // pair are loaded into registers and those of the second are copied into LDS (region
            // U), all before the q / k_new / v_new words of both are polled, so the second item
            // costs no second load round trip.  Each wave scores its 16-key groups v, v + 4, ...
            // of both items with one softmax pass per item and leaves (max, sum, P.V) in LDS;
            // after one barrier waves 0 and 1 combine the four waves of item 0 and item 1.
            {
                const int nkeys = pos + 1, n_items = Bl * H;
                const int kk = lane >> 2, part = lane & 3;  // score lanes: key kk, dims part*HD/4..
                const int d4 = lane & 15, kq = lane >> 4;   // P.V lanes: dims 4 d4.., keys kq + 4 i
                const int gp = pos >> 4;                    // the 16-key group holding key pos
                float* pl = pls + wave * 64;  // this wave's p, [group][4 (k % 4) + k / 4]
                float* ow = ows + wave * 256;
                for (int i0 = w; i0 < n_items; i0 += 2 * G) {
                    const int i1 = i0 + G;
                    const bool two = i1 < n_items;  // WG-uniform
                    float* kb[2];
                    float* vb[2];
                    int ib[2], ih[2];
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const int it = u == 0 ? i0 : (two ? i1 : i0);
                        ib[u] = it / H;
                        ih[u] = it - ib[u] * H;
                        kb[u] = kc + ((size_t)ib[u] * H + ih[u]) * a.T * HD;
                        vb[u] = vc + ((size_t)ib[u] * H + ih[u]) * a.T * HD;
                    }
                    floatx4 kr[kMaxGroupsPerWave][NCK];
                    floatx4 vr[kMaxGroupsPerWave][4];
                    // The rows of this wave's groups that hold a key 0..pos (whole groups; T is a
                    // multiple of 16, so they exist).  Rows pos.. of the first item read as zero
                    // (bounded buffer loads); for the second item V rows pos.. are zeroed in LDS
                    // and K rows pos.. only enter masked scores.  Key pos is added on its own.
                    auto rows_from = [&](auto kload, auto vload) {
#pragma unroll
                        for (int gi = 0; gi < kMaxGroupsPerWave; ++gi) {
                            const int base = kKeyGroup * (wave + kWaves * gi);
                            if (base < nkeys) {  // wave-uniform
#pragma unroll
                                for (int c = 0; c < NCK; ++c) kr[gi][c] = kload((base + kk) * HD + part * (HD / 4) + 4 * c);
#pragma unroll
                                for (int i = 0; i < 4; ++i) vr[gi][i] = vload((base + kq + 4 * i) * HD + 4 * (d4 % (HD / 4)));
                            }
                        }
                    };
                    {
                        const int bytes = pos * HD * static_cast<int>(sizeof(float));
                        const auto rk = __builtin_amdgcn_make_buffer_rsrc(kb[0], 0, bytes, kRawBufferFlags);
                        const auto rv = __builtin_amdgcn_make_buffer_rsrc(vb[0], 0, bytes, kRawBufferFlags);
                        rows_from([&](int e) { return bload4(rk, e); }, [&](int e) { return bload4(rv, e); });
                    }
                    if (two) {  // second item: cached rows 0..pos-1 into LDS, 1 KB per wave copy
                        const int nfl = pos * HD;
                        for (int c0 = 256 * wave; c0 < nfl; c0 += 256 * kWaves) {
                            if (c0 + 4 * lane < nfl) {
                                copy16_to_lds(kvl + c0, kb[1] + c0 + 4 * lane);
                                copy16_to_lds(kvl + a.T * HD + c0, vb[1] + c0 + 4 * lane);
                            }
                        }
                        for (int e = nfl + tid; e < kKeyGroup * (gp + 1) * HD; e += kThreads) kvl[a.T * HD + e] = 0.f;
                    }
                    issue_here();  // the cached rows are requested before q is polled
                    if (wave < (two ? 2 : 1) && lane < HD) {
                        const size_t o = (size_t)ib[wave] * C + ih[wave] * HD + lane;
                        const uint64_t* pw[3] = {&xq[o], &xkn[o], &xvn[o]};
                        uint64_t vw[3];
                        ll_issue_n(pw, vw, ep + 1);
                        ll_settle_n(pw, vw, ep + 1, bail, a.err);
                        const float kn = ll_float(vw[1]), vn = ll_float(vw[2]);
                        qs[wave * HD + lane] = ll_float(vw[0]);
                        kns[wave * HD + lane] = kn;
                        vns[wave * HD + lane] = vn;
                        kb[wave][(size_t)pos * HD + lane] = kn;  // the cache row of this step
                        vb[wave][(size_t)pos * HD + lane] = vn;
                    }
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the LDS copies have landed
                    lds_barrier();
                    stamp(step, 1 + 16 * l + 2);
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        if (u == 1) {
                            if (!two) break;
                            rows_from([&](int e) { return *reinterpret_cast<const floatx4*>(kvl + e); },
                                      [&](int e) { return *reinterpret_cast<const floatx4*>(kvl + a.T * HD + e); });
                        }
                        floatx4 qv[NCK];
                        float s_pos = 0.f;  // score of key pos (k_new), in every lane
#pragma unroll
                        for (int c = 0; c < NCK; ++c) {
                            qv[c] = *reinterpret_cast<const floatx4*>(qs + u * HD + part * (HD / 4) + 4 * c);
                            const floatx4 t = *reinterpret_cast<const floatx4*>(kns + u * HD + part * (HD / 4) + 4 * c);
                            s_pos += qv[c][0] * t[0] + qv[c][1] * t[1] + qv[c][2] * t[2] + qv[c][3] * t[3];
                        }
                        s_pos = quad_sum(s_pos) * a.scale;
                        float sc[kMaxGroupsPerWave];
                        float mx = -INFINITY;
#pragma unroll
                        for (int gi = 0; gi < kMaxGroupsPerWave; ++gi) {
                            const int base = kKeyGroup * (wave + kWaves * gi);
                            sc[gi] = -INFINITY;
                            if (base < nkeys) {  // wave-uniform
                                float sv = 0.f;
#pragma unroll
                                for (int c = 0; c < NCK; ++c)
                                    sv += qv[c][0] * kr[gi][c][0] + qv[c][1] * kr[gi][c][1] + qv[c][2] * kr[gi][c][2] +
                                          qv[c][3] * kr[gi][c][3];
                                const float t = quad_sum(sv) * a.scale;
                                sc[gi] = base + kk == pos ? s_pos : t;
                                if (base + kk < nkeys) mx = fmaxf(mx, sc[gi]);
                            }
                        }
                        const float m = wave_max(mx);  // -inf only if this wave has no key
                        float psum = 0.f;
#pragma unroll
                        for (int gi = 0; gi < kMaxGroupsPerWave; ++gi) {
                            const int j = kKeyGroup * (wave + kWaves * gi) + kk;
                            const float pv = j < nkeys ? expf(sc[gi] - m) : 0.f;
                            if (part == 0) {
                                psum += pv;
                                pl[16 * gi + 4 * (kk & 3) + (kk >> 2)] = pv;
                            }
                        }
                        const float lsum = wave_sum(psum);
                        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // p of this wave is in LDS
                        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                        for (int gi = 0; gi < kMaxGroupsPerWave; ++gi) {
                            if (kKeyGroup * (wave + kWaves * gi) < nkeys) {  // wave-uniform
                                const floatx4 pp = *reinterpret_cast<const floatx4*>(pl + 16 * gi + 4 * kq);
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
                            const float pm = wave == (gp & 3) && kq == (pos & 3) ? expf(s_pos - m) : 0.f;
                            const floatx4 t = *reinterpret_cast<const floatx4*>(vns + u * HD + 4 * (d4 % (HD / 4)));
                            o.x += pm * t[0];
                            o.y += pm * t[1];
                            o.z += pm * t[2];
                            o.w += pm * t[3];
                        }
                        // sum the four key lane groups of this wave, then leave (max, sum, o)
                        *reinterpret_cast<float4*>(ow + kq * 64 + 4 * d4) = o;
                        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                        float* cw = comb + (u * kWaves + wave) * (HD + 2);
                        if (lane < HD) cw[2 + lane] = (ow[lane] + ow[64 + lane]) + (ow[128 + lane] + ow[192 + lane]);
                        if (lane == 0) {
                            cw[0] = m;
                            cw[1] = lsum;
                        }
                        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // ow is reused by item 1
                    }
                    lds_barrier();
                    stamp(step, 1 + 16 * l + 3);
                    if (wave < (two ? 2 : 1) && lane < HD) {
                        const float* cu = comb + wave * kWaves * (HD + 2);
                        float M = cu[0];
#pragma unroll
                        for (int v = 1; v < kWaves; ++v) M = fmaxf(M, cu[v * (HD + 2)]);
                        float od = 0.f, lt = 0.f;
#pragma unroll
                        for (int v = 0; v < kWaves; ++v) {
                            const float wv = cu[v * (HD + 2)] == -INFINITY ? 0.f : expf(cu[v * (HD + 2)] - M);
                            od += wv * cu[v * (HD + 2) + 2 + lane];
                            lt += wv * cu[v * (HD + 2) + 1];
                        }
                        ll_put(&xy[(size_t)ib[wave] * C + ih[wave] * HD + lane], od / lt, ep + 2);
                    }
                }
            }

            stamp(step, 1 + 16 * l + 4);
            load_w<TQ, NE>(wf, lw.wfcT, lo_f, hi_f - lo_f); issue_here();
            // ---- hop 3: gather y, attention proj -> dx1 ------------------------------------
            {
                gather_swz<C, C>(xy, Bl, 0, ep + 2, act, bail, a.err);
                lds_barrier();
                stamp(step, 1 + 16 * l + 5);
                floatx4 acc[1];
                mfma_rows(wp, act, Bl, acc);
                stamp(step, 1 + 16 * l + 6);
                reduce_emit<1>(acc, red, hi_p - lo_p, Bl, [&](int r, int b, float v) {
                    ll_put(&xdx1[b * C + lo_p + r], v, ep + 3);
                });
                load_w2_part<NT2, TQ>(w2, lw.w2T, C4, lo_f, hi_f - lo_f); issue_here();
            }

            stamp(step, 1 + 16 * l + 7);
            // ---- hop 4: x += dx1, LN1, FC rows + GELU -> this WG's h slice, and its proj2
            // partial for all C outputs -> part ---------------------------------------------
            {
                float gm[NE], bt[NE];
                load_vec(lw.ln1g, gm);
                load_vec(lw.ln1b, bt);
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int b = wave + kWaves * k;
                    if (b < Bl) {
                        float d[NE];
                        ll_row(xdx1 + (size_t)b * C, C, ep + 3, d, bail, a.err);
#pragma unroll
                        for (int m = 0; m < NE; ++m) x[k][m] += d[m];
                        ln_row_swz(x[k], gm, bt, act, b);
                    }
                }
                lds_barrier();
                stamp(step, 1 + 16 * l + 8);
                floatx4 acc[TQ];
                mfma_rows(wf, act, Bl, acc);
                stamp(step, 1 + 16 * l + 9);
                reduce_emit<TQ>(acc, red, hi_f - lo_f, Bl, [&](int r, int b, float v) {
                    hl[b * KR + (((r >> 2) ^ (b & 7)) << 2) + (r & 3)] = persist::gelu_ref(v);
                });
                stamp(step, 1 + 16 * l + 10);
                floatx4 pacc[NT2];
                mfma_w2_part(w2, hl, Bl, pacc);
                stamp(step, 1 + 16 * l + 11);
                {
                    // D[4 g + i][r] of tile wave + 4 i2 is output c = 16 (wave + 4 i2) + 4 g + i of
                    // sequence r: staged in pg as [r][c], then stored row by row (contiguous words)
                    const int r = lane & 15, g = lane >> 4;
                    if (r < Bl) {
#pragma unroll
                        for (int i2 = 0; i2 < NT2; ++i2)
#pragma unroll
                            for (int i = 0; i < 4; ++i) pg[r * C + kTile * (wave + 4 * i2) + 4 * g + i] = pacc[i2][i];
                    }
                    lds_barrier();
                    stamp(step, 1 + 16 * l + 12);
                    uint64_t* dst = xpart + (size_t)w * kGroupBatch * C;
                    for (int e = tid; e < Bl * C; e += kThreads) ll_put(&dst[e], pg[e], ep + 4);
                    lds_barrier();  // pg is overwritten by hop 5's gather
                }
                if (l + 1 < L) load_w<TQ, NE>(wq, a.layers[l + 1].wqkvT, lo_q, hi_q - lo_q);
                else if (cnt > 0) load_w<1, NE>(wl, a.lm, lo_l, cnt);
                issue_here();
            }

            stamp(step, 1 + 16 * l + 13);
            // ---- hop 5: add the G partials of this WG's proj2 outputs -> dx2 ------------------
            {
                const int np = hi_p - lo_p, per = Bl * np, n = G * per;
                for (int base = 0; base < n; base += 12 * kThreads) {
                    const uint64_t* pp[12];
                    uint64_t vv[12];
#pragma unroll
                    for (int k = 0; k < 12; ++k) {
                        const int i = base + tid + k * kThreads;
                        const int wg = i / per, rem = i - wg * per, b = rem / np, cc = rem - b * np;
                        pp[k] = i < n ? &xpart[((size_t)wg * kGroupBatch + b) * C + lo_p + cc] : nullptr;
                    }
                    ll_issue_n(pp, vv, ep + 4);
                    ll_settle_n(pp, vv, ep + 4, bail, a.err);
#pragma unroll
                    for (int k = 0; k < 12; ++k) {
                        const int i = base + tid + k * kThreads;
                        if (i < n) pg[i] = ll_float(vv[k]);
                    }
                }
                lds_barrier();
                stamp(step, 1 + 16 * l + 14);
                if (tid < per) {  // partials added in workgroup order
                    float sum = pg[tid];
                    for (int wg = 1; wg < G; ++wg) sum += pg[wg * per + tid];
                    const int b = tid / np, cc = tid - b * np;
                    ll_put(&xdx2[b * C + lo_p + cc], sum, ep + 5);
                }
            }
            stamp(step, 1 + 16 * l + 15);
        }

        // ---- lm_head hop: x += dx2, ln_f, logits, per-WG candidates, token ----------------
        const uint32_t ep_lm = ep0 + 5u * L + 1u;
        const int lo = lo_l;
        {
            float gm[NE], bt[NE];
            load_vec(a.lnf_g, gm);
            load_vec(a.lnf_b, bt);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int b = wave + kWaves * k;
                if (b < Bl) {
                    float d[NE];
                    ll_row(xdx2 + (size_t)b * C, C, ep_lm - 1, d, bail, a.err);
#pragma unroll
                    for (int m = 0; m < NE; ++m) x[k][m] += d[m];
                    ln_row_swz(x[k], gm, bt, act, b);
                }
            }
            lds_barrier();
            if (cnt > 0) {  // WG-uniform
                floatx4 acc[1];
                mfma_rows(wl, act, Bl, acc);
                const bool keep = a.logit_hist && (size_t)(a.gen0 + step) < a.hist_slots;
                reduce_emit<1>(acc, red, cnt, Bl, [&](int r, int b, float v) {
                    const int n = lo + r;
                    logits[(size_t)b * V + n] = v;
                    if (keep) a.logit_hist[((size_t)(a.gen0 + step) * a.B + s0 + b) * V + n] = v;
                    lgs[r * kGroupBatch + b] = v;
                });
            }
        }
        stamp(step, 1 + 16 * L + 0);
        // Per-WG first maximum of each sequence over its rows (WGs without rows publish
        // nothing), then every WG gathers the candidates and reduces them: largest value, lowest
        // index among equal values -- the first maximum (NanoLLM.cpp:192-201).
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int b = wave + kWaves * k;
            if (b < Bl && cnt > 0) {
                const float v = lane < cnt ? lgs[lane * kGroupBatch + b] : -INFINITY;
                float best;
                const int idx = wave_argmax(v, lane < cnt ? lo + lane : -1, best);
                if (lane == 0) {
                    ll_put(&xam[((size_t)w * kGroupBatch + b) * 2], best, ep_lm);
                    ll_put_bits(&xam[((size_t)w * kGroupBatch + b) * 2 + 1], static_cast<uint32_t>(idx), ep_lm);
                }
            }
        }
        if (step + 1 < a.n_steps) load_w<TQ, NE>(wq, a.layers[0].wqkvT, lo_q, hi_q - lo_q); issue_here(); issue_here();
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int b = wave + kWaves * k;
            if (b < Bl) {
                constexpr int NU = 2;  // G <= 128
                const uint64_t* pa[2 * NU];
                uint64_t va[2 * NU];
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    const int gw = lane + 64 * u;
                    const bool owns = gw < G && (static_cast<long>(V) * (gw + 1)) / G > (static_cast<long>(V) * gw) / G;
                    pa[2 * u] = owns ? &xam[((size_t)gw * kGroupBatch + b) * 2] : nullptr;
                    pa[2 * u + 1] = owns ? &xam[((size_t)gw * kGroupBatch + b) * 2 + 1] : nullptr;
                }
                ll_issue_n(pa, va, ep_lm);
                ll_settle_n(pa, va, ep_lm, bail, a.err);
                float bv = -INFINITY;
                int bi = -1;
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    if (pa[2 * u] != nullptr) {
                        const float v = ll_float(va[2 * u]);
                        const int idx = static_cast<int>(static_cast<uint32_t>(va[2 * u + 1]));
                        if (idx >= 0 && (bi < 0 || v > bv || (v == bv && idx < bi))) {
                            bv = v;
                            bi = idx;
                        }
                    }
                }
                float best;
                const int t = wave_argmax(bv, bi, best);
                tok[k] = t < 0 ? 0 : t;
                if (w == 0 && lane == 0) hist[(size_t)b * a.HS + pos + 1] = tok[k];
            }
        }
        stamp(step, 1 + 16 * L + 1);
    }
    if (blockIdx.x == 0 && tid == 0) {
        a.st_pos[0] = a.pos0 + a.n_steps;
        a.st_pos[1] = a.gen0 + a.n_steps;
    }
}

template <int HD, int NE, int TQ>
int launch(const GroupedArgs& a, const GroupedPlan& p, hipStream_t s) {
    auto kern = decode_grouped_kernel<HD, NE, TQ>;
    FMLH_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(p.smem)));
    if (inject_fault(kFaultLaunch))
        return set_error(FMLH_E_HIP, "decode_grouped_kernel: launch failed (injected by FMLH_FAULT)");
    GroupedArgs args = a;
    void* params[] = {&args};
    const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kern), dim3(p.G * p.groups),
                                                    dim3(kThreads), params, static_cast<unsigned>(p.smem), s);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        set_error(FMLH_E_HIP, "grouped decode: cooperative launch refused (%s)", hipGetErrorString(e));
        return kPersistRefused;
    }
    return FMLH_OK;
}

template <int HD, int NE>
int launch_tq(const GroupedArgs& a, const GroupedPlan& p, hipStream_t s) {
    switch (p.tq) {
        case 1: return launch<HD, NE, 1>(a, p, s);
        case 2: return launch<HD, NE, 2>(a, p, s);
        case 3: return launch<HD, NE, 3>(a, p, s);
        default: return set_error(FMLH_E_INVALID, "grouped decode: %d row tiles per workgroup", p.tq);
    }
}

}  // namespace grouped
}  // namespace fmlh
