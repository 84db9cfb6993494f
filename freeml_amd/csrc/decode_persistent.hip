// Persistent decode kernel: many greedy decode steps of the NanoLLM token loop in one
// cooperative launch, for small batches (B <= 8).
//
// Why: a decode step at batch 1 moves ~45 MB (c2) -- a few microseconds of HBM time -- but
// as ~60 separate kernels it costs ~540 us, almost all launch and dependency latency.  Here
// every workgroup (WG) stays resident for the whole loop and the phases of a step exchange
// their outputs through global memory.
//
// Exchange protocol ("LL" words).  Every value passed between WGs is a 64-bit word
// {payload bits, epoch}, written with one agent-scope store and read with agent-scope loads
// (both bypass the per-XCD L2, so no cache maintenance is needed).  A consumer spins on the
// words themselves until their epoch is the one it expects, so a hand-off costs one store and
// one load round trip instead of a grid barrier plus a load.  Epochs are unique per
// (launch, step, hop) and increase monotonically across launches.
//
// Why single buffers are safe: hops 3, 4, 5 and the lm_head hop are all-to-all -- every WG
// publishes at least one word (G <= n_embed) and every WG waits for all words.  A WG can only
// rewrite a buffer after consuming an all-to-all hop whose words each WG publishes after its
// own read of that buffer, so no reader can still be waiting on the old contents.
//
// Each WG keeps its own copy of the residual stream x[B][C] in LDS and recomputes the
// LayerNorms redundantly, so only projection outputs travel.  Per layer and step:
//   hop 1: x += dx2 (previous layer), LN0, QKV columns  -> Q, Knew, Vnew (+ KV cache rows)
//   hop 2: attention items (sequence, head, key chunk)   -> partial (max, sum, P.V)
//   hop 3: combine partials -> y, attention-proj columns -> dx1
//   hop 4: x += dx1, LN1, FC columns, GELU               -> h
//   hop 5: proj2 columns                                 -> dx2
// then x += dx2, ln_f, lm_head columns -> logits + per-WG (max, index); every WG reduces the
// G candidates itself (first maximum, NanoLLM.cpp:192-201), so the next token never leaves
// the device and the next step starts without another hand-off.
//
// Weights are read from engine-owned copies laid out one output per contiguous row
// (W_qkv^T, W_fc^T, W_proj2^T; W_proj and lm_head already are), so each WG's slice of a hop is
// one contiguous block, prefetched into registers before the WG waits for the hop's inputs.
//
// Every wait is bounded: after ~1 s of spinning a wait sets an error flag and the WG stops
// waiting for the rest of the launch, so a protocol error ends the kernel instead of hanging.
#include "decode_persistent.h"

#include <algorithm>

namespace fmlh {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kItemKeys = 64;  // keys per attention item (key chunk)
constexpr long kSpinLimit = 1L << 21;  // loads of ~0.5-1 us each: a few seconds at most

__device__ __forceinline__ uint64_t ll_pack(float v, uint32_t epoch) {
    return (static_cast<uint64_t>(epoch) << 32) | __float_as_uint(v);
}
__device__ __forceinline__ void ll_put(uint64_t* p, float v, uint32_t epoch) {
    __hip_atomic_store(p, ll_pack(v, epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_put_bits(uint64_t* p, uint32_t bits, uint32_t epoch) {
    __hip_atomic_store(p, (static_cast<uint64_t>(epoch) << 32) | bits, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Waits for word p to carry `epoch`; returns its payload bits.  `bail` (LDS) short-cuts every
// wait of the WG once any of its waits timed out.
__device__ __forceinline__ uint32_t ll_get_bits(const uint64_t* p, uint32_t epoch, int* bail,
                                               unsigned* err) {
    long it = 0;
    while (true) {
        const uint64_t v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (static_cast<uint32_t>(v >> 32) == epoch) return static_cast<uint32_t>(v);
        if (*reinterpret_cast<volatile int*>(bail)) return static_cast<uint32_t>(v);
        if (++it > kSpinLimit) {
            *reinterpret_cast<volatile int*>(bail) = 1;
            atomicOr(err, 1u);
            return static_cast<uint32_t>(v);
        }
    }
}
__device__ __forceinline__ float ll_get(const uint64_t* p, uint32_t epoch, int* bail, unsigned* err) {
    return __uint_as_float(ll_get_bits(p, epoch, bail, err));
}

// Waits for words src[0..n) to carry `epoch` and writes their payloads to dst (LDS).  Each
// thread issues the loads of up to 8 of its words back to back and only re-polls the ones
// that were not current yet, so one round trip usually covers all of them.
__device__ __forceinline__ void ll_gather(const uint64_t* src, int n, uint32_t epoch, float* dst,
                                          int* bail, unsigned* err) {
    constexpr int kBatch = 8;
    for (int base = 0; base < n; base += kBatch * kThreads) {
        uint64_t v[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int i = base + k * kThreads + threadIdx.x;
            v[k] = i < n ? __hip_atomic_load(&src[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                         : (static_cast<uint64_t>(epoch) << 32);
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const int i = base + k * kThreads + threadIdx.x;
            if (i < n) {
                const uint32_t bits = static_cast<uint32_t>(v[k] >> 32) == epoch
                                          ? static_cast<uint32_t>(v[k])
                                          : ll_get_bits(&src[i], epoch, bail, err);
                dst[i] = __uint_as_float(bits);
            }
        }
    }
}

// Coherent scalar accesses for data written during the launch (the KV cache rows).
__device__ __forceinline__ void st_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// KV-cache rows written during the launch are read with plain (cacheable) vector loads when a
// row covers whole 128-byte lines: the row was stored once, write-through (st_coherent), and
// no workgroup can have cached its lines earlier in the launch (keys beyond the current
// position are never read, and the kernel launch starts with invalidated caches).  Shorter
// rows share lines with neighbouring positions and use coherent loads.
template <int HD>
constexpr bool kPlainRows = (HD * 4) % 128 == 0;

// End of a hop: this thread's stores have completed and the whole WG is past them.
__device__ __forceinline__ void hop_end() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}

__device__ __forceinline__ float gelu_ref(float x) { return 0.5f * x * (1.0f + erff(x / 1.41421354f)); }

// Balanced split of n outputs over G WGs.
__device__ __forceinline__ void my_range(int n, int G, int w, int& lo, int& hi) {
    lo = (int)(((long)n * w) / G);
    hi = (int)(((long)n * (w + 1)) / G);
}

struct Smem {
    float* x;    // B x C residual stream
    float* act;  // B x max(4C, C): LayerNorm output / attention y / MLP h
    float* w;    // weight slice
    float* red;  // kThreads scratch
    float* part; // attention partials of every (sequence, head): B*H*max_chunks*(HD+2)
    float* lnp;  // LayerNorm gains/shifts: per layer {g0, b0, g1, b1}, then {g_f, b_f}; C each
    float* kbuf; // cached K rows of one attention item: kItemKeys x HD
    float* vbuf; // cached V rows of one attention item
    int* misc;   // [0] bail, [1..8] tokens
};

// Prefetch of a contiguous weight slice straight into LDS (global_load_lds_dwordx4: each lane
// moves 16 bytes to the wave's M0 base + 16 * lane), so the loads fly while the WG waits for
// the hop's inputs and need no registers.  Complete after s_waitcnt vmcnt(0) + a barrier.
__device__ __forceinline__ void prefetch_lds(float* lds, const float* src, int nfloats) {
    const int n4 = nfloats / 4;
    for (int i = threadIdx.x; i < n4; i += kThreads) {
        const int wave_base = i - (int)(threadIdx.x % 64);  // float4 index of lane 0's chunk
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(src + 4 * (size_t)i),
                                         (__attribute__((address_space(3))) void*)(
                                             lds + 4 * (size_t)wave_base),
                                         16, 0, 0);
    }
}

// LayerNorm of the B rows of x (LDS) into out (LDS), one wave per row (LayerNormOp,
// MatrixBase_Functions.h:481-549).
__device__ void ln_rows(const float* x, float* out, int B, int C, const float* g, const float* bta) {
    // g, bta: LDS copies
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const float inv_cols = 1.0f / (float)C;
    for (int b = wave; b < B; b += kWaves) {
        const float* xr = x + b * C;
        float s = 0.f;
        for (int c = lane; c < C; c += 64) s += xr[c];
        const float mean = wave_sum(s) * inv_cols;
        float v = 0.f;
        for (int c = lane; c < C; c += 64) {
            const float d = xr[c] - mean;
            v += d * d;
        }
        const float inv_std = 1.0f / sqrtf(wave_sum(v) * inv_cols + 1e-5f);
        for (int c = lane; c < C; c += 64)
            out[b * C + c] = (xr[c] - mean) * inv_std * g[c] + bta[c];
    }
}

// out[b][i] = sum_k act[b][k] * w[i][k] for the WG's rows i < cnt; act rows have stride K
// (K % 4 == 0).  Waves take rows i = wave, wave + 4, ...; lanes take float4 chunks of k, so
// each lane issues its LDS reads back to back; returns through `emit(i, b, v)` on lane 0.
template <class Emit>
__device__ __forceinline__ void gemv_rows(const float* w, int cnt, int K, const float* act, int B,
                                          Emit emit) {
    const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
    const int K4 = K / 4;
    for (int i = wave; i < cnt; i += kWaves) {
        const float4* wr = reinterpret_cast<const float4*>(w + (size_t)i * K);
        float acc[kMaxPersistBatch];
#pragma unroll
        for (int b = 0; b < kMaxPersistBatch; ++b) acc[b] = 0.f;
#pragma unroll 4
        for (int q = lane; q < K4; q += 64) {
            const float4 wv = wr[q];
#pragma unroll
            for (int b = 0; b < kMaxPersistBatch; ++b) {
                if (b < B) {
                    const float4 av = reinterpret_cast<const float4*>(act + (size_t)b * K)[q];
                    acc[b] += wv.x * av.x + wv.y * av.y + wv.z * av.z + wv.w * av.w;
                }
            }
        }
#pragma unroll
        for (int b = 0; b < kMaxPersistBatch; ++b) {
            if (b < B) {
                const float v = wave_sum(acc[b]);
                if (lane == 0) emit(i, b, v);
            }
        }
    }
}

template <int HD>
__global__ __launch_bounds__(kThreads) void decode_persistent_kernel(PersistArgs a) {
    extern __shared__ float smem_f[];
    const int B = a.B, C = a.C, H = a.H, L = a.L, V = a.V;
    const int G = gridDim.x, w = blockIdx.x, tid = threadIdx.x;
    const int C4 = 4 * C;
    Smem sm;
    sm.x = smem_f;
    sm.act = sm.x + B * C;
    sm.w = sm.act + B * C4;
    sm.red = sm.w + a.wcap;
    sm.part = sm.red + kThreads;
    sm.lnp = sm.part + (size_t)B * H * a.max_chunks * (HD + 2);
    sm.kbuf = sm.lnp + (size_t)(4 * L + 2) * C;
    sm.vbuf = sm.kbuf + kItemKeys * HD;
    sm.misc = reinterpret_cast<int*>(sm.vbuf + kItemKeys * HD);
    int* bail = sm.misc;
    int* toks = sm.misc + 1;
    if (tid == 0) *bail = 0;
    const int hops = 5 * L + 1;
    const float scale = a.scale;
    const int KC = a.key_chunk;

    // Optional timeline of WG 0 (development aid, FMLH_PERSIST_TRACE=1).
    int tp = 0;
    auto stamp = [&](int step) {
        if (a.trace && w == 0 && tid == 0 && step < kTraceSteps && tp < kTracePoints)
            a.trace[step * kTracePoints + tp] = wall_clock64();
        ++tp;
    };

    // LayerNorm parameters stay in LDS for the whole launch (BetaShift absent -> 0).
    for (int e = tid; e < (4 * L + 2) * C; e += kThreads) {
        const int r = e / C, c = e % C, l = r / 4, k = r % 4;
        const float* src;
        if (r < 4 * L) {
            const PersistLayer& pl = a.layers[l];
            src = k == 0 ? pl.ln0g : k == 1 ? pl.ln0b : k == 2 ? pl.ln1g : pl.ln1b;
        } else {
            src = r == 4 * L ? a.lnf_g : a.lnf_b;
        }
        sm.lnp[e] = src ? src[c] : 0.f;
    }
    // Step 0 token per sequence: the last token of the history (prefill or previous launch).
    if (tid < B) toks[tid] = a.hist[(size_t)tid * a.HS + a.pos0];
    __syncthreads();

    for (int step = 0; step < a.n_steps; ++step) {
        const int pos = a.pos0 + step;
        const uint32_t ep0 = a.epoch_base + (uint32_t)step * hops;
        tp = 0;
        stamp(step);
        // Embedding x = tok[token] + pos_emb[pos] (Embedding x2 + AddLayer; dropout p = 0).
        for (int e = tid; e < B * C; e += kThreads) {
            const int b = e / C, c = e % C;
            sm.x[e] = a.tok[(size_t)toks[b] * C + c] + a.pos_emb[(size_t)pos * C + c];
        }
        __syncthreads();

        for (int l = 0; l < L; ++l) {
            const PersistLayer& lw = a.layers[l];
            const uint32_t ep = ep0 + 5u * l;
            float* kc = a.kc + (size_t)l * a.Bmax * H * a.T * HD;
            float* vc = a.vc + (size_t)l * a.Bmax * H * a.T * HD;

            // ---- hop 1: QKV --------------------------------------------------------------
            int lo, hi;
            my_range(3 * C, G, w, lo, hi);
            int wn = (hi - lo) * C;
            prefetch_lds(sm.w, lw.wqkvT + (size_t)lo * C, wn);
            if (l > 0) {  // x += dx2 of layer l-1, published at epoch ep0 + 5(l-1) + 5 = ep
                ll_gather(a.dx2, B * C, ep, sm.act, bail, a.err);
                for (int e = tid; e < B * C; e += kThreads) sm.x[e] += sm.act[e];
            }
            __syncthreads();
            stamp(step);
            ln_rows(sm.x, sm.act, B, C, sm.lnp + (size_t)(4 * l) * C, sm.lnp + (size_t)(4 * l + 1) * C);
            __syncthreads();
            stamp(step);
            __builtin_amdgcn_s_waitcnt(0);  // weight slice landed in LDS
            (void)wn;
            __syncthreads();
            stamp(step);
            gemv_rows(sm.w, hi - lo, C, sm.act, B, [&](int i, int b, float v) {
                const int n = lo + i;
                uint64_t* dst = n < C ? a.q : (n < 2 * C ? a.kn : a.vn);
                ll_put(&dst[b * C + n % C], v, ep + 1);
            });
            __syncthreads();
            stamp(step);
            hop_end();
            stamp(step);

            // ---- hop 2: attention partials (sequence, head, key chunk) ---------------------
            // Item (chunk ch, pair bh) always runs on WG (ch * B * H + bh) % G, so the WG that
            // writes a new K/V row (the owner of the chunk holding pos) is the only one that
            // reads it in later steps: plain stores and loads on one CU need no cross-CU
            // coherence.  Cached rows go to LDS by DMA before the WG waits for q.
            const int nch = pos / kItemKeys + 1;
            const int pairs = B * H;
            float* qs = sm.red;              // HD
            float* kn = sm.red + 64;         // HD
            float* vn = sm.red + 128;        // HD
            float* sc = sm.act;              // kItemKeys scores (act is free until hop 3)
            float* pv = sm.act + kItemKeys;  // kThreads partial P.V
            for (int item = w; item < nch * pairs; item += G) {
                const int ch = item / pairs, bh = item % pairs;
                const int b = bh / H, hh = bh % H;
                const int j0 = ch * kItemKeys, j1 = min(j0 + kItemKeys, pos + 1);
                const bool has_new = j1 == pos + 1;
                const int nold = has_new ? j1 - 1 - j0 : j1 - j0;  // cached rows in the chunk
                float* kb = kc + ((size_t)bh * a.T) * HD;
                float* vb = vc + ((size_t)bh * a.T) * HD;
                prefetch_lds(sm.kbuf, kb + (size_t)j0 * HD, nold * HD);
                prefetch_lds(sm.vbuf, vb + (size_t)j0 * HD, nold * HD);
                if (tid < HD) {
                    qs[tid] = ll_get(&a.q[b * C + hh * HD + tid], ep + 1, bail, a.err);
                    if (has_new) {
                        const float kv = ll_get(&a.kn[b * C + hh * HD + tid], ep + 1, bail, a.err);
                        const float vv = ll_get(&a.vn[b * C + hh * HD + tid], ep + 1, bail, a.err);
                        kn[tid] = kv;
                        vn[tid] = vv;
                        kb[(size_t)pos * HD + tid] = kv;  // the cache row of this step
                        vb[(size_t)pos * HD + tid] = vv;
                    }
                }
                __builtin_amdgcn_s_waitcnt(0);  // K/V rows landed in LDS
                __syncthreads();
                // scores: 4 threads per key, HD/4 dims each (the 4 lanes of a key leave the
                // loop together, so the xor-shuffles stay inside active lane groups)
                const int n = j1 - j0;
                for (int jj = tid / 4; jj < n; jj += kThreads / 4) {
                    const int part = tid % 4;
                    constexpr int DQ = HD / 4;
                    const float* kr = jj < nold ? sm.kbuf + (size_t)jj * HD : kn;
                    float s = 0.f;
#pragma unroll
                    for (int d = part * DQ; d < (part + 1) * DQ; ++d) s += qs[d] * kr[d];
                    s += __shfl_xor(s, 1, 64);
                    s += __shfl_xor(s, 2, 64);
                    if (part == 0) sc[jj] = s * scale;
                }
                __syncthreads();
                float m = -INFINITY;
                for (int j = tid; j < n; j += kThreads) m = fmaxf(m, sc[j]);
                m = wave_max(m);
                if (tid % 64 == 0) pv[tid / 64] = m;
                __syncthreads();
                m = fmaxf(fmaxf(pv[0], pv[1]), fmaxf(pv[2], pv[3]));
                __syncthreads();
                float lsum = 0.f;
                for (int j = tid; j < n; j += kThreads) {
                    const float p = expf(sc[j] - m);
                    sc[j] = p;
                    lsum += p;
                }
                lsum = wave_sum(lsum);
                if (tid % 64 == 0) pv[tid / 64] = lsum;
                __syncthreads();
                lsum = (pv[0] + pv[1]) + (pv[2] + pv[3]);
                __syncthreads();
                {
                    constexpr int GR = kThreads / HD;
                    const int d = tid % HD, g = tid / HD;
                    float acc = 0.f;
                    for (int j = g; j < n; j += GR) acc += sc[j] * (j < nold ? sm.vbuf[(size_t)j * HD + d] : vn[d]);
                    pv[tid] = acc;
                }
                __syncthreads();
                // partials laid out [chunk][sequence * H + head][HD + 2]: the current words of
                // a layer are one contiguous range
                uint64_t* slot = a.att + ((size_t)ch * pairs + bh) * (HD + 2);
                if (tid < HD) {
                    float o = 0.f;
#pragma unroll
                    for (int g = 0; g < kThreads / HD; ++g) o += pv[g * HD + tid];
                    ll_put(&slot[2 + tid], o, ep + 2);
                }
                if (tid == 0) {
                    ll_put(&slot[0], m, ep + 2);
                    ll_put(&slot[1], lsum, ep + 2);
                }
                __syncthreads();
            }
            hop_end();
            stamp(step);

            // ---- hop 3: combine -> y, attention proj -> dx1 -----------------------------
            my_range(C, G, w, lo, hi);
            wn = (hi - lo) * C;
            prefetch_lds(sm.w, lw.wproj + (size_t)lo * C, wn);
            // All partials of this layer: nch chunks x B*H pairs x (HD + 2) words.
            const int pstride = B * H * (HD + 2);  // words per chunk
            ll_gather(a.att, nch * pstride, ep + 2, sm.part, bail, a.err);
            __syncthreads();
            stamp(step);
            for (int e = tid; e < B * C; e += kThreads) {
                const int b = e / C, c = e % C, hh = c / HD, d = c % HD;
                const float* pp = sm.part + (size_t)(b * H + hh) * (HD + 2);
                float m = -INFINITY;
                for (int ch = 0; ch < nch; ++ch) m = fmaxf(m, pp[ch * pstride]);
                float lsum = 0.f, o = 0.f;
                for (int ch = 0; ch < nch; ++ch) {
                    const float wgt = expf(pp[ch * pstride] - m);
                    lsum += wgt * pp[ch * pstride + 1];
                    o += wgt * pp[ch * pstride + 2 + d];
                }
                sm.act[e] = o / lsum;
            }
            __builtin_amdgcn_s_waitcnt(0);  // weight slice landed in LDS
            (void)wn;
            __syncthreads();
            gemv_rows(sm.w, hi - lo, C, sm.act, B,
                      [&](int i, int b, float v) { ll_put(&a.dx1[b * C + lo + i], v, ep + 3); });
            hop_end();
            stamp(step);

            // ---- hop 4: x += dx1, LN1, FC + GELU -> h ------------------------------------
            my_range(C4, G, w, lo, hi);
            wn = (hi - lo) * C;
            prefetch_lds(sm.w, lw.wfcT + (size_t)lo * C, wn);
            ll_gather(a.dx1, B * C, ep + 3, sm.act, bail, a.err);
            for (int e = tid; e < B * C; e += kThreads) sm.x[e] += sm.act[e];
            __syncthreads();
            stamp(step);
            ln_rows(sm.x, sm.act, B, C, sm.lnp + (size_t)(4 * l + 2) * C, sm.lnp + (size_t)(4 * l + 3) * C);
            __builtin_amdgcn_s_waitcnt(0);  // weight slice landed in LDS
            (void)wn;
            __syncthreads();
            gemv_rows(sm.w, hi - lo, C, sm.act, B,
                      [&](int i, int b, float v) { ll_put(&a.hb[b * C4 + lo + i], gelu_ref(v), ep + 4); });
            hop_end();
            stamp(step);

            // ---- hop 5: proj2 -> dx2 -------------------------------------------------------
            my_range(C, G, w, lo, hi);
            wn = (hi - lo) * C4;
            prefetch_lds(sm.w, lw.w2T + (size_t)lo * C4, wn);
            ll_gather(a.hb, B * C4, ep + 4, sm.act, bail, a.err);
            stamp(step);
            __builtin_amdgcn_s_waitcnt(0);  // weight slice landed in LDS
            (void)wn;
            __syncthreads();
            gemv_rows(sm.w, hi - lo, C4, sm.act, B,
                      [&](int i, int b, float v) { ll_put(&a.dx2[b * C + lo + i], v, ep + 5); });
            hop_end();
            stamp(step);
        }

        // ---- lm_head hop: x += dx2, ln_f, logits, per-WG candidates ----------------------
        const uint32_t ep_lm = ep0 + 5u * L + 1u;
        int lo, hi;
        my_range(V, G, w, lo, hi);
        const int wn = (hi - lo) * C;
        prefetch_lds(sm.w, a.lm + (size_t)lo * C, wn);
        ll_gather(a.dx2, B * C, ep_lm - 1, sm.act, bail, a.err);
        for (int e = tid; e < B * C; e += kThreads) sm.x[e] += sm.act[e];
        __syncthreads();
        ln_rows(sm.x, sm.act, B, C, sm.lnp + (size_t)(4 * L) * C, sm.lnp + (size_t)(4 * L + 1) * C);
        __builtin_amdgcn_s_waitcnt(0);  // weight slice landed in LDS
            (void)wn;
        __syncthreads();
        float* lgs = sm.act + B * C;  // this WG's logits, after the LN output
        gemv_rows(sm.w, hi - lo, C, sm.act, B, [&](int i, int b, float v) {
            const int n = lo + i;
            a.logits[(size_t)b * V + n] = v;
            if (a.logit_hist && (size_t)(a.gen0 + step) < a.hist_slots)
                a.logit_hist[((size_t)(a.gen0 + step) * B + b) * V + n] = v;
            lgs[i * B + b] = v;
        });
        __syncthreads();
        // per-WG first maximum of each row over its slice; empty slices publish -inf
        if (tid < B) {
            float bv = -INFINITY;
            int bi = -1;
            for (int i = 0; i < hi - lo; ++i) {
                const float v = lgs[i * B + tid];
                if (bi < 0 || v > bv) { bv = v; bi = lo + i; }
            }
            ll_put(&a.am[((size_t)w * B + tid) * 2], bv, ep_lm);
            ll_put_bits(&a.am[((size_t)w * B + tid) * 2 + 1], (uint32_t)bi, ep_lm);
        }
        hop_end();
        stamp(step);
        // every WG gathers the G candidates and reduces them in WG order: the lowest index
        // wins ties (first maximum)
        ll_gather(a.am, 2 * G * B, ep_lm, sm.act, bail, a.err);
        __syncthreads();
        if (tid < B) {
            float bv = -INFINITY;
            int bi = -1;
            for (int g = 0; g < G; ++g) {
                const float v = sm.act[(g * B + tid) * 2];
                const int idx = (int)__float_as_uint(sm.act[(g * B + tid) * 2 + 1]);
                if (idx >= 0 && (bi < 0 || v > bv || (v == bv && idx < bi))) { bv = v; bi = idx; }
            }
            toks[tid] = bi < 0 ? 0 : bi;
            if (w == 0) a.hist[(size_t)tid * a.HS + pos + 1] = toks[tid];
        }
        __syncthreads();
        stamp(step);
    }
    if (w == 0 && tid == 0) {
        a.st_pos[0] = a.pos0 + a.n_steps;
        a.st_pos[1] = a.gen0 + a.n_steps;
    }
}

__global__ void transpose_kernel(float* __restrict__ out, const float* __restrict__ in, int rows,
                                 int cols) {
    __shared__ float tile[32][33];
    const int bx = blockIdx.x * 32, by = blockIdx.y * 32;
    const int tx = threadIdx.x % 32, ty = threadIdx.x / 32;  // 256 threads: 32 x 8
    for (int r = ty; r < 32; r += 8) {
        const int gr = by + r, gc = bx + tx;
        tile[r][tx] = (gr < rows && gc < cols) ? in[(size_t)gr * cols + gc] : 0.f;
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        const int orow = bx + r, ocol = by + tx;  // out is cols x rows
        if (orow < cols && ocol < rows) out[(size_t)orow * rows + ocol] = tile[tx][r];
    }
}

template <int HD>
int launch(const PersistArgs& a, int G, size_t smem, hipStream_t s) {
    auto kern = decode_persistent_kernel<HD>;
    FMLH_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
    PersistArgs args = a;
    void* params[] = {&args};
    FMLH_HIP(hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kern), dim3(G), dim3(kThreads),
                                        params, (unsigned)smem, s));
    return FMLH_OK;
}

}  // namespace

size_t smem_limit() { return 160 * 1024; }

int persist_transpose(float* out, const float* in, int rows, int cols, hipStream_t s) {
    dim3 grid((cols + 31) / 32, (rows + 31) / 32);
    hipLaunchKernelGGL(transpose_kernel, grid, dim3(256), 0, s, out, in, rows, cols);
    FMLH_LAUNCHED("transpose_kernel");
    return FMLH_OK;
}

PersistPlan persist_plan(int B, int C, int H, int L, int V, int T, int cus) {
    PersistPlan p;
    const int hd = H > 0 ? C / H : 0;
    if (B < 1 || B > kMaxPersistBatch || (hd != 16 && hd != 32 && hd != 64) || C % 4 != 0) return p;
    p.G = std::min({C, cus, 128});
    // LDS for the largest per-WG weight slice (FC or proj2: ~4C*C/G floats, lm_head rows).
    const long slice = ((long)4 * C * C + p.G - 1) / p.G + 4L * C;  // + one row of slack
    const long lm_slice = ((long)(V + p.G - 1) / p.G) * C;
    p.wcap = (int)((std::max(slice, lm_slice) + 63) / 64 * 64);
    // One key chunk per attention item; the partials of all chunks are staged in LDS.
    if (T > 1024) return p;
    p.key_chunk = kItemKeys;
    p.max_chunks = (T + kItemKeys - 1) / kItemKeys;
    const size_t part = (size_t)B * H * p.max_chunks * (hd + 2);
    const size_t floats = (size_t)B * C + (size_t)B * 4 * C + (size_t)p.wcap + kThreads + part +
                          (size_t)(4 * L + 2) * C + 2 * kItemKeys * hd + 16;
    p.smem = floats * sizeof(float);
    if (p.smem > smem_limit()) return PersistPlan{};
    // act also holds the item's scores + P.V partials, and the 2 x G x B argmax candidates.
    if ((size_t)B * 4 * C < (size_t)kItemKeys + kThreads || (size_t)B * 4 * C < 2 * (size_t)p.G * B)
        return PersistPlan{};
    p.ok = true;
    return p;
}

int persist_decode(const PersistArgs& a, const PersistPlan& p, int hd, hipStream_t s) {
    if (!p.ok) return set_error(FMLH_E_INVALID, "persistent decode not planned for this shape");
    if (hd == 64) return launch<64>(a, p.G, p.smem, s);
    if (hd == 32) return launch<32>(a, p.G, p.smem, s);
    if (hd == 16) return launch<16>(a, p.G, p.smem, s);
    return set_error(FMLH_E_INVALID, "persistent decode: head_dim %d unsupported", hd);
}

}  // namespace fmlh
