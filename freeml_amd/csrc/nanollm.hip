// The NanoLLM token loop on one gfx950 device.
//
// Graph (Examples/NanoLLM/NanoLLM.cpp:255-376, Model.h:764-788):
//   x = tok_emb[id] + pos_emb[p]                          (Embedding x2 + AddLayer; dropout p=0)
//   per TransformerBlock (TransformerBlock.h:355-401):
//     qkv = LN0(x) W_qkv ; K,V -> cache ; y = causal_attention(q, K, V)
//     x  += y W_proj^T                                    (CSA proj + residual Add)
//     x  += gelu(LN1(x) W_fc) W_proj2                     (MLP + residual Add)
//   logits = LN_f(x) lm_head^T ; next = first argmax      (ln_f, FlattenCopy, lm_head, pick)
//
// Loop (the reference has none; its per-step oracle is Model::Run over the padded window at
// row len-1): prefill runs all prompt rows, then each decode step runs one row per sequence
// against the KV cache.  Between steps nothing leaves the device: the next token is written
// into the device token history by the argmax kernel and the step position is a device
// counter, so one captured HIP graph replays every step.
#include "attention.h"
#include "decode_grouped.h"
#include "decode_persistent.h"
#include "decode_relay.h"
#include "decode_wide.h"
#include "fmlh_internal.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <unordered_set>
#include <vector>

namespace fmlh {
namespace {

struct DevState {
    int pos;  // position processed by the next decode step
    int gen;  // tokens generated so far (the prefill's counts as 1)
};

// x[b*rows + r] = tok[hist[b][first + r]] + pos_emb[first + r]; first = st->pos if given.
// hist rows have stride HS.
__global__ void embed_kernel(float* __restrict__ x, const int32_t* __restrict__ hist, int HS,
                             int rows, int first_const, const DevState* st,
                             const float* __restrict__ tok, const float* __restrict__ pos_emb,
                             int C, int total_rows) {
    const int first = st ? st->pos : first_const;
    const size_t total = (size_t)total_rows * C;
    for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < total;
         e += (size_t)gridDim.x * blockDim.x) {
        const int m = (int)(e / C), c = (int)(e % C);
        const int b = m / rows, p = first + m % rows;
        const int id = hist[(size_t)b * HS + p];
        x[e] = tok[(size_t)id * C + c] + pos_emb[(size_t)p * C + c];
    }
}

// Copies row (b*rows + rows-1) of x to row b of out (the last prompt row of each sequence).
__global__ void last_rows_kernel(float* __restrict__ out, const float* __restrict__ x, int rows,
                                 int C, int batch) {
    const size_t total = (size_t)batch * C;
    for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < total;
         e += (size_t)gridDim.x * blockDim.x) {
        const int b = (int)(e / C), c = (int)(e % C);
        out[e] = x[((size_t)b * rows + rows - 1) * C + c];
    }
}

// First-max argmax of logits row b (NanoLLM.cpp:192-201) written to hist[b][pos + 1].  One
// 1024-thread work-group per row: each thread scans every 1024th logit (eight loads in flight),
// then waves and the work-group keep the larger value, the lower index on ties.
constexpr int kArgmaxThreads = 1024;

__device__ __forceinline__ void argmax_merge(float& bv, int& bi, float ov, int oi) {
    if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) {
        bv = ov;
        bi = oi;
    }
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_hist_kernel(int32_t* __restrict__ hist, int HS,
                                                                     const float* __restrict__ logits, int V,
                                                                     const DevState* st, int pos_const) {
    __shared__ float sv[kArgmaxThreads / 64];
    __shared__ int si[kArgmaxThreads / 64];
    const int b = blockIdx.x, tid = threadIdx.x;
    const float* row = logits + (size_t)b * V;
    float bv = -INFINITY;
    int bi = -1;
#pragma unroll 8
    for (int c = tid; c < V; c += kArgmaxThreads) {
        const float v = row[c];
        if (bi < 0 || v > bv) { bv = v; bi = c; }  // c increases: the first maximum stays
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        argmax_merge(bv, bi, ov, oi);
    }
    if ((tid & 63) == 0) {
        sv[tid >> 6] = bv;
        si[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < kArgmaxThreads / 64; ++w) argmax_merge(bv, bi, sv[w], si[w]);
        const int p = (st ? st->pos : pos_const) + 1;
        if (p < HS) hist[(size_t)b * HS + p] = bi < 0 ? 0 : bi;
    }
}

// ---- sampling (no counterpart in the reference, whose NanoLLM decodes greedily) ----------
//
// Token i of a row is drawn with probability proportional to exp((z_i - max z) / temperature)
// over the top_k largest logits (ties at the k-th value go to the lower indices; top_k 0 or
// >= V keeps every logit), by inverse CDF in index order: the first i whose running weight sum
// exceeds u * (total), u uniform in [0, 1) from the sequence index, the position being filled
// and the seed (splitmix64, 24 bits).  Each thread owns a contiguous chunk of the row so the
// block scans run in index order.
struct SampleCfg {
    float inv_temp;
    int top_k;
    unsigned long long seed;
};

__device__ __forceinline__ unsigned long long splitmix64(unsigned long long x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

__device__ __forceinline__ float sample_uniform(unsigned long long seed, int b, int p) {
    const unsigned long long key = ((unsigned long long)(unsigned)b << 32) | (unsigned)p;
    return (float)(splitmix64(seed ^ splitmix64(key)) >> 40) * (1.0f / 16777216.0f);
}

// Order-preserving float -> uint32 (larger float, larger key; -0 and +0 distinct, no NaNs).
__device__ __forceinline__ uint32_t float_key(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive prefix sum over the block's threads in thread order (T = blockDim.x, a multiple of
// 64); also returns the total.
template <class V>
__device__ V block_exclusive_scan(V x, V* sh, V* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    V incl = x;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const V y = __shfl_up(incl, off);
        if (lane >= off) incl += y;
    }
    __syncthreads();
    if (lane == 63) sh[w] = incl;
    __syncthreads();
    V base = 0, tot = 0;
    for (int i = 0; i < nw; ++i) {
        if (i < w) base += sh[i];
        tot += sh[i];
    }
    *total = tot;
    return base + incl - x;
}

__global__ __launch_bounds__(kArgmaxThreads) void sample_hist_kernel(int32_t* __restrict__ hist, int HS,
                                                                     const float* __restrict__ logits, int V,
                                                                     const DevState* st, int pos_const,
                                                                     SampleCfg cfg) {
    __shared__ float shf[kArgmaxThreads / 64];
    __shared__ uint32_t shu[kArgmaxThreads / 64];
    __shared__ uint32_t hist256[256];
    __shared__ uint32_t radix_sh[2];
    __shared__ int pick_sh[2];
    const int b = blockIdx.x, tid = threadIdx.x;
    const float* row = logits + (size_t)b * V;
    const int chunk = (V + (int)blockDim.x - 1) / (int)blockDim.x;
    const int c0 = min(V, tid * chunk), c1 = min(V, c0 + chunk);

    // 1) row maximum
    float m = -INFINITY;
    for (int c = c0; c < c1; ++c) m = fmaxf(m, row[c]);
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    __syncthreads();
    if ((tid & 63) == 0) shf[tid >> 6] = m;
    __syncthreads();
    for (int i = 0; i < (int)blockDim.x / 64; ++i) m = fmaxf(m, shf[i]);

    // 2) top-k threshold: the k-th largest key, by four 8-bit radix passes from the top.
    const bool topk = cfg.top_k > 0 && cfg.top_k < V;
    uint32_t thr = 0, ties_kept = 0;
    if (topk) {
        uint32_t prefix = 0, mask = 0, need = (uint32_t)cfg.top_k;
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int i = tid; i < 256; i += blockDim.x) hist256[i] = 0;
            __syncthreads();
            for (int c = c0; c < c1; ++c) {
                const uint32_t k = float_key(row[c]);
                if ((k & mask) == prefix) atomicAdd(&hist256[(k >> shift) & 255u], 1u);
            }
            __syncthreads();
            // The digit where the count from the largest digit down reaches `need`: wave 0,
            // lane l holding digits 4l..4l+3, a suffix scan over lanes, then the one lane
            // whose digits contain the crossing resolves it.
            if (tid < 64) {
                const int lane = tid;
                uint32_t c[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) c[t] = hist256[4 * lane + t];
                const uint32_t local = c[0] + c[1] + c[2] + c[3];
                uint32_t suf = local;  // counts of digits >= 4 lane
#pragma unroll
                for (int off = 1; off < 64; off <<= 1) {
                    const uint32_t y = __shfl_down(suf, off);
                    if (lane + off < 64) suf += y;
                }
                const uint32_t above = suf - local;  // counts of digits > 4 lane + 3
                if (above < need && need <= suf) {
                    uint32_t acc = above;
                    for (int t = 3; t >= 0; --t) {
                        if (acc + c[t] >= need) {
                            radix_sh[0] = (uint32_t)(4 * lane + t);
                            radix_sh[1] = need - acc;
                            break;
                        }
                        acc += c[t];
                    }
                }
            }
            __syncthreads();
            const uint32_t digit = radix_sh[0];
            need = radix_sh[1];
            prefix |= digit << shift;
            mask |= 255u << shift;
            __syncthreads();
        }
        thr = prefix;        // key of the k-th largest logit
        ties_kept = need;    // how many logits equal to it are kept (the lowest indices)
    }

    // 3) weights: tie ranks in index order, then per-chunk sums and their prefix.
    uint32_t my_ties = 0;
    if (topk)
        for (int c = c0; c < c1; ++c) my_ties += float_key(row[c]) == thr ? 1u : 0u;
    uint32_t ties_total;
    uint32_t tie_base = block_exclusive_scan<uint32_t>(my_ties, shu, &ties_total);
    auto weight = [&](int c, uint32_t& tie_rank) -> float {
        const float z = row[c];
        if (topk) {
            const uint32_t k = float_key(z);
            if (k < thr) return 0.0f;
            if (k == thr && tie_rank++ >= ties_kept) return 0.0f;
        }
        return expf((z - m) * cfg.inv_temp);
    };
    float part = 0.0f;
    {
        uint32_t tr = tie_base;
        for (int c = c0; c < c1; ++c) part += weight(c, tr);
    }
    float total;
    const float base = block_exclusive_scan<float>(part, shf, &total);

    // 4) inverse CDF at u * total.
    const int p = (st ? st->pos : pos_const) + 1;
    const float target = sample_uniform(cfg.seed, b, p) * total;
    if (tid == 0) {
        pick_sh[0] = 0x7fffffff;
        pick_sh[1] = -1;
    }
    __syncthreads();
    {
        uint32_t tr = tie_base;
        float acc = base;
        int found = -1, last = -1;
        for (int c = c0; c < c1; ++c) {
            const float w = weight(c, tr);
            if (w > 0.0f) last = c;
            acc += w;
            if (found < 0 && w > 0.0f && acc > target) found = c;
        }
        if (found >= 0) atomicMin(&pick_sh[0], found);
        if (last >= 0) atomicMax(&pick_sh[1], last);
    }
    __syncthreads();
    if (tid == 0) {
        // u * total can round up to total: the last kept index then.
        const int chosen = pick_sh[0] != 0x7fffffff ? pick_sh[0] : (pick_sh[1] >= 0 ? pick_sh[1] : 0);
        if (p < HS) hist[(size_t)b * HS + p] = chosen;
    }
}

// Saves this step's logits into slot st->gen of the history (B x V per slot).
__global__ void capture_logits_kernel(float* __restrict__ hist, size_t slots,
                                      const float* __restrict__ logits, size_t n,
                                      const DevState* st) {
    const int g = st->gen;
    if ((size_t)g >= slots) return;
    for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < n;
         e += (size_t)gridDim.x * blockDim.x)
        hist[(size_t)g * n + e] = logits[e];
}

// ---- fused batched-decode kernels (graph path, split-K products) -------------------------

constexpr int kRowNE = 16;  // row elements per lane of the one-wave-per-row kernels (C <= 1024)

// LayerNormOp of one row held in a wave (lane l: elements l + 64 m), written to y; the sums
// run in the same order as layernorm_kernel's, so the result is the same.
__device__ __forceinline__ void row_layernorm(const float (&v)[kRowNE], int C, const float* g,
                                              const float* bta, float* y) {
    const int lane = threadIdx.x & 63;
    const float inv_cols = 1.0f / (float)C;
    float s = 0.0f;
#pragma unroll
    for (int m = 0; m < kRowNE; ++m)
        if (lane + 64 * m < C) s += v[m];
    const float mean = wave_sum(s) * inv_cols;
    float q = 0.0f;
#pragma unroll
    for (int m = 0; m < kRowNE; ++m)
        if (lane + 64 * m < C) {
            const float d = v[m] - mean;
            q += d * d;
        }
    const float inv_std = 1.0f / sqrtf(wave_sum(q) * inv_cols + 1e-5f);
#pragma unroll
    for (int m = 0; m < kRowNE; ++m) {
        const int c = lane + 64 * m;
        if (c < C) y[c] = (v[m] - mean) * inv_std * g[c] + (bta ? bta[c] : 0.0f);
    }
}

// Decode step start: x[b] = tok[hist[b][pos]] + pos_emb[pos] (embed_kernel), xn[b] = LN0(x[b]).
// One wave (work-group) per row.
__global__ __launch_bounds__(64) void embed_ln_kernel(float* __restrict__ x, float* __restrict__ xn,
                                                      const int32_t* __restrict__ hist, int HS,
                                                      const DevState* st, const float* __restrict__ tok,
                                                      const float* __restrict__ pos_emb, int C,
                                                      const float* g, const float* bta) {
    const int lane = threadIdx.x;
    const int b = blockIdx.x;
    const int p = st->pos;
    const int id = hist[(size_t)b * HS + p];
    float v[kRowNE];
#pragma unroll
    for (int m = 0; m < kRowNE; ++m) {
        const int c = lane + 64 * m;
        v[m] = 0.0f;
        if (c < C) {
            v[m] = tok[(size_t)id * C + c] + pos_emb[(size_t)p * C + c];
            x[(size_t)b * C + c] = v[m];
        }
    }
    row_layernorm(v, C, g, bta, xn + (size_t)b * C);
}

// Split-K reduction of a residual projection fused with the next LayerNorm: for row r,
// x[r] += sum_z part[z][r] (splitk_reduce_kernel's order), then xn[r] = LN(x[r]) with the
// LayerNormOp formula (two-pass mean / variance).  One 256-thread work-group per row, thread t
// on columns t + 256 j; the partials of 8 splits are loaded together before they are added.
__global__ __launch_bounds__(256) void reduce_resid_ln_kernel(const float* __restrict__ part, int splits,
                                                              int M, int C, float* __restrict__ x,
                                                              float* __restrict__ xn, const float* g,
                                                              const float* bta) {
    constexpr int kZ = 8, kNJ = 64 * kRowNE / 256;  // columns per thread (C <= 1024)
    __shared__ float red[8];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int r = blockIdx.x;
    const size_t total = (size_t)M * C;
    const float* pr = part + (size_t)r * C;
    float xv[kNJ];  // the residual row, loaded with the first partials
#pragma unroll
    for (int j = 0; j < kNJ; ++j) {
        const int c = t + 256 * j;
        xv[j] = c < C ? x[(size_t)r * C + c] : 0.0f;
    }
    float acc[kNJ];
#pragma unroll
    for (int j = 0; j < kNJ; ++j) acc[j] = 0.0f;
    for (int z0 = 0; z0 < splits; z0 += kZ) {
        float pv[kZ][kNJ];
#pragma unroll
        for (int z = 0; z < kZ; ++z)
#pragma unroll
            for (int j = 0; j < kNJ; ++j) {
                const int c = t + 256 * j;
                pv[z][j] = (z0 + z < splits && c < C) ? pr[(size_t)(z0 + z) * total + c] : 0.0f;
            }
#pragma unroll
        for (int z = 0; z < kZ; ++z)
#pragma unroll
            for (int j = 0; j < kNJ; ++j)
                if (z0 + z < splits) acc[j] += pv[z][j];
    }
    float v[kNJ];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kNJ; ++j) {
        const int c = t + 256 * j;
        v[j] = 0.0f;
        if (c < C) {
            v[j] = xv[j] + acc[j];
            x[(size_t)r * C + c] = v[j];
            s += v[j];
        }
    }
    const float inv_cols = 1.0f / (float)C;
    s = wave_sum(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    const float mean = ((red[0] + red[1]) + (red[2] + red[3])) * inv_cols;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < kNJ; ++j)
        if (t + 256 * j < C) {
            const float d = v[j] - mean;
            q += d * d;
        }
    q = wave_sum(q);
    if (lane == 0) red[4 + wave] = q;
    __syncthreads();
    const float inv_std = 1.0f / sqrtf(((red[4] + red[5]) + (red[6] + red[7])) * inv_cols + 1e-5f);
    float* y = xn + (size_t)r * C;
#pragma unroll
    for (int j = 0; j < kNJ; ++j) {
        const int c = t + 256 * j;
        if (c < C) y[c] = (v[j] - mean) * inv_std * g[c] + (bta ? bta[c] : 0.0f);
    }
}

// reduce_resid_ln_kernel for many rows and two partials (the prefill's residual projections):
// one wave per row, lane on the float2 at columns 2 lane + 128 j, so a 384-wide row keeps
// every lane busy (the work-group-per-row form leaves 5/8 of its threads idle there).  Same
// formula; the mean and variance are summed in another order.
__global__ __launch_bounds__(256) void resid_ln2_rows_kernel(const float* __restrict__ part, int M, int C,
                                                             float* __restrict__ x, float* __restrict__ xn,
                                                             const float* __restrict__ g,
                                                             const float* __restrict__ bta) {
    constexpr int kJ = kRowNE / 2;  // float2 per lane (C <= 1024)
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= M) return;
    // gamma / beta requested with the row (not after its statistics: one round trip less);
    // 8-byte loads where the caller's pointers allow them.
    float2 gg[kJ], bb[kJ];
    const bool pair_ok = ((uintptr_t)g % 8 == 0) && (bta == nullptr || (uintptr_t)bta % 8 == 0);
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
        const int c2 = lane + 64 * j;
        gg[j] = bb[j] = make_float2(0.0f, 0.0f);
        if (2 * c2 < C) {
            if (pair_ok) {
                gg[j] = reinterpret_cast<const float2*>(g)[c2];
                if (bta) bb[j] = reinterpret_cast<const float2*>(bta)[c2];
            } else {
                gg[j] = make_float2(g[2 * c2], g[2 * c2 + 1]);
                if (bta) bb[j] = make_float2(bta[2 * c2], bta[2 * c2 + 1]);
            }
        }
    }
    const size_t total = (size_t)M * C;
    const float2* xr = reinterpret_cast<const float2*>(x + (size_t)r * C);
    const float2* p0 = reinterpret_cast<const float2*>(part + (size_t)r * C);
    const float2* p1 = reinterpret_cast<const float2*>(part + total + (size_t)r * C);
    float2 v[kJ];
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
        const int c2 = lane + 64 * j;
        v[j] = make_float2(0.0f, 0.0f);
        if (2 * c2 < C) {
            const float2 a = xr[c2], b = p0[c2], d = p1[c2];
            v[j].x = a.x + (b.x + d.x);
            v[j].y = a.y + (b.y + d.y);
            s += v[j].x + v[j].y;
        }
    }
    float2* xw = reinterpret_cast<float2*>(x + (size_t)r * C);
#pragma unroll
    for (int j = 0; j < kJ; ++j)
        if (2 * (lane + 64 * j) < C) xw[lane + 64 * j] = v[j];
    const float inv_cols = 1.0f / (float)C;
    const float mean = wave_sum(s) * inv_cols;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < kJ; ++j)
        if (2 * (lane + 64 * j) < C) {
            const float dx = v[j].x - mean, dy = v[j].y - mean;
            q += dx * dx + dy * dy;
        }
    const float inv_std = 1.0f / sqrtf(wave_sum(q) * inv_cols + 1e-5f);
    float2* y = reinterpret_cast<float2*>(xn + (size_t)r * C);
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
        const int c2 = lane + 64 * j;
        if (2 * c2 < C)
            y[c2] = make_float2((v[j].x - mean) * inv_std * gg[j].x + bb[j].x,
                                (v[j].y - mean) * inv_std * gg[j].y + bb[j].y);
    }
}

__global__ void advance_kernel(DevState* st) {
    st->pos += 1;
    st->gen += 1;
}

__global__ void set_state_kernel(DevState* st, int pos, int gen) {
    st->pos = pos;
    st->gen = gen;
}

// Projection weights with one output per row (N x K): W_qkv, W_fc and W_proj2 transposed from
// the reference's C x 3C, C x 4C and 4C x C (Dense_Weights, Mul<None>); the attention output
// projection is stored that way already (Dense_Transposed, Mul<Right>).
struct LayerW {
    const float *wqkvT, *wproj, *wfcT, *w2T, *ln0g, *ln0b, *ln1g, *ln1b;
};

}  // namespace
}  // namespace fmlh

using namespace fmlh;

struct fmlh_nanollm {
    fmlh_nanollm_config cfg{};
    int V = 0, T = 0, C = 0, H = 0, L = 0, hd = 0, Bmax = 0;
    int HS = 0;  // token-history row stride: block_size + 1 (the token chosen at position T-1)
    float scale = 0.f;
    const float *tok = nullptr, *pos = nullptr, *lnf_g = nullptr, *lnf_b = nullptr, *lm = nullptr;
    std::vector<LayerW> layers;
    // weights_on_device: the caller's W_qkv, W_fc, W_proj2 of each layer (sources of the
    // transposed copies, re-taken by fmlh_nanollm_refresh_weights); empty for host weights.
    std::vector<const float*> t_src;
    std::vector<void*> owned;
    float *kc = nullptr, *vc = nullptr;
    float *x = nullptr, *xn = nullptr, *qkv = nullptr, *y = nullptr, *h = nullptr;
    float *xlast = nullptr, *logits = nullptr;
    int32_t* hist = nullptr;
    int32_t* hist_host = nullptr;  // pinned staging of the prompt history, [Bmax][HS]
    // Extra streams of the fused prefill (default priority) and their fork / join events.
    static constexpr int kPrefillParts = 4;
    hipStream_t s2[kPrefillParts - 1] = {};
    hipEvent_t ev_fork = nullptr, ev_join[kPrefillParts - 1] = {};
    DevState* st = nullptr;
    float* ws = nullptr;
    size_t ws_elems = 0;
    float* attn_ws = nullptr;
    float* logit_hist = nullptr;
    size_t logit_hist_slots = 0;
    uint32_t batch = 0, prompt_len = 0, generated = 0;
    bool prefilled = false;
    hipGraphExec_t graph[2] = {nullptr, nullptr};  // [capture logits?]
    uint32_t graph_batch[2] = {0, 0};
    bool use_graph = true;
    // Sampling (fmlh_nanollm_set_sampling): temperature 0 = greedy.
    float temperature = 0.0f;
    uint32_t top_k = 0;
    unsigned long long seed = 0;
    // Persistent decode (decode_persistent.hip): weight copies with one output per row,
    // exchange words, error flag, and the next launch's first epoch.
    bool persist = false;
    PersistLayer* d_players = nullptr;
    uint64_t *x_q = nullptr, *x_kn = nullptr, *x_vn = nullptr, *x_att = nullptr, *x_dx1 = nullptr,
             *x_hb = nullptr, *x_dx2 = nullptr, *x_am = nullptr;
    unsigned* d_err = nullptr;
    unsigned long long* d_trace = nullptr;  // FMLH_PERSIST_TRACE=<file>: per-WG timelines
    std::string d_trace_path;               // <file>, as set when the engine was created
    uint32_t epoch = 1;
    int persist_G = 0, persist_chunks = 0, persist_groups = 0;  // exchange buffers sized for these
    // Grouped decode (decode_grouped.hip): batches of more than one group of sequences.
    bool grouped = false;
    int grouped_groups = 0;   // exchange buffers hold this many groups
    size_t grouped_gw[2] = {0, 0};
    uint64_t *g_qkv = nullptr, *g_y = nullptr, *g_dx1 = nullptr, *g_part = nullptr, *g_dx2 = nullptr,
             *g_am = nullptr;
    unsigned long long* g_trace = nullptr;  // FMLH_GROUPED_TRACE=<file>: per-WG timelines
    std::string g_trace_path;
    unsigned long long* r_trace = nullptr;  // FMLH_RELAY_TRACE=<file>: per-role timelines
    std::string r_trace_path;
    int r_roles = 0;                 // the trace holds this many roles (the largest plan's)
    int r_last_roles = 0, r_last_nq = 0, r_last_nf = 0, r_last_nf2 = 0, r_last_nA = 1, r_last_nlm = 1;  // plan of the last relay launch
    size_t persist_gw[5] = {0, 0, 0, 0, 0};                          // per-group words (see PersistArgs)
    // Relay decode (decode_relay.hip): one sequence, a team of workgroups per product.
    bool relay = false;
    int r_bmax = 0;  // sequences the relay exchange buffers hold
    uint64_t *r_x = nullptr, *r_part = nullptr, *r_qkv = nullptr, *r_dx1 = nullptr, *r_xp = nullptr;
    // Wide decode (decode_wide.hip): up to 8 sequences of shapes the kernels above refuse.
    bool wide = false;
    WideLayer* d_wlayers = nullptr;
    std::vector<float*> w2;  // per layer: W_proj2 as 4C x C (the column split reads its rows)
    uint64_t *w_q = nullptr, *w_part = nullptr, *w_y = nullptr, *w_dx1 = nullptr, *w_p2 = nullptr,
             *w_dx2 = nullptr, *w_cand = nullptr, *w_h = nullptr;
    unsigned long long* w_trace = nullptr;  // FMLH_WIDE_TRACE=<file>: per-WG timeline of a step
    std::string w_trace_path;
    // Every exchange buffer of the decode kernels with its word count: cleared together when the
    // epoch count would wrap (reserve_epochs).
    std::vector<std::pair<uint64_t*, size_t>> xbufs;
};

namespace {

// Live engines, so that fmlh_shutdown can release them and a stale handle is refused.
std::mutex g_engines_mu;
std::unordered_set<fmlh_nanollm*> g_engines;

int alloc(fmlh_nanollm* m, void** p, size_t bytes) {
    FMLH_TRY(device_malloc(p, bytes ? bytes : 4));
    m->owned.push_back(*p);
    return FMLH_OK;
}

template <class Tp>
int alloc_t(fmlh_nanollm* m, Tp** p, size_t count) {
    void* v = nullptr;
    FMLH_TRY(alloc(m, &v, count * sizeof(Tp)));
    *p = static_cast<Tp*>(v);
    return FMLH_OK;
}

int upload(fmlh_nanollm* m, const float* src, size_t count, int on_device, const float** dst) {
    if (!src) { *dst = nullptr; return FMLH_OK; }
    if (on_device) { *dst = src; return FMLH_OK; }
    float* d = nullptr;
    FMLH_TRY(alloc_t(m, &d, count));
    FMLH_HIP(hipMemcpy(d, src, count * sizeof(float), hipMemcpyHostToDevice));
    *dst = d;
    return FMLH_OK;
}

// rows x cols weight (host or device) -> an engine-owned cols x rows copy on the device.
int upload_transposed(fmlh_nanollm* m, const float* src, int rows, int cols, int on_device,
                      const float** dst) {
    const size_t n = (size_t)rows * cols;
    const float* d_src = src;
    float* staged = nullptr;
    if (!on_device) {
        FMLH_TRY(device_malloc(reinterpret_cast<void**>(&staged), n * sizeof(float)));
        if (hipMemcpy(staged, src, n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipFree(staged);
            return set_error(FMLH_E_HIP, "upload_transposed: copy to device failed");
        }
        d_src = staged;
    }
    float* t = nullptr;
    int rc = alloc_t(m, &t, n);
    if (rc == FMLH_OK) rc = persist_transpose(t, d_src, rows, cols, stream());
    if (staged) {
        (void)hipStreamSynchronize(stream());
        (void)hipFree(staged);
    }
    *dst = t;
    return rc;
}

void release(fmlh_nanollm* m) {
    for (auto& g : m->graph)
        if (g) { (void)hipGraphExecDestroy(g); g = nullptr; }
    for (void* p : m->owned) (void)hipFree(p);
    m->owned.clear();
    if (m->hist_host) (void)hipHostFree(m->hist_host);
    m->hist_host = nullptr;
    if (m->ev_fork) (void)hipEventDestroy(m->ev_fork);
    m->ev_fork = nullptr;
    for (int i = 0; i < fmlh_nanollm::kPrefillParts - 1; ++i) {
        if (m->ev_join[i]) (void)hipEventDestroy(m->ev_join[i]);
        if (m->s2[i]) (void)hipStreamDestroy(m->s2[i]);
        m->ev_join[i] = nullptr;
        m->s2[i] = nullptr;
    }
}

// Split-K workspace for the five projections at M rows.
size_t gemm_ws_for(const fmlh_nanollm* m, int M) {
    const int C = m->C;
    size_t w = 0;
    w = std::max(w, plan_gemm(M, 3 * C, C, 1).ws_elems);
    w = std::max(w, plan_gemm(M, C, C, 1).ws_elems);
    w = std::max(w, plan_gemm(M, 4 * C, C, 1).ws_elems);
    w = std::max(w, plan_gemm(M, C, 4 * C, 1).ws_elems);
    w = std::max(w, plan_gemm(M, m->V, C, 1).ws_elems);  // lm_head
    return w;
}

int ensure_ws(fmlh_nanollm* m, size_t elems) {
    if (elems <= m->ws_elems) return FMLH_OK;
    if (m->ws) {
        FMLH_HIP(hipStreamSynchronize(stream()));
        for (auto& p : m->owned)
            if (p == m->ws) p = nullptr;
        (void)hipFree(m->ws);
        // No workspace until the new one exists: a failed allocation leaves the engine without
        // one (the next call allocates again), never with the freed address.
        m->ws = nullptr;
        m->ws_elems = 0;
    }
    // Captured decode graphs hold the old workspace address.
    for (auto& g : m->graph)
        if (g) { (void)hipGraphExecDestroy(g); g = nullptr; }
    FMLH_TRY(alloc_t(m, &m->ws, elems));
    m->ws_elems = elems;
    return FMLH_OK;
}

// ln_g != nullptr: A holds rows before a LayerNorm (gamma ln_g, beta ln_b) that the product
// applies to them itself (gemm_takes_ln shapes only).
int proj(fmlh_nanollm* m, const float* A, int lda, const float* W, int ldw, int trans, float* Cout,
         int ldc, int M, int N, int K, int epi, const float* R, int ldr, const float* ln_g = nullptr,
         const float* ln_b = nullptr) {
    GemmArgs g;
    g.A = A; g.lda = lda; g.B = W; g.ldb = ldw; g.b_trans = trans;
    g.C = Cout; g.ldc = ldc; g.M = M; g.N = N; g.K = K; g.epi = epi; g.R = R; g.ldr = ldr;
    g.ln_g = ln_g; g.ln_b = ln_b; g.ln_eps = 1e-5f;
    g.s = stream();
    return gemm(g, m->ws, m->ws_elems);
}

// Whether a product of `rows` rows of x (K = C) by N weight rows applies its LayerNorm inside
// the skinny kernel (no LayerNorm launch, no normalised copy).  Every work-group of the product
// forms the rows' statistics itself, so a wide product (c4's 50304-row lm_head: 12576
// work-groups) keeps the separate LayerNorm.  FMLH_LN_IN_GEMV=0 turns it off, =1 on for any N.
bool ln_in_gemv(const fmlh_nanollm* m, int rows, int N) {
    const char* e = std::getenv("FMLH_LN_IN_GEMV");
    if (e && e[0] == '0') return false;
    if (!(e && e[0] == '1') && N > 4096) return false;
    return gemm_takes_ln(rows, N, m->C, 1);
}

// Whether a decode step of `batch` rows runs the fused graph path: every residual / QKV
// projection splits K, so its reduction can carry the next op (LayerNorm, cache write).
bool decode_fused(const fmlh_nanollm* m, int batch) {
    const int C = m->C;
    if (C > 64 * kRowNE) return false;
    const int shapes[3][2] = {{3 * C, C}, {C, C}, {C, 4 * C}};
    for (const auto& nk : shapes) {
        const GemmPlan p = plan_gemm(batch, nk[0], nk[1], 1);
        if (p.kind != GemmPlan::kMfma || p.splits < 2) return false;
    }
    return true;
}

int split_partials(fmlh_nanollm* m, const float* A, int lda, const float* W, int ldw, int M, int N,
                   int K, int* splits) {
    GemmArgs g;
    g.A = A; g.lda = lda; g.B = W; g.ldb = ldw; g.b_trans = 1;
    g.M = M; g.N = N; g.K = K;
    g.s = stream();
    FMLH_TRY(gemm_split_partials(g, m->ws, m->ws_elems, splits));
    FMLH_REQUIRE(*splits > 1, "fused decode: product %dx%dx%d does not split", M, N, K);
    return FMLH_OK;
}

// Fused-path QKV of layer l on M rows of xn: the split partials only (m->ws); the attention
// kernel adds them up (q) and writes this step's K / V rows to the caches.
int fused_qkv(fmlh_nanollm* m, int l, int M, int* splits) {
    const int C = m->C;
    return split_partials(m, m->xn, C, m->layers[l].wqkvT, C, M, 3 * C, C, splits);
}

// Fused-path residual projection: x += A W^T (K-long rows of A), then xn = LN(x; g, bta).
int fused_resid_ln(fmlh_nanollm* m, const float* A, const float* W, int K, int M, const float* g,
                   const float* bta) {
    const int C = m->C;
    int sp = 0;
    FMLH_TRY(split_partials(m, A, K, W, K, M, C, K, &sp));
    hipLaunchKernelGGL(reduce_resid_ln_kernel, dim3(M), dim3(256), 0, stream(), m->ws, sp, M, C, m->x,
                       m->xn, g, bta);
    FMLH_LAUNCHED("reduce_resid_ln_kernel");
    return FMLH_OK;
}

// Decode step on the fused path (batch rows at position st->pos; xn already holds LN0(x) of
// layer 0): per layer QKV partials -> attention (adds them up, writes the step's K / V rows
// to the caches), proj partials ->
// reduce + residual + LN1, FC + GELU, proj2 partials -> reduce + residual + LN0 of the next
// layer (ln_f after the last), leaving xn ready for the lm_head.
int run_blocks_decode_fused(fmlh_nanollm* m, int batch) {
    const int C = m->C, M = batch;
    for (int l = 0; l < m->L; ++l) {
        const LayerW& w = m->layers[l];
        const size_t lofs = (size_t)l * m->Bmax * m->H * m->T * m->hd;
        int sp = 0;
        FMLH_TRY(fused_qkv(m, l, M, &sp));
        FMLH_TRY(attn_decode(m->ws, 3 * C, m->kc + lofs, m->vc + lofs, m->y, C, batch, m->H, m->hd,
                             m->T, &m->st->pos, m->scale, m->attn_ws, m->Bmax, stream(), sp));
        FMLH_TRY(fused_resid_ln(m, m->y, w.wproj, C, M, w.ln1g, w.ln1b));
        FMLH_TRY(proj(m, m->xn, C, w.wfcT, C, 1, m->h, 4 * C, M, 4 * C, C, kEpiGelu, nullptr, 0));
        const bool last = l + 1 == m->L;
        FMLH_TRY(fused_resid_ln(m, m->h, w.w2T, 4 * C, M, last ? m->lnf_g : m->layers[l + 1].ln0g,
                                last ? m->lnf_b : m->layers[l + 1].ln0b));
    }
    return FMLH_OK;
}

// Whether a prefill of M rows runs its residual projections as two K halves whose reduction
// adds the residual and applies the next LayerNorm (reduce_resid_ln_kernel: no LayerNorm
// launches, and the attention projection's grid no longer leaves CUs idle).  Only where that
// grid has fewer than two 64 x 64 tiles per CU (c3): with more, the halves' extra partial
// traffic costs what the LayerNorm launches save.  FMLH_PREFILL_FUSED=0 turns it off, =1 on.
bool prefill_fused(const fmlh_nanollm* m, int M) {
    const int C = m->C;
    const char* e = std::getenv("FMLH_PREFILL_FUSED");
    if (e && e[0] == '0') return false;
    if (C > 64 * kRowNE || C % 32 != 0) return false;
    const long tiles = (long)((M + 63) / 64) * ((C + 63) / 64);
    if (!(e && e[0] == '1') && tiles >= 2L * cu_count()) return false;
    GemmArgs g;
    g.A = m->y; g.lda = C; g.B = m->layers[0].wproj; g.ldb = C; g.b_trans = 1; g.M = M; g.N = C; g.K = C;
    if (!gemm_runs_nt(g)) return false;
    g.A = m->h; g.lda = 4 * C; g.B = m->layers[0].w2T; g.ldb = 4 * C; g.K = 4 * C;
    return gemm_runs_nt(g);
}

// Prefill residual projection in two K halves (partials in ws, 2 M C floats), then
// x += both halves and xn = LN(x; g, bta), on M rows.
int prefill_resid_ln(int C, const float* A, const float* W, int K, int M, float* x, float* xn, const float* g,
                     const float* bta, float* ws, hipStream_t s) {
    GemmArgs ga;
    ga.A = A; ga.lda = K; ga.B = W; ga.ldb = K; ga.b_trans = 1; ga.M = M; ga.N = C; ga.K = K;
    ga.s = s;
    FMLH_TRY(gemm_nt_partials(ga, 2, ws, (size_t)2 * M * C));
    hipLaunchKernelGGL(resid_ln2_rows_kernel, dim3((M + 3) / 4), dim3(256), 0, s, ws, M, C, x, xn, g, bta);
    FMLH_LAUNCHED("resid_ln2_rows_kernel");
    return FMLH_OK;
}

// Workspace floats one part of a fused prefill takes for Mp rows: the residual projections'
// two K halves (2 Mp C) or whatever the QKV and FC products plan at Mp rows (a part can be
// small enough for them to split K), whichever is larger.
size_t fused_part_ws(const fmlh_nanollm* m, int Mp) {
    const int C = m->C;
    return std::max({(size_t)2 * Mp * C, plan_gemm(Mp, 3 * C, C, 1).ws_elems, plan_gemm(Mp, 4 * C, C, 1).ws_elems});
}

// Layer l (l = -1: LN0 of layer 0) of a fused prefill (prefill_fused) for sequences b0 ..
// b0 + nb - 1 of P rows each, on stream s, with ws (ws_cap >= fused_part_ws(m, nb P) floats)
// for the partial sums: the rows, cache entries and partials of these sequences only, so
// disjoint ranges can run on different streams at once.  x holds the embeddings before layer
// -1; xn holds ln_f(x) of every row after the last layer.
int prefill_seqs_layer(fmlh_nanollm* m, int l, int b0, int nb, int P, hipStream_t s, float* ws, size_t ws_cap) {
    const int C = m->C, M = nb * P;
    const size_t r0 = (size_t)b0 * P;
    float* x = m->x + r0 * C;
    float* xn = m->xn + r0 * C;
    float* qkv = m->qkv + r0 * 3 * C;
    float* y = m->y + r0 * C;
    float* h = m->h + r0 * 4 * C;
    const size_t kv0 = (size_t)b0 * m->H * m->T * m->hd;
    if (l < 0) return layernorm_rows(xn, x, m->layers[0].ln0g, m->layers[0].ln0b, nullptr, M, C, 1e-5f, s);
    {
        const LayerW& w = m->layers[l];
        const size_t lofs = (size_t)l * m->Bmax * m->H * m->T * m->hd;
        float* kc = m->kc + lofs + kv0;
        float* vc = m->vc + lofs + kv0;
        GemmArgs g;
        g.A = xn; g.lda = C; g.B = w.wqkvT; g.ldb = C; g.b_trans = 1;
        g.C = qkv; g.ldc = 3 * C; g.M = M; g.N = 3 * C; g.K = C; g.s = s;
        if (gemm_runs_nt(g)) {  // K / V columns written straight into the caches
            g.epi = kEpiKV;
            g.kv.kc = kc; g.kv.vc = vc; g.kv.C = C; g.kv.H = m->H; g.kv.hd = m->hd; g.kv.T = m->T;
            g.kv.rows_per_seq = P;
            FMLH_TRY(gemm(g, ws, ws_cap));
        } else {
            FMLH_TRY(gemm(g, ws, ws_cap));
            FMLH_TRY(kv_scatter(qkv, 3 * C, kc, vc, M, P, C, m->H, m->T, nullptr, 0, s));
        }
        FMLH_TRY(attn_prefill(qkv, 3 * C, kc, vc, y, C, nb, P, m->H, m->hd, m->T, m->scale, s));
        FMLH_TRY(prefill_resid_ln(C, y, w.wproj, C, M, x, xn, w.ln1g, w.ln1b, ws, s));
        GemmArgs f;
        f.A = xn; f.lda = C; f.B = w.wfcT; f.ldb = C; f.b_trans = 1;
        f.C = h; f.ldc = 4 * C; f.M = M; f.N = 4 * C; f.K = C; f.epi = kEpiGelu; f.s = s;
        FMLH_TRY(gemm(f, ws, ws_cap));
        const bool last = l + 1 == m->L;
        FMLH_TRY(prefill_resid_ln(C, h, w.w2T, 4 * C, M, x, xn, last ? m->lnf_g : m->layers[l + 1].ln0g,
                                  last ? m->lnf_b : m->layers[l + 1].ln0b, ws, s));
    }
    return FMLH_OK;
}

int prefill_seqs(fmlh_nanollm* m, int b0, int nb, int P, hipStream_t s, float* ws, size_t ws_cap) {
    for (int l = -1; l < m->L; ++l) FMLH_TRY(prefill_seqs_layer(m, l, b0, nb, P, s, ws, ws_cap));
    return FMLH_OK;
}

// The blocks on `rows` rows per sequence (prefill: the prompt; decode: 1 row at *st->pos).
int run_blocks(fmlh_nanollm* m, int batch, int rows, bool decode) {
    const int C = m->C, M = batch * rows;
    hipStream_t s = stream();
    for (int l = 0; l < m->L; ++l) {
        const LayerW& w = m->layers[l];
        const size_t lofs = (size_t)l * m->Bmax * m->H * m->T * m->hd;
        float* kc = m->kc + lofs;
        float* vc = m->vc + lofs;
        // decode on <= 8 rows: LN0 / LN1 applied by the products that read them
        const bool ln_qkv = decode && ln_in_gemv(m, M, 3 * C), ln_fc = decode && ln_in_gemv(m, M, 4 * C);
        if (!ln_qkv) FMLH_TRY(layernorm_rows(m->xn, m->x, w.ln0g, w.ln0b, nullptr, M, C, 1e-5f, s));
        GemmArgs g;
        g.A = ln_qkv ? m->x : m->xn; g.lda = C; g.B = w.wqkvT; g.ldb = C; g.b_trans = 1;
        g.C = m->qkv; g.ldc = 3 * C; g.M = M; g.N = 3 * C; g.K = C; g.s = s;
        if (ln_qkv) {
            g.ln_g = w.ln0g;
            g.ln_b = w.ln0b;
        }
        if (!decode && gemm_runs_nt(g)) {
            // prefill: K / V columns written straight into the caches (positions 0..rows-1)
            g.epi = kEpiKV;
            g.kv.kc = kc; g.kv.vc = vc; g.kv.C = C; g.kv.H = m->H; g.kv.hd = m->hd; g.kv.T = m->T;
            g.kv.rows_per_seq = rows;
            FMLH_TRY(gemm(g, m->ws, m->ws_elems));
        } else {
            FMLH_TRY(gemm(g, m->ws, m->ws_elems));
            // decode: the attention kernel writes this step's K / V rows to the caches itself
            // (the QKV product read as one split)
            if (!decode) FMLH_TRY(kv_scatter(m->qkv, 3 * C, kc, vc, M, rows, C, m->H, m->T, nullptr, 0, s));
        }
        if (decode) {
            FMLH_TRY(attn_decode(m->qkv, 3 * C, kc, vc, m->y, C, batch, m->H, m->hd, m->T,
                                 &m->st->pos, m->scale, m->attn_ws, m->Bmax, s, 1));
        } else {
            FMLH_TRY(attn_prefill(m->qkv, 3 * C, kc, vc, m->y, C, batch, rows, m->H, m->hd, m->T,
                                  m->scale, s));
        }
        FMLH_TRY(proj(m, m->y, C, w.wproj, C, 1, m->x, C, M, C, C, kEpiResid, m->x, C));
        if (ln_fc) {
            FMLH_TRY(proj(m, m->x, C, w.wfcT, C, 1, m->h, 4 * C, M, 4 * C, C, kEpiGelu, nullptr, 0, w.ln1g,
                          w.ln1b));
        } else {
            FMLH_TRY(layernorm_rows(m->xn, m->x, w.ln1g, w.ln1b, nullptr, M, C, 1e-5f, s));
            FMLH_TRY(proj(m, m->xn, C, w.wfcT, C, 1, m->h, 4 * C, M, 4 * C, C, kEpiGelu, nullptr, 0));
        }
        FMLH_TRY(proj(m, m->h, 4 * C, w.w2T, 4 * C, 1, m->x, C, M, C, 4 * C, kEpiResid, m->x, C));
    }
    return FMLH_OK;
}

// ln_f + lm_head on `batch` rows of `src` (src == nullptr: xn already holds ln_f of them), then
// the device argmax into the history.
int head_and_pick(fmlh_nanollm* m, const float* src, int batch, bool decode, int pos_const,
                  bool src_normalized = false) {
    hipStream_t s = stream();
    if (src_normalized) {  // src already holds ln_f of the rows
        FMLH_TRY(proj(m, src, m->C, m->lm, m->C, 1, m->logits, m->V, batch, m->V, m->C, kEpiNone, nullptr, 0));
    } else if (src && ln_in_gemv(m, batch, m->V)) {  // ln_f applied by the lm_head product
        FMLH_TRY(proj(m, src, m->C, m->lm, m->C, 1, m->logits, m->V, batch, m->V, m->C, kEpiNone, nullptr, 0,
                      m->lnf_g, m->lnf_b));
    } else {
        if (src) FMLH_TRY(layernorm_rows(m->xn, src, m->lnf_g, m->lnf_b, nullptr, batch, m->C, 1e-5f, s));
        FMLH_TRY(proj(m, m->xn, m->C, m->lm, m->C, 1, m->logits, m->V, batch, m->V, m->C, kEpiNone,
                      nullptr, 0));
    }
    if (m->temperature > 0.0f) {
        const SampleCfg cfg{1.0f / m->temperature, (int)m->top_k, m->seed};
        hipLaunchKernelGGL(sample_hist_kernel, dim3(batch), dim3(kArgmaxThreads), 0, s, m->hist, m->HS, m->logits,
                           m->V, decode ? m->st : nullptr, pos_const, cfg);
        FMLH_LAUNCHED("sample_hist_kernel");
        return FMLH_OK;
    }
    hipLaunchKernelGGL(argmax_hist_kernel, dim3(batch), dim3(kArgmaxThreads), 0, s, m->hist, m->HS, m->logits,
                       m->V, decode ? m->st : nullptr, pos_const);
    FMLH_LAUNCHED("argmax_hist_kernel");
    return FMLH_OK;
}

int enqueue_decode_step(fmlh_nanollm* m, bool capture_logits) {
    hipStream_t s = stream();
    const int B = (int)m->batch;
    const size_t n = (size_t)B * m->C;
    if (decode_fused(m, B)) {
        hipLaunchKernelGGL(embed_ln_kernel, dim3(B), dim3(64), 0, s, m->x, m->xn, m->hist, m->HS, m->st,
                           m->tok, m->pos, m->C, m->layers[0].ln0g, m->layers[0].ln0b);
        FMLH_LAUNCHED("embed_ln_kernel");
        FMLH_TRY(run_blocks_decode_fused(m, B));
        FMLH_TRY(head_and_pick(m, nullptr, B, true, 0));
    } else {
        hipLaunchKernelGGL(embed_kernel, dim3(blocks_for(n, 256, 2048u)), dim3(256), 0, s, m->x, m->hist,
                           m->HS, 1, 0, m->st, m->tok, m->pos, m->C, B);
        FMLH_LAUNCHED("embed_kernel");
        FMLH_TRY(run_blocks(m, B, 1, true));
        FMLH_TRY(head_and_pick(m, m->x, B, true, 0));
    }
    if (capture_logits) {
        const size_t nl = (size_t)B * m->V;
        hipLaunchKernelGGL(capture_logits_kernel, dim3(blocks_for(nl, 256, 1024u)), dim3(256), 0, s,
                           m->logit_hist, m->logit_hist_slots, m->logits, nl, m->st);
        FMLH_LAUNCHED("capture_logits_kernel");
    }
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, s, m->st);
    FMLH_LAUNCHED("advance_kernel");
    return FMLH_OK;
}

int build_graph(fmlh_nanollm* m, int which) {
    if (m->graph[which] && m->graph_batch[which] == m->batch) return FMLH_OK;
    if (m->graph[which]) {
        (void)hipGraphExecDestroy(m->graph[which]);
        m->graph[which] = nullptr;
    }
    hipStream_t s = stream();
    FMLH_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int rc = enqueue_decode_step(m, which == 1);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(s, &g);
    if (rc != FMLH_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture", __FILE__, __LINE__);
    e = hipGraphInstantiate(&m->graph[which], g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate", __FILE__, __LINE__);
    m->graph_batch[which] = m->batch;
    return FMLH_OK;
}

int ensure_logit_hist(fmlh_nanollm* m, size_t slots) {
    if (m->logit_hist && m->logit_hist_slots >= slots) return FMLH_OK;
    if (m->logit_hist) {
        FMLH_HIP(hipStreamSynchronize(stream()));
        (void)hipFree(m->logit_hist);
        for (auto& p : m->owned)
            if (p == m->logit_hist) p = nullptr;
        m->logit_hist = nullptr;
    }
    FMLH_TRY(alloc_t(m, &m->logit_hist, slots * m->Bmax * (size_t)m->V));
    m->logit_hist_slots = slots;
    // The decode graphs with logits capture baked in the old buffer.
    if (m->graph[1]) { (void)hipGraphExecDestroy(m->graph[1]); m->graph[1] = nullptr; }
    return FMLH_OK;
}

// Device table of each layer's weights as the persistent kernels read them.
int setup_layer_table(fmlh_nanollm* m) {
    if (m->d_players) return FMLH_OK;
    std::vector<PersistLayer> pl(m->L);
    for (int l = 0; l < m->L; ++l) {
        const LayerW& w = m->layers[l];
        pl[l] = PersistLayer{w.wqkvT, w.wproj, w.wfcT, w.w2T, w.ln0g, w.ln0b, w.ln1g, w.ln1b};
    }
    FMLH_TRY(alloc_t(m, &m->d_players, (size_t)m->L));
    FMLH_HIP(hipMemcpy(m->d_players, pl.data(), pl.size() * sizeof(PersistLayer), hipMemcpyHostToDevice));
    return FMLH_OK;
}

// Exchange buffers for the persistent decode kernel.
int setup_persistent(fmlh_nanollm* m) {
    const char* env = std::getenv("FMLH_DECODE");
    if (env && std::strcmp(env, "graph") == 0) return FMLH_OK;
    const PersistPlan p = persist_plan(1, m->C, m->H, m->L, m->V, m->T, cu_count());
    if (!p.ok) return FMLH_OK;
    hipStream_t s = stream();
    const size_t C = m->C, B = m->Bmax;
    FMLH_TRY(setup_layer_table(m));
    // Exchange buffers: one slice per group of up to kMaxPersistBatch sequences, for as many
    // groups as max_batch needs (the plan for one sequence has the most WGs per group).
    m->persist_G = p.G;
    m->persist_chunks = p.max_chunks;
    const size_t Bp = std::min<size_t>(B, (size_t)kMaxPersistBatch * kMaxPersistGroups);
    m->persist_groups = (int)((Bp + kMaxPersistBatch - 1) / kMaxPersistBatch);
    persist_group_words((int)C, m->H, m->hd, p.max_chunks, p.G, (int)std::min<size_t>(Bp, kMaxPersistBatch),
                        m->persist_gw);
    const size_t ng = m->persist_groups;
    const size_t* gw = m->persist_gw;
    uint64_t** bufs[] = {&m->x_q, &m->x_kn, &m->x_vn, &m->x_att, &m->x_dx1, &m->x_hb, &m->x_dx2, &m->x_am};
    const size_t sizes[] = {ng * gw[0], ng * gw[0], ng * gw[0], ng * gw[1], ng * gw[2], ng * gw[3],
                            ng * gw[2], ng * gw[4]};
    for (int i = 0; i < 8; ++i) {
        FMLH_TRY(alloc_t(m, bufs[i], sizes[i]));
        FMLH_HIP(hipMemsetAsync(*bufs[i], 0, sizes[i] * sizeof(uint64_t), s));  // epoch 0: never current
        m->xbufs.emplace_back(*bufs[i], sizes[i]);
    }
    FMLH_TRY(alloc_t(m, &m->d_err, 1));
    FMLH_HIP(hipMemsetAsync(m->d_err, 0, sizeof(unsigned), s));
    if (const char* tp = std::getenv("FMLH_PERSIST_TRACE")) {
        m->d_trace_path = tp;
        const size_t n = (size_t)kTraceSteps * kMaxPersistG * kTracePoints;
        FMLH_TRY(alloc_t(m, &m->d_trace, n));
        FMLH_HIP(hipMemsetAsync(m->d_trace, 0, sizeof(unsigned long long) * n, s));
    }
    FMLH_HIP(hipStreamSynchronize(s));
    m->persist = true;
    return FMLH_OK;
}

// Exchange buffers of the grouped decode kernel, for max_batch sequences (up to 64).
int setup_grouped(fmlh_nanollm* m) {
    const char* env = std::getenv("FMLH_DECODE");
    if (env && std::strcmp(env, "graph") == 0) return FMLH_OK;
    const int bmax = std::min(m->Bmax, kGroupBatch * kMaxGroups);
    if (bmax < 2 || !grouped_plan(bmax, m->C, m->H, m->L, m->V, m->T, cu_count()).ok) return FMLH_OK;
    FMLH_TRY(setup_layer_table(m));
    m->grouped_groups = (bmax + kGroupBatch - 1) / kGroupBatch;
    grouped_group_words(m->C, 128, m->grouped_gw);
    const size_t ng = m->grouped_groups;
    uint64_t** bufs[] = {&m->g_qkv, &m->g_y, &m->g_dx1, &m->g_part, &m->g_dx2, &m->g_am};
    const size_t* gw = m->grouped_gw;
    // proj2 partials: [group][workgroup][kGroupBatch][C] with groups x workgroups <= 256
    const size_t part_words = (size_t)kMaxPersistG * kGroupBatch * m->C;
    const size_t sizes[] = {3 * ng * gw[0], ng * gw[0], ng * gw[0], part_words, ng * gw[0], ng * gw[1]};
    hipStream_t s = stream();
    for (int i = 0; i < 6; ++i) {
        FMLH_TRY(alloc_t(m, bufs[i], sizes[i]));
        FMLH_HIP(hipMemsetAsync(*bufs[i], 0, sizes[i] * sizeof(uint64_t), s));  // epoch 0: never current
        m->xbufs.emplace_back(*bufs[i], sizes[i]);
    }
    if (!m->d_err) {
        FMLH_TRY(alloc_t(m, &m->d_err, 1));
        FMLH_HIP(hipMemsetAsync(m->d_err, 0, sizeof(unsigned), s));
    }
    if (const char* tp = std::getenv("FMLH_GROUPED_TRACE")) {
        m->g_trace_path = tp;
        const size_t n = (size_t)kGroupedTraceSteps * kGroupedTraceWGs * kGroupedTracePoints;
        FMLH_TRY(alloc_t(m, &m->g_trace, n));
        FMLH_HIP(hipMemsetAsync(m->g_trace, 0, sizeof(unsigned long long) * n, s));
    }
    FMLH_HIP(hipStreamSynchronize(s));
    m->grouped = true;
    return FMLH_OK;
}

// Exchange buffers of the relay decode kernel (batches of up to min(max_batch, kRelayMaxBatch)).
int setup_relay(fmlh_nanollm* m) {
    const char* env = std::getenv("FMLH_DECODE");
    if (env && std::strcmp(env, "graph") == 0) return FMLH_OK;
    if (!relay_plan(1, m->C, m->H, m->L, m->V, m->T, cu_count()).ok) return FMLH_OK;
    FMLH_TRY(setup_layer_table(m));
    m->r_bmax = std::min((int)m->Bmax, kRelayMaxBatch);
    size_t words[5];
    relay_words(m->C, m->H, m->L, m->r_bmax, words);
    uint64_t** bufs[] = {&m->r_x, &m->r_part, &m->r_qkv, &m->r_dx1, &m->r_xp};
    const size_t sizes[] = {words[0], words[1], words[2], words[3], words[4]};
    hipStream_t s = stream();
    for (int i = 0; i < 5; ++i) {
        FMLH_TRY(alloc_t(m, bufs[i], sizes[i]));
        FMLH_HIP(hipMemsetAsync(*bufs[i], 0, sizes[i] * sizeof(uint64_t), s));  // epoch 0: never current
        m->xbufs.emplace_back(*bufs[i], sizes[i]);
    }
    if (!m->d_err) {
        FMLH_TRY(alloc_t(m, &m->d_err, 1));
        FMLH_HIP(hipMemsetAsync(m->d_err, 0, sizeof(unsigned), s));
    }
    if (const char* tp = std::getenv("FMLH_RELAY_TRACE")) {
        m->r_trace_path = tp;
        // The team cuts differ in their role counts (qa, big): room for the largest.
        m->r_roles = 0;
        for (int b : {1, std::min(m->r_bmax, kRelayBigBatch - 1), std::min(m->r_bmax, kRelaySplitBatch - 1), m->r_bmax})
            m->r_roles = std::max(m->r_roles, relay_plan(b, m->C, m->H, m->L, m->V, m->T, cu_count()).roles);
        const size_t n = (size_t)kRelayTraceSteps * m->r_roles * kRelayTracePoints;
        FMLH_TRY(alloc_t(m, &m->r_trace, n));
        FMLH_HIP(hipMemsetAsync(m->r_trace, 0, sizeof(unsigned long long) * n, s));
    }
    FMLH_HIP(hipStreamSynchronize(s));
    m->relay = true;
    return FMLH_OK;
}

int reserve_epochs(fmlh_nanollm* m, uint64_t span);

// Weights and exchange buffers of the wide decode kernel, for shapes it plans (batches of up to
// min(max_batch, 8) sequences).
int setup_wide(fmlh_nanollm* m) {
    const char* env = std::getenv("FMLH_DECODE");
    if (env && std::strcmp(env, "graph") == 0) return FMLH_OK;
    const char* we = std::getenv("FMLH_WIDE");
    if (we && we[0] == '0') return FMLH_OK;
    const WidePlan p = wide_plan(1, m->C, m->H, m->L, m->V, m->T, cu_count());
    if (!p.ok) return FMLH_OK;
    hipStream_t s = stream();
    const int C = m->C;
    m->w2.assign(m->L, nullptr);
    std::vector<WideLayer> wl(m->L);
    for (int l = 0; l < m->L; ++l) {
        const LayerW& w = m->layers[l];
        FMLH_TRY(alloc_t(m, &m->w2[l], (size_t)4 * C * C));
        FMLH_TRY(persist_transpose(m->w2[l], w.w2T, C, 4 * C, s));  // C x 4C -> 4C x C
        wl[l] = WideLayer{w.wqkvT, w.wproj, w.wfcT, m->w2[l], w.ln0g, w.ln0b, w.ln1g, w.ln1b};
    }
    FMLH_TRY(alloc_t(m, &m->d_wlayers, (size_t)m->L));
    FMLH_HIP(hipMemcpy(m->d_wlayers, wl.data(), wl.size() * sizeof(WideLayer), hipMemcpyHostToDevice));
    size_t words[6];
    wide_words(C, m->H, m->Bmax, p.G, p.S, words);
    words[1] = (size_t)p.G * (kWideHD + 2);  // P S <= G records at any batch
    uint64_t** bufs[] = {&m->w_q, &m->w_part, &m->w_y, &m->w_dx1, &m->w_dx2, &m->w_p2, &m->w_cand, &m->w_h};
    const size_t sizes[] = {words[0], words[1], words[2], words[2], words[2], words[3], words[4], words[5]};
    for (int i = 0; i < 8; ++i) {
        FMLH_TRY(alloc_t(m, bufs[i], sizes[i]));
        FMLH_HIP(hipMemsetAsync(*bufs[i], 0, sizes[i] * sizeof(uint64_t), s));  // epoch 0: never current
        m->xbufs.emplace_back(*bufs[i], sizes[i]);
    }
    if (!m->d_err) {
        FMLH_TRY(alloc_t(m, &m->d_err, 1));
        FMLH_HIP(hipMemsetAsync(m->d_err, 0, sizeof(unsigned), s));
    }
    // The timeline holds 12 points per layer and 4 for the lm_head (kWideTracePoints): deeper
    // models decode untraced.
    const char* tp_env = std::getenv("FMLH_WIDE_TRACE");
    if (const char* tp = 12 * m->L + 4 <= kWideTracePoints ? tp_env : nullptr) {
        m->w_trace_path = tp;
        FMLH_TRY(alloc_t(m, &m->w_trace, (size_t)p.G * kWideTracePoints));
        FMLH_HIP(hipMemsetAsync(m->w_trace, 0, sizeof(unsigned long long) * p.G * kWideTracePoints, s));
    }
    FMLH_HIP(hipStreamSynchronize(s));
    m->wide = true;
    return FMLH_OK;
}

// Whether a batch decodes on the wide kernel: greedy batches of up to 8 sequences of a shape it
// plans where no other one-launch kernel applies (c4, c5); FMLH_WIDE=1 also takes the shapes
// the persistent kernel plans (for comparisons), =0 never.
bool use_wide(const fmlh_nanollm* m, int batch) {
    if (!m->wide || batch < 1 || batch > std::min(m->Bmax, kWideMaxBatch) || m->temperature != 0.0f) return false;
    if (!wide_plan(batch, m->C, m->H, m->L, m->V, m->T, cu_count()).ok) return false;
    const char* env = std::getenv("FMLH_WIDE");
    if (env && env[0] == '1') return true;
    return !(m->persist && persist_plan(batch, m->C, m->H, m->L, m->V, m->T, cu_count()).ok);
}

int wide_steps(fmlh_nanollm* m, uint32_t n_steps, bool capture) {
    const WidePlan p = wide_plan((int)m->batch, m->C, m->H, m->L, m->V, m->T, cu_count());
    WideArgs a{};
    a.B = (int)m->batch; a.C = m->C; a.H = m->H; a.L = m->L; a.V = m->V; a.T = m->T; a.HS = m->HS;
    a.Bmax = m->Bmax; a.G = p.G; a.S = p.S;
    a.n_steps = (int)n_steps;
    a.pos0 = (int)(m->prompt_len + m->generated - 1);
    a.gen0 = (int)m->generated;
    FMLH_TRY(reserve_epochs(m, wide_epochs(m->L, (int)n_steps)));
    a.epoch_base = m->epoch;
    a.scale = m->scale;
    a.layers = m->d_wlayers;
    a.tok = m->tok; a.pos_emb = m->pos; a.lnf_g = m->lnf_g; a.lnf_b = m->lnf_b; a.lm = m->lm;
    a.kc = m->kc; a.vc = m->vc; a.hist = m->hist; a.st_pos = reinterpret_cast<int*>(m->st);
    a.logits = m->logits;
    a.logit_hist = capture ? m->logit_hist : nullptr;
    a.hist_slots = capture ? m->logit_hist_slots : 0;
    a.wq = m->w_q; a.wpart = m->w_part; a.wy = m->w_y; a.wdx1 = m->w_dx1; a.wp2 = m->w_p2; a.wdx2 = m->w_dx2;
    a.wh = m->w_h;
    a.wcand = m->w_cand; a.err = m->d_err;
    a.trace = m->w_trace;
    a.trace_step = n_steps > 1 ? 1 : 0;
    FMLH_TRY(wide_decode(a, p, stream()));
    m->epoch += (uint32_t)wide_epochs(m->L, (int)n_steps);
    if (m->w_trace) {  // step 1's timeline, appended raw: {G, points, L, B} then [G][points]
        const size_t n = (size_t)p.G * kWideTracePoints;
        std::vector<unsigned long long> tr(n);
        FMLH_HIP(hipStreamSynchronize(stream()));
        FMLH_HIP(hipMemcpy(tr.data(), m->w_trace, n * sizeof(unsigned long long), hipMemcpyDeviceToHost));
        if (FILE* f = std::fopen(m->w_trace_path.c_str(), "ab")) {
            const unsigned long long hdr[4] = {(unsigned long long)p.G, (unsigned long long)kWideTracePoints,
                                               (unsigned long long)m->L, (unsigned long long)m->batch};
            std::fwrite(hdr, sizeof(hdr), 1, f);
            std::fwrite(tr.data(), sizeof(unsigned long long), n, f);
            std::fclose(f);
        }
    }
    return FMLH_OK;
}

bool use_grouped(const fmlh_nanollm* m, int batch);

// Whether a batch decodes on the relay kernel: by default wherever it is planned for greedy
// batches of up to kRelayDefaultMaxBatch sequences of a compiled shape, and above that where
// the grouped kernel (faster there) does not take the batch; FMLH_RELAY=1 takes it up to
// kRelayMaxBatch, FMLH_RELAY=0 keeps the persistent and grouped kernels.
bool use_relay(const fmlh_nanollm* m, int batch) {
    if (!m->relay || batch < 1 || batch > m->r_bmax || m->temperature != 0.0f) return false;
    const char* env = std::getenv("FMLH_RELAY");
    if (env && env[0] == '0') return false;
    if (batch > kRelayDefaultMaxBatch && !(env && env[0] == '1') && use_grouped(m, batch)) return false;
    return relay_plan(batch, m->C, m->H, m->L, m->V, m->T, cu_count()).ok;
}

// The next launch uses epochs [m->epoch, m->epoch + span).  Exchange words carry 32-bit epochs
// and a word is current when its epoch equals the one awaited, so the count must never wrap:
// where it would, every exchange buffer is cleared back to epoch 0 (never awaited) and the
// count restarts at 1, after which no word left by an earlier launch can match.  (About 4e9
// epochs: ~1e8 steps of a c2 engine.)  FMLH_EPOCH_START=<n>, read at engine creation, starts
// the count at n so that tests reach the wrap.
int reserve_epochs(fmlh_nanollm* m, uint64_t span) {
    FMLH_REQUIRE(span < 0x40000000ull, "decode: %llu epochs in one launch", (unsigned long long)span);
    if ((uint64_t)m->epoch + span <= 0xffffffffull) return FMLH_OK;
    hipStream_t s = stream();
    for (const auto& b : m->xbufs) FMLH_HIP(hipMemsetAsync(b.first, 0, b.second * sizeof(uint64_t), s));
    m->epoch = 1;
    return FMLH_OK;
}

int relay_steps(fmlh_nanollm* m, uint32_t n_steps, bool capture) {
    const RelayPlan p = relay_plan((int)m->batch, m->C, m->H, m->L, m->V, m->T, cu_count());
    RelayArgs a{};
    a.B = (int)m->batch; a.L = m->L;
    a.lag_rows = a.B >= kRelayLagBatch; a.V = m->V; a.T = m->T; a.HS = m->HS; a.Bmax = m->Bmax;
    a.nq = p.nq; a.nf = p.nf; a.nf2 = p.nf2; a.nA = p.nA; a.nlm = p.nlm; a.roles = p.roles;
    a.n_steps = (int)n_steps;
    a.pos0 = (int)(m->prompt_len + m->generated - 1);
    a.gen0 = (int)m->generated;
    FMLH_TRY(reserve_epochs(m, (uint64_t)n_steps + 1u));
    a.epoch_base = m->epoch;
    a.scale = m->scale;
    a.layers = m->d_players;
    a.tok = m->tok; a.pos_emb = m->pos; a.lnf_g = m->lnf_g; a.lnf_b = m->lnf_b; a.lm = m->lm;
    a.kc = m->kc; a.vc = m->vc; a.hist = m->hist; a.st_pos = reinterpret_cast<int*>(m->st);
    a.logits = m->logits;
    a.logit_hist = capture ? m->logit_hist : nullptr;
    a.hist_slots = capture ? m->logit_hist_slots : 0;
    a.xw = m->r_x; a.partw = m->r_part; a.qkvw = m->r_qkv; a.dx1w = m->r_dx1; a.xpw = m->r_xp; a.err = m->d_err;
    a.trace = m->r_trace;

    FMLH_TRY(relay_decode(a, p, m->C, m->hd, stream()));
    m->r_last_roles = p.roles;
    m->r_last_nq = p.nq;
    m->r_last_nf = p.nf;
    m->r_last_nf2 = p.nf2;
    m->r_last_nA = p.nA;
    m->r_last_nlm = p.nlm;
    m->epoch += n_steps + 1u;
    return FMLH_OK;
}

// Whether a batch decodes on the grouped kernel: more sequences than one group of the batch-1
// kernel holds (FMLH_GROUPED=1 also takes smaller batches, for comparisons; =0 never).
bool use_grouped(const fmlh_nanollm* m, int batch) {
    if (!m->grouped || m->temperature != 0.0f) return false;
    if (!grouped_plan(batch, m->C, m->H, m->L, m->V, m->T, cu_count()).ok) return false;
    if ((batch + kGroupBatch - 1) / kGroupBatch > m->grouped_groups) return false;
    const char* env = std::getenv("FMLH_GROUPED");
    if (env && env[0] == '0') return false;
    if (env && env[0] == '1') return batch >= 2;
    return batch > kMaxPersistBatch;
}

int grouped_steps(fmlh_nanollm* m, uint32_t n_steps, bool capture) {
    const GroupedPlan p = grouped_plan((int)m->batch, m->C, m->H, m->L, m->V, m->T, cu_count());
    GroupedArgs a{};
    a.B = (int)m->batch; a.L = m->L; a.V = m->V; a.T = m->T; a.HS = m->HS; a.Bmax = m->Bmax;
    a.groups = p.groups; a.Bg = p.Bg;
    a.gw_c = m->grouped_gw[0]; a.gw_am = m->grouped_gw[1];
    a.n_steps = (int)n_steps;
    a.pos0 = (int)(m->prompt_len + m->generated - 1);
    a.gen0 = (int)m->generated;
    FMLH_TRY(reserve_epochs(m, (uint64_t)n_steps * (5u * m->L + 1u) + 1u));
    a.epoch_base = m->epoch;
    a.scale = m->scale;
    a.layers = m->d_players;
    a.tok = m->tok; a.pos_emb = m->pos; a.lnf_g = m->lnf_g; a.lnf_b = m->lnf_b; a.lm = m->lm;
    a.kc = m->kc; a.vc = m->vc; a.hist = m->hist; a.st_pos = reinterpret_cast<int*>(m->st);
    a.logits = m->logits;
    a.logit_hist = capture ? m->logit_hist : nullptr;
    a.hist_slots = capture ? m->logit_hist_slots : 0;
    a.q = m->g_qkv; a.qkv_stride = (size_t)m->grouped_groups * m->grouped_gw[0];
    a.y = m->g_y; a.dx1 = m->g_dx1; a.part = m->g_part; a.dx2 = m->g_dx2; a.am = m->g_am; a.err = m->d_err;
    a.trace = m->g_trace;
    if (p.groups > m->grouped_groups || (size_t)p.G * kGroupBatch * 2 > m->grouped_gw[1] ||
        p.G * p.groups > kMaxPersistG)
        return set_error(FMLH_E_STATE, "grouped plan does not fit the exchange buffers");
    FMLH_TRY(grouped_decode(a, p, m->C, m->hd, stream()));
    m->epoch += n_steps * (uint32_t)(5 * m->L + 1) + 1u;
    return FMLH_OK;
}

int persistent_steps(fmlh_nanollm* m, uint32_t n_steps, bool capture) {
    const PersistPlan p = persist_plan((int)m->batch, m->C, m->H, m->L, m->V, m->T, cu_count());
    PersistArgs a{};
    a.B = (int)m->batch; a.C = m->C; a.H = m->H; a.L = m->L; a.V = m->V; a.T = m->T;
    a.HS = m->HS; a.Bmax = m->Bmax;
    a.groups = p.groups; a.Bg = p.Bg;
    a.gw_qkv = m->persist_gw[0]; a.gw_att = m->persist_gw[1]; a.gw_c = m->persist_gw[2];
    a.gw_h4 = m->persist_gw[3]; a.gw_am = m->persist_gw[4];
    a.max_chunks = m->persist_chunks; a.h4p = p.h4p; a.wcap = p.wcap; a.ufloats = p.ufloats; a.kv_sep = p.kv_sep ? 1 : 0;
    a.n_steps = (int)n_steps;
    a.pos0 = (int)(m->prompt_len + m->generated - 1);
    a.gen0 = (int)m->generated;
    FMLH_TRY(reserve_epochs(m, (uint64_t)n_steps * (5u * m->L + 1u) + 1u));
    a.epoch_base = m->epoch;
    a.scale = m->scale;
    a.layers = m->d_players;
    a.tok = m->tok; a.pos_emb = m->pos; a.lnf_g = m->lnf_g; a.lnf_b = m->lnf_b; a.lm = m->lm;
    a.kc = m->kc; a.vc = m->vc; a.hist = m->hist; a.st_pos = reinterpret_cast<int*>(m->st);
    a.logits = m->logits;
    a.logit_hist = capture ? m->logit_hist : nullptr;
    a.hist_slots = capture ? m->logit_hist_slots : 0;
    a.q = m->x_q; a.kn = m->x_kn; a.vn = m->x_vn; a.att = m->x_att; a.dx1 = m->x_dx1;
    a.hb = m->x_hb; a.dx2 = m->x_dx2; a.am = m->x_am; a.err = m->d_err; a.trace = m->d_trace;
    if (p.G > m->persist_G || p.groups > m->persist_groups || p.max_chunks != m->persist_chunks)
        return set_error(FMLH_E_STATE, "persistent plan does not fit the exchange buffers");
    FMLH_TRY(persist_decode(a, p, m->hd, stream()));
    m->epoch += n_steps * (uint32_t)(5 * m->L + 1) + 1u;
    return FMLH_OK;
}

// Reports (and clears) a timed-out exchange of the persistent kernel; synchronizes.
int check_persistent(fmlh_nanollm* m) {
    if (!m->d_err) return FMLH_OK;  // neither persistent kernel was set up
    unsigned err = 0;
    FMLH_HIP(hipMemcpyAsync(&err, m->d_err, sizeof(unsigned), hipMemcpyDeviceToHost, stream()));
    FMLH_HIP(hipStreamSynchronize(stream()));
    if (m->d_trace) {  // timeline of the last launch, appended raw to the FMLH_PERSIST_TRACE file
        const size_t n = (size_t)kTraceSteps * kMaxPersistG * kTracePoints;
        std::vector<unsigned long long> t(n);
        FMLH_HIP(hipMemcpy(t.data(), m->d_trace, n * sizeof(unsigned long long), hipMemcpyDeviceToHost));
        FMLH_HIP(hipMemset(m->d_trace, 0, n * sizeof(unsigned long long)));
        if (FILE* f = std::fopen(m->d_trace_path.c_str(), "ab")) {
            const unsigned long long hdr[4] = {kTraceSteps, kMaxPersistG, kTracePoints, (unsigned long long)m->persist_G};
            std::fwrite(hdr, sizeof(hdr), 1, f);
            std::fwrite(t.data(), sizeof(unsigned long long), n, f);
            std::fclose(f);
        }
    }
    if (m->r_trace && m->r_last_roles) {  // timeline of the last relay launch, appended raw to FMLH_RELAY_TRACE
        const size_t n = (size_t)kRelayTraceSteps * m->r_last_roles * kRelayTracePoints;
        std::vector<unsigned long long> t(n);
        FMLH_HIP(hipMemcpy(t.data(), m->r_trace, n * sizeof(unsigned long long), hipMemcpyDeviceToHost));
        FMLH_HIP(hipMemset(m->r_trace, 0, n * sizeof(unsigned long long)));
        if (FILE* f = std::fopen(m->r_trace_path.c_str(), "ab")) {
            const unsigned long long hdr[10] = {kRelayTraceSteps, (unsigned long long)m->r_last_roles,
                                                kRelayTracePoints, (unsigned long long)m->L,
                                                (unsigned long long)m->r_last_nq, (unsigned long long)m->H,
                                                (unsigned long long)m->r_last_nf, (unsigned long long)m->r_last_nf2,
                                                (unsigned long long)m->r_last_nA, (unsigned long long)m->r_last_nlm};
            std::fwrite(hdr, sizeof(hdr), 1, f);
            std::fwrite(t.data(), sizeof(unsigned long long), n, f);
            std::fclose(f);
        }
    }
    if (m->g_trace) {  // timeline of the last grouped launch, appended raw to FMLH_GROUPED_TRACE
        const size_t n = (size_t)kGroupedTraceSteps * kGroupedTraceWGs * kGroupedTracePoints;
        std::vector<unsigned long long> t(n);
        FMLH_HIP(hipMemcpy(t.data(), m->g_trace, n * sizeof(unsigned long long), hipMemcpyDeviceToHost));
        FMLH_HIP(hipMemset(m->g_trace, 0, n * sizeof(unsigned long long)));
        if (FILE* f = std::fopen(m->g_trace_path.c_str(), "ab")) {
            const unsigned long long hdr[4] = {kGroupedTraceSteps, kGroupedTraceWGs, kGroupedTracePoints,
                                               (unsigned long long)m->L};
            std::fwrite(hdr, sizeof(hdr), 1, f);
            std::fwrite(t.data(), sizeof(unsigned long long), n, f);
            std::fclose(f);
        }
    }
    if (err) {
        FMLH_HIP(hipMemsetAsync(m->d_err, 0, sizeof(unsigned), stream()));
        return set_error(FMLH_E_HIP, "persistent decode: an exchange between workgroups timed out");
    }
    return FMLH_OK;
}

int generate_body(fmlh_nanollm* m, const int32_t* prompts, uint32_t batch, uint32_t prompt_len,
                  uint32_t n_gen, int32_t* tokens_out, float* logits_out);

// check_persistent for the readers: a failure found there also ends the loop (prefill again).
int checked_state(fmlh_nanollm* m) {
    const int rc = check_persistent(m);
    if (rc != FMLH_OK) m->prefilled = false;
    return rc;
}

int decode_steps(fmlh_nanollm* m, uint32_t n_steps, bool capture) {
    if (n_steps == 0) return FMLH_OK;
    if (use_relay(m, (int)m->batch)) {
        const int rc = relay_steps(m, n_steps, capture);
        if (rc == FMLH_OK) {
            m->generated += n_steps;
            return FMLH_OK;
        }
        if (rc != kPersistRefused) return rc;
        m->relay = false;  // cooperative launch refused: the other paths from now on
    }
    if (use_grouped(m, (int)m->batch)) {
        const int rc = grouped_steps(m, n_steps, capture);
        if (rc == FMLH_OK) {
            m->generated += n_steps;
            return FMLH_OK;
        }
        if (rc != kPersistRefused) return rc;
        m->grouped = false;  // cooperative launch refused: the graph path from now on
    }
    if (use_wide(m, (int)m->batch)) {
        const int rc = wide_steps(m, n_steps, capture);
        if (rc == FMLH_OK) {
            m->generated += n_steps;
            return FMLH_OK;
        }
        if (rc != kPersistRefused) return rc;
        m->wide = false;  // cooperative launch refused: the other paths from now on
    }
    if (m->persist && m->temperature == 0.0f &&
        persist_plan((int)m->batch, m->C, m->H, m->L, m->V, m->T, cu_count()).ok) {
        const int rc = persistent_steps(m, n_steps, capture);
        if (rc == FMLH_OK) {
            m->generated += n_steps;
            return FMLH_OK;
        }
        if (rc != kPersistRefused) return rc;
        // The runtime refused the cooperative launch (another process holds the device's
        // cooperative-launch resource): nothing was enqueued, so this and later steps of this
        // model run on the graph path, which computes the same tokens.
        m->persist = false;
    }
    const int which = capture ? 1 : 0;
    FMLH_TRY(ensure_ws(m, gemm_ws_for(m, (int)m->batch)));
    if (m->use_graph) {
        FMLH_TRY(build_graph(m, which));
        for (uint32_t i = 0; i < n_steps; ++i) FMLH_HIP(hipGraphLaunch(m->graph[which], stream()));
    } else {
        for (uint32_t i = 0; i < n_steps; ++i) FMLH_TRY(enqueue_decode_step(m, capture));
    }
    m->generated += n_steps;
    return FMLH_OK;
}

int do_prefill(fmlh_nanollm* m, const int32_t* prompts, uint32_t batch, uint32_t P) {
    hipStream_t s = stream();
    // The pinned staging buffer is free: every call that copies from it ends with a stream
    // synchronization.
    int32_t* hist = m->hist_host;
    std::fill(hist, hist + (size_t)batch * m->HS, 0);
    for (uint32_t b = 0; b < batch; ++b)
        for (uint32_t p = 0; p < P; ++p) {
            const int32_t id = prompts[(size_t)b * P + p];
            FMLH_REQUIRE(id >= 0 && (uint32_t)id < (uint32_t)m->V,
                         "prefill: token id %d of sequence %u outside [0, %d)", id, b, m->V);
            hist[(size_t)b * m->HS + p] = id;
        }
    FMLH_HIP(hipMemcpyAsync(m->hist, hist, (size_t)batch * m->HS * sizeof(int32_t), hipMemcpyHostToDevice,
                            s));
    const int M = (int)(batch * P);
    const bool fused = prefill_fused(m, M);
    // FMLH_PREFILL_STREAMS=n: the fused prefill in n parts (1 .. 4; default 2).
    const char* parts_env = std::getenv("FMLH_PREFILL_STREAMS");
    const int parts = std::min<int>((int)batch, parts_env ? std::max(1, std::min(fmlh_nanollm::kPrefillParts,
                                                                                   std::atoi(parts_env)))
                                                          : 2);
    // Every part's workspace slice holds what any part plans (a smaller part can plan a split
    // that a larger one does not: 320 rows of c3's FC product split K, 384 rows do not).
    size_t part_ws = 0;
    for (int i = 0; fused && i < parts; ++i) {
        const int nb = (int)batch * (i + 1) / parts - (int)batch * i / parts;
        part_ws = std::max(part_ws, fused_part_ws(m, nb * (int)P));
    }
    FMLH_TRY(ensure_ws(m, std::max(gemm_ws_for(m, M), (size_t)parts * part_ws)));
    const size_t n = (size_t)M * m->C;
    hipLaunchKernelGGL(embed_kernel, dim3(blocks_for(n, 256, 8192u)), dim3(256), 0, s, m->x, m->hist,
                       m->HS, (int)P, 0, nullptr, m->tok, m->pos, m->C, M);
    FMLH_LAUNCHED("embed_kernel");
    if (!fused) {
        FMLH_TRY(run_blocks(m, (int)batch, (int)P, false));
    } else if (parts == 1) {
        FMLH_TRY(prefill_seqs(m, 0, (int)batch, (int)P, s, m->ws, part_ws));
    } else {
        // The batch in parts of whole sequences on their own streams: each part's small kernels
        // (attention, the reductions) and the tails of its products overlap the other parts'
        // products.  Part i takes sequences [i B / n, (i + 1) B / n) and its own workspace rows.
        if (!m->ev_fork) FMLH_HIP(hipEventCreateWithFlags(&m->ev_fork, hipEventDisableTiming));
        for (int i = 0; i < parts - 1; ++i)
            if (!m->s2[i]) {
                FMLH_HIP(hipStreamCreateWithFlags(&m->s2[i], hipStreamNonBlocking));
                FMLH_HIP(hipEventCreateWithFlags(&m->ev_join[i], hipEventDisableTiming));
            }
        FMLH_HIP(hipEventRecord(m->ev_fork, s));
        for (int i = 0; i < parts - 1; ++i) FMLH_HIP(hipStreamWaitEvent(m->s2[i], m->ev_fork, 0));
        int rc = FMLH_OK;
        for (int l = -1; l < m->L && rc == FMLH_OK; ++l)  // layer by layer, so every stream has work
            for (int i = 0; i < parts && rc == FMLH_OK; ++i) {
                const int b0 = (int)batch * i / parts, b1 = (int)batch * (i + 1) / parts;
                rc = prefill_seqs_layer(m, l, b0, b1 - b0, (int)P, i == 0 ? s : m->s2[i - 1],
                                        m->ws + (size_t)i * part_ws, part_ws);
            }
        // Joined on every path: after a failed launch the library stream still orders the next
        // call behind whatever the other streams had been given.
        for (int i = 0; i < parts - 1; ++i) {
            FMLH_HIP(hipEventRecord(m->ev_join[i], m->s2[i]));
            FMLH_HIP(hipStreamWaitEvent(s, m->ev_join[i], 0));
        }
        FMLH_TRY(rc);
    }
    const size_t nl = (size_t)batch * m->C;
    hipLaunchKernelGGL(last_rows_kernel, dim3(blocks_for(nl, 256, 1024u)), dim3(256), 0, s, m->xlast,
                       fused ? m->xn : m->x, (int)P, m->C, (int)batch);
    FMLH_LAUNCHED("last_rows_kernel");
    FMLH_TRY(head_and_pick(m, m->xlast, (int)batch, false, (int)P - 1, fused));
    hipLaunchKernelGGL(set_state_kernel, dim3(1), dim3(1), 0, s, m->st, (int)P, 1);
    FMLH_LAUNCHED("set_state_kernel");
    // The history staging buffer is reused by the next call: its copy must have happened.
    FMLH_HIP(hipStreamSynchronize(s));
    m->batch = batch;
    m->prompt_len = P;
    m->generated = 1;
    m->prefilled = true;
    return FMLH_OK;
}

}  // namespace

extern "C" {

int fmlh_nanollm_create(const fmlh_nanollm_config* cfg, const fmlh_nanollm_weights* w,
                        int weights_on_device, fmlh_nanollm** out) {
    FMLH_REQUIRE(cfg && w && out, "fmlh_nanollm_create: null argument");
    *out = nullptr;
    FMLH_REQUIRE(cfg->vocab && cfg->block_size && cfg->n_embed && cfg->n_head && cfg->n_layer &&
                     cfg->max_batch,
                 "fmlh_nanollm_create: zero-sized dimension");
    FMLH_REQUIRE(cfg->n_embed % cfg->n_head == 0, "n_embed %u not divisible by n_head %u",
                 cfg->n_embed, cfg->n_head);
    FMLH_REQUIRE(cfg->n_embed % 16 == 0, "n_embed %u must be a multiple of 16", cfg->n_embed);
    FMLH_REQUIRE(attn_head_dim_supported((int)(cfg->n_embed / cfg->n_head)),
                 "head_dim %u unsupported (16, 32 or 64)", cfg->n_embed / cfg->n_head);
    FMLH_REQUIRE(w->tok_emb && w->pos_emb && w->layers && w->lnf_gamma,
                 "fmlh_nanollm_create: missing weights");
    FMLH_TRY(ensure_init());

    auto* m = new fmlh_nanollm();
    m->cfg = *cfg;
    m->V = (int)cfg->vocab; m->T = (int)cfg->block_size; m->C = (int)cfg->n_embed;
    m->H = (int)cfg->n_head; m->L = (int)cfg->n_layer; m->hd = m->C / m->H;
    m->Bmax = (int)cfg->max_batch;
    m->HS = m->T + 1;
    m->scale = 1.0f / sqrtf((float)m->hd);  // CausalSelfAttentionLayer.h:73-74
    const char* env = std::getenv("FMLH_NO_GRAPH");
    m->use_graph = !(env && env[0] == '1');
    if (const char* ep = std::getenv("FMLH_EPOCH_START")) m->epoch = (uint32_t)std::strtoul(ep, nullptr, 10);
    if (m->epoch == 0) m->epoch = 1;
    const size_t C = m->C, V = m->V, T = m->T;
    int rc = FMLH_OK;
    auto fail = [&](int code) { release(m); delete m; return code; };
    if ((rc = upload(m, w->tok_emb, V * C, weights_on_device, &m->tok))) return fail(rc);
    if ((rc = upload(m, w->pos_emb, T * C, weights_on_device, &m->pos))) return fail(rc);
    if ((rc = upload(m, w->lnf_gamma, C, weights_on_device, &m->lnf_g))) return fail(rc);
    if ((rc = upload(m, w->lnf_beta, C, weights_on_device, &m->lnf_b))) return fail(rc);
    if (w->lm_head == nullptr || w->lm_head == w->tok_emb) m->lm = m->tok;  // tied
    else if ((rc = upload(m, w->lm_head, V * C, weights_on_device, &m->lm))) return fail(rc);
    m->layers.resize(m->L);
    for (int l = 0; l < m->L; ++l) {
        const float* const* p = w->layers + 8 * l;
        LayerW& lw = m->layers[l];
        if (!p[0] || !p[1] || !p[2] || !p[3] || !p[4] || !p[6])
            return fail(set_error(FMLH_E_INVALID, "layer %d: missing weight", l));
        if ((rc = upload_transposed(m, p[0], (int)C, (int)(3 * C), weights_on_device, &lw.wqkvT)))
            return fail(rc);
        if ((rc = upload(m, p[1], C * C, weights_on_device, &lw.wproj))) return fail(rc);
        if ((rc = upload_transposed(m, p[2], (int)C, (int)(4 * C), weights_on_device, &lw.wfcT)))
            return fail(rc);
        if ((rc = upload_transposed(m, p[3], (int)(4 * C), (int)C, weights_on_device, &lw.w2T)))
            return fail(rc);
        if ((rc = upload(m, p[4], C, weights_on_device, &lw.ln0g))) return fail(rc);
        if ((rc = upload(m, p[5], C, weights_on_device, &lw.ln0b))) return fail(rc);
        if ((rc = upload(m, p[6], C, weights_on_device, &lw.ln1g))) return fail(rc);
        if ((rc = upload(m, p[7], C, weights_on_device, &lw.ln1b))) return fail(rc);
        if (weights_on_device) m->t_src.insert(m->t_src.end(), {p[0], p[2], p[3]});
    }
    const size_t B = m->Bmax, R = B * T;
    const size_t cache = (size_t)m->L * B * T * C;
    if ((rc = alloc_t(m, &m->kc, cache)) || (rc = alloc_t(m, &m->vc, cache)) ||
        (rc = alloc_t(m, &m->x, R * C)) || (rc = alloc_t(m, &m->xn, R * C)) ||
        (rc = alloc_t(m, &m->qkv, R * 3 * C)) || (rc = alloc_t(m, &m->y, R * C)) ||
        (rc = alloc_t(m, &m->h, R * 4 * C)) || (rc = alloc_t(m, &m->xlast, B * C)) ||
        (rc = alloc_t(m, &m->logits, B * V)) || (rc = alloc_t(m, &m->hist, B * (T + 1))) ||
        (rc = alloc_t(m, &m->st, 1)))
        return fail(rc);
    {
        const hipError_t e = hipHostMalloc((void**)&m->hist_host, B * (T + 1) * sizeof(int32_t));
        if (e != hipSuccess) return fail(hip_fail(e, "hipHostMalloc(hist_host)", __FILE__, __LINE__));
    }
    const size_t aws = attn_decode_workspace((int)B, m->H, m->hd, m->T);
    if (aws && (rc = alloc_t(m, &m->attn_ws, aws))) return fail(rc);
    if (aws) {  // the arrival counts at its tail start at zero (every decode call leaves them so)
        const hipError_t e = hipMemset(m->attn_ws, 0, aws * sizeof(float));
        if (e != hipSuccess) return fail(hip_fail(e, "hipMemset(attn_ws)", __FILE__, __LINE__));
    }
    if ((rc = ensure_ws(m, gemm_ws_for(m, (int)B)))) return fail(rc);
    if ((rc = setup_persistent(m))) return fail(rc);
    if ((rc = setup_grouped(m))) return fail(rc);
    if ((rc = setup_relay(m))) return fail(rc);
    if ((rc = setup_wide(m))) return fail(rc);
    {
        std::lock_guard<std::mutex> lock(g_engines_mu);
        g_engines.insert(m);
    }
    *out = m;
    return FMLH_OK;
}

int fmlh_nanollm_refresh_weights(fmlh_nanollm* m) {
    FMLH_REQUIRE(m, "fmlh_nanollm_refresh_weights: null handle");
    if (m->t_src.empty())
        return set_error(FMLH_E_STATE, "fmlh_nanollm_refresh_weights: the engine was created from host "
                                       "weights and owns every copy");
    const int C = m->C;
    for (int l = 0; l < m->L; ++l) {
        const LayerW& lw = m->layers[l];
        // The transposed copies are engine-owned allocations (upload_transposed).
        FMLH_TRY(persist_transpose(const_cast<float*>(lw.wqkvT), m->t_src[3 * l + 0], C, 3 * C, stream()));
        FMLH_TRY(persist_transpose(const_cast<float*>(lw.wfcT), m->t_src[3 * l + 1], C, 4 * C, stream()));
        FMLH_TRY(persist_transpose(const_cast<float*>(lw.w2T), m->t_src[3 * l + 2], 4 * C, C, stream()));
        if (!m->w2.empty())  // the wide kernel's copy in FreeML's own 4C x C layout
            FMLH_HIP(hipMemcpyAsync(m->w2[l], m->t_src[3 * l + 2], sizeof(float) * 4 * C * C, hipMemcpyDeviceToDevice,
                                    stream()));
    }
    return FMLH_OK;
}

int fmlh_nanollm_destroy(fmlh_nanollm* m) {
    if (!m) return FMLH_OK;
    {
        std::lock_guard<std::mutex> lock(g_engines_mu);
        if (!g_engines.erase(m))
            return set_error(FMLH_E_STATE, "fmlh_nanollm_destroy: unknown handle (destroyed, or released by fmlh_shutdown)");
    }
    (void)hipStreamSynchronize(stream());
    release(m);
    delete m;
    return FMLH_OK;
}

int fmlh_nanollm_prefill(fmlh_nanollm* m, const int32_t* prompts, uint32_t batch,
                         uint32_t prompt_len) {
    FMLH_REQUIRE(m && prompts, "fmlh_nanollm_prefill: null argument");
    FMLH_REQUIRE(batch >= 1 && batch <= (uint32_t)m->Bmax, "batch %u outside [1, %d]", batch, m->Bmax);
    FMLH_REQUIRE(prompt_len >= 1 && prompt_len <= (uint32_t)m->T, "prompt_len %u outside [1, %d]",
                 prompt_len, m->T);
    m->prefilled = false;
    return do_prefill(m, prompts, batch, prompt_len);
}

int fmlh_nanollm_decode(fmlh_nanollm* m, uint32_t n_steps) {
    FMLH_REQUIRE(m, "fmlh_nanollm_decode: null handle");
    if (!m->prefilled) return set_error(FMLH_E_STATE, "decode before prefill");
    // Decode step g (g >= 1) processes position prompt_len + g - 1; the last position a
    // block_size window holds is T - 1.
    if ((size_t)m->prompt_len + m->generated + n_steps > (size_t)m->T + 1)
        return set_error(FMLH_E_STATE, "decode of %u steps passes block_size %d", n_steps, m->T);
    // A failed decode leaves no readable state: tokens and logits of earlier steps would be
    // stale, so the loop must start again with a prefill.
    const int rc = decode_steps(m, n_steps, false);
    if (rc != FMLH_OK) m->prefilled = false;
    return rc;
}

int fmlh_nanollm_read_tokens(fmlh_nanollm* m, int32_t* out, uint32_t first, uint32_t count) {
    FMLH_REQUIRE(m && out, "fmlh_nanollm_read_tokens: null argument");
    if (!m->prefilled) return set_error(FMLH_E_STATE, "no tokens before prefill");
    // Checked without forming first + count, which can wrap in 32 bits.
    FMLH_REQUIRE(first <= m->generated && count <= m->generated - first,
                 "tokens [%u, %llu) not generated (have %u)", first,
                 (unsigned long long)first + count, m->generated);
    FMLH_TRY(checked_state(m));
    if (count == 0) return FMLH_OK;
    FMLH_HIP(hipMemcpy2DAsync(out, count * sizeof(int32_t), m->hist + m->prompt_len + first,
                              (size_t)m->HS * sizeof(int32_t), count * sizeof(int32_t), m->batch,
                              hipMemcpyDeviceToHost, stream()));
    FMLH_HIP(hipStreamSynchronize(stream()));
    return FMLH_OK;
}

int fmlh_nanollm_read_logits(fmlh_nanollm* m, float* out) {
    FMLH_REQUIRE(m && out, "fmlh_nanollm_read_logits: null argument");
    if (!m->prefilled) return set_error(FMLH_E_STATE, "no logits before prefill");
    FMLH_TRY(checked_state(m));
    FMLH_HIP(hipMemcpyAsync(out, m->logits, (size_t)m->batch * m->V * sizeof(float),
                            hipMemcpyDeviceToHost, stream()));
    FMLH_HIP(hipStreamSynchronize(stream()));
    return FMLH_OK;
}

int fmlh_nanollm_status(fmlh_nanollm* m, uint32_t* generated, uint32_t* batch) {
    FMLH_REQUIRE(m, "fmlh_nanollm_status: null handle");
    if (generated) *generated = m->prefilled ? m->generated : 0;
    if (batch) *batch = m->prefilled ? m->batch : 0;
    return FMLH_OK;
}

int fmlh_nanollm_decode_path(fmlh_nanollm* m, uint32_t batch, int* path, int* workgroups) {
    FMLH_REQUIRE(m && path, "fmlh_nanollm_decode_path: null argument");
    FMLH_REQUIRE(batch >= 1 && batch <= (uint32_t)m->Bmax, "batch %u outside [1, %d]", batch, m->Bmax);
    const PersistPlan p = persist_plan((int)batch, m->C, m->H, m->L, m->V, m->T, cu_count());
    if (use_relay(m, (int)batch)) {
        *path = FMLH_DECODE_RELAY;
        if (workgroups) *workgroups = relay_plan((int)batch, m->C, m->H, m->L, m->V, m->T, cu_count()).G;
        return FMLH_OK;
    }
    if (use_grouped(m, (int)batch)) {
        const GroupedPlan gp = grouped_plan((int)batch, m->C, m->H, m->L, m->V, m->T, cu_count());
        *path = FMLH_DECODE_GROUPED;
        if (workgroups) *workgroups = gp.G * gp.groups;
        return FMLH_OK;
    }
    if (use_wide(m, (int)batch)) {
        *path = FMLH_DECODE_WIDE;
        if (workgroups) *workgroups = wide_plan((int)batch, m->C, m->H, m->L, m->V, m->T, cu_count()).G;
        return FMLH_OK;
    }
    const bool persistent = m->persist && m->temperature == 0.0f && p.ok;
    *path = persistent ? FMLH_DECODE_PERSISTENT : FMLH_DECODE_GRAPH;
    if (workgroups) *workgroups = persistent ? p.G * p.groups : 0;
    return FMLH_OK;
}

int fmlh_nanollm_set_sampling(fmlh_nanollm* m, float temperature, uint32_t top_k, unsigned long long seed) {
    FMLH_REQUIRE(m, "fmlh_nanollm_set_sampling: null handle");
    FMLH_REQUIRE(temperature >= 0.0f && temperature < INFINITY, "fmlh_nanollm_set_sampling: temperature %g", temperature);
    FMLH_TRY(ensure_init());
    m->temperature = temperature;
    m->top_k = top_k;
    m->seed = seed;
    // The captured decode steps baked the previous pick in.
    for (int w = 0; w < 2; ++w)
        if (m->graph[w]) {
            (void)hipGraphExecDestroy(m->graph[w]);
            m->graph[w] = nullptr;
        }
    return FMLH_OK;
}

int fmlh_nanollm_generate(fmlh_nanollm* m, const int32_t* prompts, uint32_t batch,
                          uint32_t prompt_len, uint32_t n_gen, int32_t* tokens_out,
                          float* logits_out) {
    FMLH_REQUIRE(m && prompts && tokens_out, "fmlh_nanollm_generate: null argument");
    FMLH_REQUIRE(n_gen >= 1, "n_gen must be >= 1");
    FMLH_REQUIRE(batch >= 1 && batch <= (uint32_t)m->Bmax, "batch %u outside [1, %d]", batch, m->Bmax);
    FMLH_REQUIRE(prompt_len >= 1 && (uint64_t)prompt_len + n_gen - 1 <= (uint64_t)m->T,
                 "prompt_len %u + n_gen %u - 1 exceeds block_size %d", prompt_len, n_gen, m->T);
    m->prefilled = false;
    const int rc = generate_body(m, prompts, batch, prompt_len, n_gen, tokens_out, logits_out);
    if (rc != FMLH_OK) m->prefilled = false;
    return rc;
}

}  // extern "C"

namespace {

int generate_body(fmlh_nanollm* m, const int32_t* prompts, uint32_t batch, uint32_t prompt_len,
                    uint32_t n_gen, int32_t* tokens_out, float* logits_out) {
    FMLH_TRY(do_prefill(m, prompts, batch, prompt_len));
    const bool capture = logits_out != nullptr;
    if (capture) {
        FMLH_TRY(ensure_logit_hist(m, n_gen));
        FMLH_HIP(hipMemcpyAsync(m->logit_hist, m->logits, (size_t)batch * m->V * sizeof(float),
                                hipMemcpyDeviceToDevice, stream()));
    }
    FMLH_TRY(decode_steps(m, n_gen - 1, capture));
    FMLH_TRY(fmlh_nanollm_read_tokens(m, tokens_out, 0, n_gen));
    if (capture) {
        // slot g holds batch x V; the caller wants batch x n_gen x V.
        for (uint32_t g = 0; g < n_gen; ++g)
            FMLH_HIP(hipMemcpy2DAsync(logits_out + (size_t)g * m->V,
                                      (size_t)n_gen * m->V * sizeof(float),
                                      m->logit_hist + (size_t)g * batch * m->V,
                                      (size_t)m->V * sizeof(float), (size_t)m->V * sizeof(float),
                                      batch, hipMemcpyDeviceToHost, stream()));
        FMLH_HIP(hipStreamSynchronize(stream()));
    }
    return FMLH_OK;
}

}  // namespace

extern "C" {

int fmlh_nanollm_profile_op(fmlh_nanollm* m, int op, uint32_t iters, float* avg_ms,
                            double* bytes) {
    FMLH_REQUIRE(m && avg_ms && bytes, "fmlh_nanollm_profile_op: null argument");
    FMLH_REQUIRE(iters >= 1, "fmlh_nanollm_profile_op: iters must be >= 1");
    if (!m->prefilled) return set_error(FMLH_E_STATE, "profile_op needs a prefilled loop");
    const int B = (int)m->batch, C = m->C;
    const double f = sizeof(float);
    const LayerW& w = m->layers[0];
    float* kc = m->kc;
    float* vc = m->vc;
    FMLH_TRY(ensure_ws(m, gemm_ws_for(m, B)));
    // Position of the next decode step: the attention op reads keys 0..pos.
    const double keys = (double)m->prompt_len + m->generated - 1 + 1;
    // The kernels a decode step runs for the op: on the fused path (batched decode) the residual
    // projections include their fused reductions, the QKV product is its split partials and the
    // attention adds them up (the QKV partials are made once before the attention is timed).
    const bool fused = decode_fused(m, B);
    int qkv_splits = 0;
    if (fused && op == FMLH_OP_ATTENTION) FMLH_TRY(fused_qkv(m, 0, B, &qkv_splits));
    auto run = [&]() -> int {
        int sp = 0;
        switch (op) {
            case FMLH_OP_QKV:
                if (fused) return fused_qkv(m, 0, B, &sp);
                return proj(m, m->xn, C, w.wqkvT, C, 1, m->qkv, 3 * C, B, 3 * C, C, kEpiNone, nullptr, 0);
            case FMLH_OP_ATTENTION:
                if (fused)
                    return attn_decode(m->ws, 3 * C, kc, vc, m->y, C, B, m->H, m->hd, m->T, &m->st->pos,
                                       m->scale, m->attn_ws, m->Bmax, stream(), qkv_splits);
                return attn_decode(m->qkv, 3 * C, kc, vc, m->y, C, B, m->H, m->hd, m->T, &m->st->pos,
                                   m->scale, m->attn_ws, m->Bmax, stream(), 1);
            case FMLH_OP_ATTN_PROJ:
                if (fused) return fused_resid_ln(m, m->y, w.wproj, C, B, w.ln1g, w.ln1b);
                return proj(m, m->y, C, w.wproj, C, 1, m->x, C, B, C, C, kEpiResid, m->x, C);
            case FMLH_OP_MLP_FC:
                return proj(m, m->xn, C, w.wfcT, C, 1, m->h, 4 * C, B, 4 * C, C, kEpiGelu, nullptr, 0);
            case FMLH_OP_MLP_PROJ:
                if (fused) return fused_resid_ln(m, m->h, w.w2T, 4 * C, B, w.ln1g, w.ln1b);
                return proj(m, m->h, 4 * C, w.w2T, 4 * C, 1, m->x, C, B, C, 4 * C, kEpiResid, m->x, C);
            case FMLH_OP_LM_HEAD:
                return proj(m, m->xn, C, m->lm, C, 1, m->logits, m->V, B, m->V, C, kEpiNone, nullptr, 0);
            default:
                return set_error(FMLH_E_INVALID, "profile_op: unknown op %d", op);
        }
    };
    switch (op) {
        case FMLH_OP_QKV: *bytes = f * ((double)C * 3 * C + (double)B * C + (double)B * 3 * C); break;
        case FMLH_OP_ATTENTION:  // + the QKV partials read and the K / V rows written when fused
            *bytes = f * ((double)B * m->H * keys * m->hd * 2 + (double)B * C * 2 +
                          (fused ? (double)qkv_splits * B * 3 * C + 2.0 * B * C : 0.0));
            break;
        case FMLH_OP_ATTN_PROJ:  // + the LayerNorm's output and parameters when fused
            *bytes = f * ((double)C * C + 3.0 * B * C + (fused ? (double)B * C + 2.0 * C : 0.0)); break;
        case FMLH_OP_MLP_FC: *bytes = f * ((double)C * 4 * C + (double)B * C + (double)B * 4 * C); break;
        case FMLH_OP_MLP_PROJ:
            *bytes = f * ((double)4 * C * C + (double)B * 4 * C + 2.0 * B * C +
                          (fused ? (double)B * C + 2.0 * C : 0.0));
            break;
        case FMLH_OP_LM_HEAD: *bytes = f * ((double)m->V * C + (double)B * C + (double)B * m->V); break;
        default: return set_error(FMLH_E_INVALID, "profile_op: unknown op %d", op);
    }
    FMLH_TRY(run());  // warm-up
    hipEvent_t e0, e1;
    FMLH_HIP(hipEventCreate(&e0));
    FMLH_HIP(hipEventCreate(&e1));
    int rc = FMLH_OK;
    hipError_t e = hipEventRecord(e0, stream());
    for (uint32_t i = 0; i < iters && rc == FMLH_OK && e == hipSuccess; ++i) rc = run();
    if (e == hipSuccess) e = hipEventRecord(e1, stream());
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (rc != FMLH_OK) return rc;
    if (e != hipSuccess) return hip_fail(e, "profile_op timing", __FILE__, __LINE__);
    *avg_ms = ms / (float)iters;
    return FMLH_OK;
}

int fmlh_nanollm_forward_window(fmlh_nanollm* m, const int32_t* ids, uint32_t batch,
                                float* logits_out) {
    FMLH_REQUIRE(m && ids && logits_out, "fmlh_nanollm_forward_window: null argument");
    FMLH_REQUIRE(batch >= 1 && batch <= (uint32_t)m->Bmax, "batch %u outside [1, %d]", batch, m->Bmax);
    m->prefilled = false;
    const uint32_t T = (uint32_t)m->T;
    FMLH_TRY(do_prefill(m, ids, batch, T));
    // Logits for every row: ln_f over all rows, then lm_head on all of them.
    const int M = (int)(batch * T);
    hipStream_t s = stream();
    float* all = nullptr;
    FMLH_TRY(device_malloc(reinterpret_cast<void**>(&all), (size_t)M * m->V * sizeof(float)));
    int rc = layernorm_rows(m->xn, m->x, m->lnf_g, m->lnf_b, nullptr, M, m->C, 1e-5f, s);
    if (rc == FMLH_OK) {
        GemmArgs g;
        g.A = m->xn; g.lda = m->C; g.B = m->lm; g.ldb = m->C; g.b_trans = 1;
        g.C = all; g.ldc = m->V; g.M = M; g.N = m->V; g.K = m->C; g.s = s;
        rc = gemm(g, nullptr, 0);
    }
    if (rc == FMLH_OK) {
        hipError_t e = hipMemcpyAsync(logits_out, all, (size_t)M * m->V * sizeof(float),
                                      hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = hip_fail(e, "forward_window copy", __FILE__, __LINE__);
    }
    (void)hipStreamSynchronize(s);
    (void)hipFree(all);
    m->prefilled = false;  // the window run is not a loop start
    return rc;
}

}  // extern "C"

namespace fmlh {

void destroy_all_engines() {
    std::lock_guard<std::mutex> lock(g_engines_mu);
    for (fmlh_nanollm* m : g_engines) {
        release(m);
        delete m;
    }
    g_engines.clear();
}

}  // namespace fmlh

