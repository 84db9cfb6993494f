// Causal self-attention over the device KV cache (CausalSelfAttentionLayer::Forward,
// CausalSelfAttentionLayer.h:424-499: S = Q_h K_h^T * (1/sqrt(hd)) + causal -inf mask,
// row softmax, Y_h = P V_h).  The reference materialises every T x T score matrix; here no
// score matrix is stored:
//   * prefill: one work-group per block of query rows of one (sequence, head) -- 128 rows on
//     the 32x32x2 matrix cores for head_dim 64, 64 rows on 16x16x4 for head_dim 32, one wave
//     per lane-row for head_dim 16 -- keys streamed through LDS in 64-key tiles up to the
//     diagonal, online softmax (running max / sum) per query row; work-groups dispatched
//     longest (latest) query block first;
//   * decode: one query row per (sequence, head), the cached keys split into 256-position
//     chunks across work-groups; each chunk leaves (max, sum, unnormalised output) and the
//     last chunk to finish merges them in chunk order.
// Masked positions (j > i) are skipped: in the reference they contribute exp(-inf) = 0.
//
// KV cache layout: [layer][sequence][head][position][head_dim], fp32.
#include "attention.h"

#include <cstdlib>
#include <cstring>

namespace fmlh {

namespace {

constexpr int kTile = 64;  // keys per LDS tile (prefill)
constexpr int kChunk = 16; // keys per online-softmax update

template <int HD>
__global__ __launch_bounds__(64) void attn_prefill_kernel(
    const float* __restrict__ qkv, int qkv_ld, const float* __restrict__ kc,
    const float* __restrict__ vc, float* __restrict__ y, int y_ld, int rows_per_seq, int H,
    int T, float scale) {
    __shared__ float Ks[kTile][HD];
    __shared__ float Vs[kTile][HD];
    const int lane = threadIdx.x;
    const int qb = gridDim.y - 1 - blockIdx.y;  // query block, longest first (x-fastest dispatch)
    const int bh = blockIdx.x;                  // sequence * H + head
    const int b = bh / H, h = bh % H;
    const int i = qb * 64 + lane;       // query position (prefill starts at position 0)
    const bool active = i < rows_per_seq;
    const size_t row = (size_t)b * rows_per_seq + (active ? i : 0);
    const float* kbase = kc + (size_t)bh * T * HD;
    const float* vbase = vc + (size_t)bh * T * HD;

    float q[HD], o[HD];
#pragma unroll
    for (int d = 0; d < HD; ++d) {
        q[d] = active ? qkv[row * qkv_ld + h * HD + d] : 0.0f;
        o[d] = 0.0f;
    }
    float m = -INFINITY, l = 0.0f;
    const int last_row = min(rows_per_seq, qb * 64 + 64) - 1;  // highest query in the block
    for (int t0 = 0; t0 <= last_row; t0 += kTile) {
        __syncthreads();
        for (int e = lane; e < kTile * HD; e += 64) {
            const int j = e / HD, d = e % HD;
            const int pos = t0 + j;
            Ks[j][d] = pos <= last_row ? kbase[(size_t)pos * HD + d] : 0.0f;
            Vs[j][d] = pos <= last_row ? vbase[(size_t)pos * HD + d] : 0.0f;
        }
        __syncthreads();
        if (!active) continue;
        const int jmax = min(kTile, i - t0 + 1);  // keys t0 .. i
        for (int j0 = 0; j0 < jmax; j0 += kChunk) {
            float s[kChunk];
            float cmax = -INFINITY;
#pragma unroll
            for (int jj = 0; jj < kChunk; ++jj) {
                const int j = j0 + jj;
                float acc = 0.0f;
                if (j < jmax) {
#pragma unroll
                    for (int d = 0; d < HD; ++d) acc += q[d] * Ks[j][d];
                    acc *= scale;
                } else {
                    acc = -INFINITY;
                }
                s[jj] = acc;
                cmax = fmaxf(cmax, acc);
            }
            const float mnew = fmaxf(m, cmax);
            const float corr = expf(m - mnew);  // m = -inf on the first chunk -> 0
            l *= corr;
#pragma unroll
            for (int d = 0; d < HD; ++d) o[d] *= corr;
#pragma unroll
            for (int jj = 0; jj < kChunk; ++jj) {
                const int j = j0 + jj;
                if (j < jmax) {
                    const float p = expf(s[jj] - mnew);
                    l += p;
#pragma unroll
                    for (int d = 0; d < HD; ++d) o[d] += p * Vs[j][d];
                }
            }
            m = mnew;
        }
    }
    if (active) {
        const float inv = 1.0f / l;
        float* dst = y + row * y_ld + h * HD;
#pragma unroll
        for (int d = 0; d < HD; ++d) dst[d] = o[d] * inv;
    }
}

constexpr int kDecChunk = 256;  // cached positions per decode work-group
constexpr int kCombineChunks = 16;  // chunk partials merged from registers (block_size 4096)

__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One (sequence, head, chunk).  pos: the query position (keys 0..pos are valid).
// QP: qkv holds `splits` split-K partial sums of the QKV product ([split][row][qkv_ld], plane
// floats apart) instead of the product: the work-group adds its head's q, k and v columns in
// split order (splitk_reduce_kernel's order), writes the step's K / V row to the caches (the
// work-group of the chunk holding pos) and takes that key from LDS.
// Every thread requests its key's K row and its share of the chunk's V rows before it waits
// for q, so the chunk costs one memory round trip.
// More than one chunk (DIRECT false): each chunk leaves (max, sum, unnormalised output) in
// `part` with agent-scope stores, then counts itself in cnt[sequence, head]; the work-group
// that counts last merges the chunks in chunk order (as a separate combine pass would) and
// writes y, then clears the count for the next call.  The partials bypass the per-XCD L2s
// (agent scope) and each work-group's stores have completed before it counts, so the last
// work-group reads every partial from the coherent level.
template <int HD, bool DIRECT, bool QP>
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const float* __restrict__ qkv, int qkv_ld, float* __restrict__ kc,
    float* __restrict__ vc, float* __restrict__ y, int y_ld, const int* __restrict__ d_pos,
    int H, int T, float scale, float* __restrict__ part, unsigned* __restrict__ cnt, int nchunks,
    int splits, size_t plane) {
    constexpr int DQ = HD / 4;    // float4 columns of a V row
    constexpr int G = 256 / DQ;   // key groups in the P.V phase
    constexpr int NV = kDecChunk / G;  // V rows per thread
    __shared__ float qs[HD];
    __shared__ float4 kvs4[QP ? 2 * HD / 4 : 1];  // the step's K and V rows (QP)
    __shared__ float ps[kDecChunk];
    __shared__ float red[4];
    __shared__ float4 red4[256];
    __shared__ float stat[2];
    __shared__ int last;
    const int tid = threadIdx.x;
    const int bh = blockIdx.x, chunk = blockIdx.y;
    const int b = bh / H, h = bh % H;
    const int pos = *d_pos;
    const int j0 = chunk * kDecChunk;
    float* kbase = kc + (size_t)bh * T * HD;
    float* vbase = vc + (size_t)bh * T * HD;
    float* pslot = DIRECT ? nullptr : part + ((size_t)bh * nchunks + chunk) * (HD + 2);
    const bool live = j0 <= pos;  // otherwise the chunk is entirely beyond the query
    const int nvalid = live ? min(kDecChunk, pos - j0 + 1) : 0;
    const bool has_pos = live && pos < j0 + kDecChunk;  // this chunk holds the step's own key
    const int j = j0 + tid;
    const int dq = tid % DQ, g = tid / DQ;
    // This thread's K row (key j) and V rows (keys g, g + G, ... of the chunk), requested now.
    float4 kr[DQ], vr[NV];
    if (live) {
        const float4* k4 = reinterpret_cast<const float4*>(kbase + (size_t)min(j, pos) * HD);
#pragma unroll
        for (int d = 0; d < DQ; ++d) kr[d] = k4[d];
        const float4* v4 = reinterpret_cast<const float4*>(vbase + (size_t)j0 * HD) + dq;
#pragma unroll
        for (int t = 0; t < NV; ++t) {
            const int jj = g + G * t;
            vr[t] = v4[(size_t)min(jj, nvalid - 1) * DQ];
        }
    }
    float* kvs = reinterpret_cast<float*>(kvs4);
    if (live && tid < HD) {
        const size_t e = (size_t)b * qkv_ld + h * HD + tid;
        if constexpr (QP) {
            const int C = H * HD;
            float q = 0.0f, k = 0.0f, v = 0.0f;
            for (int z = 0; z < splits; ++z) {
                const float* pz = qkv + (size_t)z * plane + e;
                q += pz[0];
                k += pz[C];
                v += pz[2 * C];
            }
            qs[tid] = q;
            kvs[tid] = k;
            kvs[HD + tid] = v;
            if (has_pos) {
                kbase[(size_t)pos * HD + tid] = k;
                vbase[(size_t)pos * HD + tid] = v;
            }
        } else {
            qs[tid] = qkv[e];
        }
    }
    __syncthreads();
    if (live) {
        float s = -INFINITY;
        if (j <= pos) {
            float acc = 0.0f;
            const bool own = QP && j == pos;
#pragma unroll
            for (int d = 0; d < HD; d += 4) {
                const float4 kv = own ? kvs4[d / 4] : kr[d / 4];
                acc += qs[d] * kv.x + qs[d + 1] * kv.y + qs[d + 2] * kv.z + qs[d + 3] * kv.w;
            }
            s = acc * scale;
        }
        // chunk max
        float mx = wave_max(s);
        if (tid % 64 == 0) red[tid / 64] = mx;
        __syncthreads();
        if (tid == 0) stat[0] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        __syncthreads();
        const float m = stat[0];
        const float p = (j <= pos) ? expf(s - m) : 0.0f;
        ps[tid] = p;
        float sm = wave_sum(p);
        __syncthreads();
        if (tid % 64 == 0) red[tid / 64] = sm;
        __syncthreads();
        if (tid == 0) stat[1] = (red[0] + red[1]) + (red[2] + red[3]);
        __syncthreads();
        // o[d] = sum_j p_j V[j][d]: thread (g, dq) sums keys g, g+G, ... over dims 4 dq .. 4 dq + 3,
        // then the G groups add up in group order.
        float4 acc4 = make_float4(0.f, 0.f, 0.f, 0.f);
        const int jpos = (QP && has_pos) ? pos - j0 : -1;  // the step's own key, from LDS
#pragma unroll
        for (int t = 0; t < NV; ++t) {
            const int jj = g + G * t;
            if (jj < nvalid) {
                const float4 vv = jj == jpos ? kvs4[HD / 4 + dq] : vr[t];
                const float pj = ps[jj];
                acc4.x += pj * vv.x;
                acc4.y += pj * vv.y;
                acc4.z += pj * vv.z;
                acc4.w += pj * vv.w;
            }
        }
        red4[tid] = acc4;
        __syncthreads();
        if (tid < HD) {
            const float* rf = reinterpret_cast<const float*>(red4);
            float o = 0.0f;
#pragma unroll
            for (int gg = 0; gg < G; ++gg) o += rf[gg * HD + tid];
            if (DIRECT) {
                y[(size_t)b * y_ld + h * HD + tid] = o / stat[1];
            } else {
                store_coherent(pslot + 2 + tid, o);
                if (tid == 0) {
                    store_coherent(pslot, m);
                    store_coherent(pslot + 1, stat[1]);
                }
            }
        }
    }
    if constexpr (!DIRECT) {
        // Ordering.  The count is a relaxed atomic, so the language model alone does not order
        // the partials before it; the instructions do.  Every partial word is written and read
        // only by agent-scope atomic instructions (store_coherent / load_coherent: sc1 stores
        // and loads, which the per-XCD L2s do not keep), so the agent-scope release and acquire
        // fences would add nothing for them but an L2 writeback / invalidate of unrelated lines
        // (device-scope fences in a split-K reduction of the batched decode took it from 208k
        // to 142k tok/s).  What release
        // must guarantee -- each partial store acknowledged at the agent coherence point
        // before the count is incremented -- is the vmcnt(0) wait below followed by the
        // barrier; the last work-group issues its partial loads only after the count's result
        // has come back (the barrier after `last`), so they are served from that same point.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores are done
        __syncthreads();
        if (tid == 0) {
            const unsigned prev = __hip_atomic_fetch_add(cnt + bh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = prev == (unsigned)(nchunks - 1);
        }
        __syncthreads();
        if (!last) return;
        // Merge the chunks holding keys (chunk c is live iff 256 c <= pos), in chunk order.
        const int nlive = min(nchunks, pos / kDecChunk + 1);
        if (tid < HD) {
            const float* base = part + (size_t)bh * nchunks * (HD + 2);
            float m = -INFINITY, l = 0.0f, o = 0.0f;
            float pm[kCombineChunks], pl[kCombineChunks], po[kCombineChunks];
            for (int c0 = 0; c0 < nlive; c0 += kCombineChunks) {
#pragma unroll
                for (int c = 0; c < kCombineChunks; ++c) {
                    if (c0 + c < nlive) {
                        const float* pc = base + (size_t)(c0 + c) * (HD + 2);
                        pm[c] = load_coherent(pc);
                        pl[c] = load_coherent(pc + 1);
                        po[c] = load_coherent(pc + 2 + tid);
                    }
                }
                float mn = m;
#pragma unroll
                for (int c = 0; c < kCombineChunks; ++c)
                    if (c0 + c < nlive) mn = fmaxf(mn, pm[c]);
                if (mn != m && m != -INFINITY) {  // rescale what earlier batches summed
                    const float w = expf(m - mn);
                    l *= w;
                    o *= w;
                }
                m = mn;
#pragma unroll
                for (int c = 0; c < kCombineChunks; ++c) {
                    if (c0 + c < nlive && pl[c] != 0.0f) {
                        const float w = expf(pm[c] - m);
                        l += w * pl[c];
                        o += w * po[c];
                    }
                }
            }
            y[(size_t)b * y_ld + h * HD + tid] = o / l;
        }
        if (tid == 0) __hip_atomic_store(cnt + bh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// qkv rows -> cache.  Row m belongs to sequence m / rows_per_seq at position
// pos0 + m % rows_per_seq, with pos0 = *d_pos when d_pos is given.
__global__ void kv_scatter_kernel(const float* __restrict__ qkv, int qkv_ld, float* __restrict__ kc,
                                  float* __restrict__ vc, int rows, int rows_per_seq, int C, int H,
                                  int HDv, int T, const int* __restrict__ d_pos, int pos0) {
    const int base = d_pos ? *d_pos : pos0;
    const size_t total = (size_t)rows * C;
    for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < total;
         e += (size_t)gridDim.x * blockDim.x) {
        const int m = (int)(e / C), c = (int)(e % C);
        const int b = m / rows_per_seq, p = base + m % rows_per_seq;
        const int h = c / HDv, d = c % HDv;
        const size_t dst = (((size_t)b * H + h) * T + p) * HDv + d;
        kc[dst] = qkv[(size_t)m * qkv_ld + C + c];
        vc[dst] = qkv[(size_t)m * qkv_ld + 2 * C + c];
    }
}

}  // namespace

int kv_scatter(const float* qkv, int qkv_ld, float* kc, float* vc, int rows, int rows_per_seq,
               int C, int H, int T, const int* d_pos, int pos0, hipStream_t s) {
    const size_t total = (size_t)rows * C;
    hipLaunchKernelGGL(kv_scatter_kernel, dim3(blocks_for(total, 256, 4096u)), dim3(256), 0, s,
                       qkv, qkv_ld, kc, vc, rows, rows_per_seq, C, H, C / H, T, d_pos, pos0);
    FMLH_LAUNCHED("kv_scatter_kernel");
    return FMLH_OK;
}

// ---- prefill on the matrix cores -----------------------------------------------------------
//
// One work-group of 4 waves per 64 query rows of one (sequence, head); wave v owns queries
// q0 = 64 qb + 16 v .. +15.  Per 64-key tile (up to the diagonal):
//   S = Q K^T     16 x 64 per wave: 4 blocks of v_mfma_f32_16x16x4f32 over HD/4 k-steps
//   online softmax per query row (running max m, per-lane partial sums l)
//   O += P V      P goes through the wave's LDS rows to become the A operand
// MFMA 16x16x4 layouts (lane l, r = l % 16, g = l / 16): A[r][g], B[g][r], D[4g + i][r] in
// register i.  A query row's 16 S values sit in one 16-lane DPP row, so row max / sum need no
// cross-row shuffles, and the O rows (4g + i) line up with the S rows for the rescale.  The
// k-step -> head-dim assignment is d = g * HD/4 + s (any bijection sums all dims), so a lane
// reads HD/4 consecutive floats of a K row; keys in P.V likewise use key = 16 g + s.
namespace {

using f32x4 = __attribute__((ext_vector_type(4))) float;
using floatx16 = __attribute__((ext_vector_type(16))) float;
using f32x2 = __attribute__((ext_vector_type(2))) float;

template <int kCtrl>
__device__ __forceinline__ float row16_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}
// Max / sum over the 16 lanes of a DPP row, result in every lane of the row (row_ror 8, 4, 2, 1).
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, row16_move<0x128>(v));
    v = fmaxf(v, row16_move<0x124>(v));
    v = fmaxf(v, row16_move<0x122>(v));
    v = fmaxf(v, row16_move<0x121>(v));
    return v;
}
__device__ __forceinline__ float row16_sum(float v) {
    v += row16_move<0x128>(v);
    v += row16_move<0x124>(v);
    v += row16_move<0x122>(v);
    v += row16_move<0x121>(v);
    return v;
}

template <int HD>
__global__ __launch_bounds__(256) void attn_prefill_mfma_kernel(
    const float* __restrict__ qkv, int qkv_ld, const float* __restrict__ kc,
    const float* __restrict__ vc, float* __restrict__ y, int y_ld, int rows_per_seq, int H,
    int T, float scale) {
    constexpr int KT = 64;       // keys per tile
    constexpr int KS = HD / 4;   // MFMA k-steps over the head dims (dims per lane group)
    constexpr int NB = HD / 16;  // 16-wide blocks of output dims
    constexpr int LDK = HD + 4;  // padded LDS strides (bank spread)
    constexpr int LDP = KT + 4;
    __shared__ float Ks[KT * LDK];       // K tile [key][dim]
    __shared__ float Vt[HD * LDP];       // V tile transposed [dim][key]
    __shared__ float Ps[4 * 16 * LDP];   // per wave: P [query][key]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, g = lane >> 4;
    // Work-groups are dispatched x-fastest: every (sequence, head) of a query block, the
    // longest (latest) query blocks first.
    const int qb = gridDim.y - 1 - blockIdx.y;
    const int bh = blockIdx.x, b = bh / H, h = bh % H;
    const int q0 = qb * 64 + wave * 16;
    const int last_q = min(rows_per_seq, qb * 64 + 64) - 1;  // last query of the work-group
    const float* kbase = kc + (size_t)bh * T * HD;
    const float* vbase = vc + (size_t)bh * T * HD;
    float* pw = Ps + wave * 16 * LDP;

    // Q operand: row q0 + r, dims g*KS .. g*KS + KS - 1 (rows past the sequence read its last
    // row: their results are not stored).
    float qa[KS];
    {
        const int qrow = min(q0 + r, rows_per_seq - 1);
        const float* qp = qkv + ((size_t)b * rows_per_seq + qrow) * qkv_ld + h * HD + g * KS;
#pragma unroll
        for (int s = 0; s < KS; s += 4) {
            const float4 v = *reinterpret_cast<const float4*>(qp + s);
            qa[s] = v.x; qa[s + 1] = v.y; qa[s + 2] = v.z; qa[s + 3] = v.w;
        }
    }
    f32x4 o[NB];
#pragma unroll
    for (int n = 0; n < NB; ++n) o[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) { m[i] = -INFINITY; l[i] = 0.f; }

    constexpr int kPer = KT * HD / 4 / 256;  // float4 of the K (and of the V) tile per thread
    static_assert(kPer * 256 * 4 == KT * HD, "tile must split evenly over the threads");
    for (int t0 = 0; t0 <= last_q; t0 += KT) {
        // Every load of the thread's share of the tile goes out before any LDS write (one
        // memory round trip per tile).  Keys past the work-group's last query read that
        // query's row: finite values, masked out of the scores, weight 0 in P.V.
        f32x4 kv[kPer], vv[kPer];  // vector elements: registers (a float4 array goes to LDS)
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int e = tid + 256 * u;
            {   // K row-major: consecutive threads take consecutive float4 of a row
                const int key = e / (HD / 4), d4 = e - key * (HD / 4);
                kv[u] = *reinterpret_cast<const f32x4*>(kbase + (size_t)min(t0 + key, last_q) * HD + 4 * d4);
            }
            {   // V transposed: consecutive threads take consecutive keys (conflict-free writes)
                const int key = e % KT, d4 = e / KT;
                vv[u] = *reinterpret_cast<const f32x4*>(vbase + (size_t)min(t0 + key, last_q) * HD + 4 * d4);
            }
        }
        __syncthreads();  // previous tile's K / V reads are done
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int e = tid + 256 * u;
            {
                const int key = e / (HD / 4), d4 = e - key * (HD / 4);
                *reinterpret_cast<f32x4*>(&Ks[key * LDK + 4 * d4]) = kv[u];
            }
            {
                const int key = e % KT, d4 = e / KT;
                Vt[(4 * d4 + 0) * LDP + key] = vv[u][0];
                Vt[(4 * d4 + 1) * LDP + key] = vv[u][1];
                Vt[(4 * d4 + 2) * LDP + key] = vv[u][2];
                Vt[(4 * d4 + 3) * LDP + key] = vv[u][3];
            }
        }
        __syncthreads();
        if (q0 >= rows_per_seq || t0 > q0 + 15) continue;  // no query of this wave sees the tile
        // S = Q K^T for keys t0 + 16 n + r.
        f32x4 sc[4];
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            sc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
            const float* kr = &Ks[(n * 16 + r) * LDK + g * KS];
#pragma unroll
            for (int s = 0; s < KS; s += 4) {
                const float4 kv = *reinterpret_cast<const float4*>(kr + s);
                sc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[s], kv.x, sc[n], 0, 0, 0);
                sc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[s + 1], kv.y, sc[n], 0, 0, 0);
                sc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[s + 2], kv.z, sc[n], 0, 0, 0);
                sc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[s + 3], kv.w, sc[n], 0, 0, 0);
            }
        }
        // Scale, causal mask (key > query -> excluded), online softmax per row 4g + i.
        const bool diag = t0 + KT - 1 > q0;  // the tile reaches past some query of the wave
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int qpos = q0 + 4 * g + i;
            float s4[4];
            float mt = -INFINITY;
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                const int kpos = t0 + n * 16 + r;
                const float sv = sc[n][i] * scale;
                s4[n] = (!diag || kpos <= qpos) ? sv : -INFINITY;
                mt = fmaxf(mt, s4[n]);
            }
            mt = row16_max(mt);
            const float mnew = fmaxf(m[i], mt);
            const float corr = expf(m[i] - mnew);  // m = -inf on the first tile -> 0
            m[i] = mnew;
            float ls = 0.f;
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                const float p = s4[n] == -INFINITY ? 0.f : expf(s4[n] - mnew);
                ls += p;
                pw[(4 * g + i) * LDP + n * 16 + r] = p;
            }
            l[i] = l[i] * corr + ls;
#pragma unroll
            for (int n = 0; n < NB; ++n) o[n][i] *= corr;
        }
        // O += P V: A = P[query r][key 16 g + s], B = V[key 16 g + s][dim 16 n + r].
        float pa[16];
#pragma unroll
        for (int s = 0; s < 16; s += 4) {
            const float4 v = *reinterpret_cast<const float4*>(&pw[r * LDP + 16 * g + s]);
            pa[s] = v.x; pa[s + 1] = v.y; pa[s + 2] = v.z; pa[s + 3] = v.w;
        }
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const float* vr = &Vt[(n * 16 + r) * LDP + 16 * g];
#pragma unroll
            for (int s = 0; s < 16; s += 4) {
                const float4 vv = *reinterpret_cast<const float4*>(vr + s);
                o[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[s], vv.x, o[n], 0, 0, 0);
                o[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[s + 1], vv.y, o[n], 0, 0, 0);
                o[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[s + 2], vv.z, o[n], 0, 0, 0);
                o[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[s + 3], vv.w, o[n], 0, 0, 0);
            }
        }
    }
    if (q0 >= rows_per_seq) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int qpos = q0 + 4 * g + i;
        const float inv = 1.0f / row16_sum(l[i]);
        if (qpos < rows_per_seq) {
            float* dst = y + ((size_t)b * rows_per_seq + qpos) * y_ld + h * HD;
#pragma unroll
            for (int n = 0; n < NB; ++n) dst[n * 16 + r] = o[n][i] * inv;
        }
    }
}

// ---- prefill, head_dim 64, on v_mfma_f32_32x32x2f32 ----------------------------------------
//
// One work-group of 4 waves per 128 query rows of one (sequence, head); wave v owns the 32
// queries q0 = 128 qb + 32 v .. +31, one per lane column c = lane % 32 (h = lane / 32).  Per
// 64-key tile up to the diagonal, with the products taken transposed:
//   S^T (64 keys x 32 queries) = K Q^T       2 blocks of 32 keys x 32 k-steps over the dims
//   O^T (64 dims x 32 queries) += V^T P^T    2 blocks of 32 dims x 32 k-steps over the keys
// MFMA 32x32x2 layouts: A (32 x 2) lane supplies A[c][h], B (2 x 32) B[h][c], D (32 x 32)
// D[8 (r/4) + 4h + r%4][c] in register r.  So lane (h, c) holds, for query c, the scores of
// keys 32 j + 8 (r/4) + 4h + r%4 (block j, register r) -- half of the tile's keys, the other
// half in lane c ^ 32.  The row max needs one exchange between the halves; the sum stays a
// per-lane partial until the end; O^T's registers all belong to query c, so the rescale is
// lane-local.  Taking the P^T k-step t as key 32 (t/16) + 8 ((t%16)/4) + 4h + t%4 makes
// register t%16 of score block t/16 exactly lane (h, c)'s B operand: P never leaves registers.
// The Q k-step t is dim 32h + t (Q row c's half h in 32 registers); row rho of O^T block i
// is dim 2 rho + i.
//
// K and V tiles are copied global -> LDS directly (global_load_lds), two stages: the copy of
// tile t+1 runs while tile t is multiplied.  Rows are 256 bytes, stored with their 16-byte
// quads permuted so both read patterns are conflict-free: K (32 lanes read one quad of 32
// different rows) at quad q ^ (row % 16); V (each half-wave reads a whole key row, 8 bytes
// per lane, the two halves keys 4 apart) at quad q ^ 8 (key bit 2).  Keys past the work-group's last query copy
// that query's key row (finite values, masked out).
constexpr int kAttnQPerWave = 32;
constexpr int kAttnQPerWG = 4 * kAttnQPerWave;
constexpr int kAttnKT = 64;                                        // keys per tile
constexpr size_t kAttnMfma32Lds = 2 * 2 * kAttnKT * 64 * sizeof(float);  // 2 stages x (K, V)

__device__ __forceinline__ int attn_k_swz(int row) { return row & 15; }
__device__ __forceinline__ int attn_v_swz(int row) { return ((row >> 2) & 1) << 3; }

__global__ __launch_bounds__(256) void attn_prefill_mfma32_kernel(
    const float* __restrict__ qkv, int qkv_ld, const float* __restrict__ kc,
    const float* __restrict__ vc, float* __restrict__ y, int y_ld, int rows_per_seq, int H,
    int T, float scale_log2) {
    constexpr int HD = 64;
    constexpr int TILE = kAttnKT * HD;  // floats of one K or V tile
    extern __shared__ __attribute__((aligned(16))) float lds[];  // [stage][K | V][64][64]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, c = lane & 31;
    // Dispatched x-fastest: every (sequence, head) of a query block, longest blocks first.
    const int qb = gridDim.y - 1 - blockIdx.y;
    const int bh = blockIdx.x, b = bh / H, hh = bh % H;
    const int q0 = qb * kAttnQPerWG + wave * kAttnQPerWave;
    const int last_q = min(rows_per_seq, (qb + 1) * kAttnQPerWG) - 1;  // work-group's last query
    const int ntiles = last_q / kAttnKT + 1;
    const float* kbase = kc + (size_t)bh * T * HD;
    const float* vbase = vc + (size_t)bh * T * HD;

    // Copy assignment: chunk (wave + 4 u) of a tile = rows 4 chunk .. +3; lane -> row
    // 4 chunk + lane / 16, stored quad lane % 16, which holds global quad (lane % 16) ^ swz(row).
    const int crow_in = lane >> 4, cpos = lane & 15;
    auto issue = [&](int tile, int st) {
        float* kd = lds + st * 2 * TILE;
        float* vd = kd + TILE;
        const int t0 = tile * kAttnKT;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int chunk = wave + 4 * u;
            const int row = 4 * chunk + crow_in;
            const size_t src = (size_t)min(t0 + row, last_q) * HD;
            copy16_to_lds(kd + chunk * 256, kbase + src + 4 * (cpos ^ attn_k_swz(row)));
            copy16_to_lds(vd + chunk * 256, vbase + src + 4 * (cpos ^ attn_v_swz(row)));
        }
    };
    issue(0, 0);

    // Q^T operand: lane (h, c) holds Q[q0 + c][32h .. 32h + 31] (rows past the sequence read
    // its last row; their results are not stored).
    const bool wave_live = q0 < rows_per_seq;
    float qv[32];
    {
        const int qrow = min(q0 + c, rows_per_seq - 1);
        const float* qp = qkv + ((size_t)b * rows_per_seq + qrow) * qkv_ld + hh * HD + 32 * h;
#pragma unroll
        for (int t = 0; t < 32; t += 4) {
            const float4 v = *reinterpret_cast<const float4*>(qp + t);
            qv[t] = v.x; qv[t + 1] = v.y; qv[t + 2] = v.z; qv[t + 3] = v.w;
        }
    }
    floatx16 o[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
    float mrun = -INFINITY, lsum = 0.f;
    const int qpos = q0 + c;

    for (int tile = 0; tile < ntiles; ++tile) {
        // Tile `tile` has landed in every wave's part; all reads of the other stage are done.
        copies_barrier<0>();
        if (tile + 1 < ntiles) issue(tile + 1, (tile + 1) & 1);
        const int t0 = tile * kAttnKT;
        if (!wave_live || t0 > q0 + kAttnQPerWave - 1) continue;  // no query of the wave sees it
        const float* ks = lds + (tile & 1) * 2 * TILE;
        const float* vs = ks + TILE;

        // S^T = K Q^T.
        floatx16 s[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) s[j][r] = 0.f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {  // quads 8h + u of key rows c and 32 + c
            f32x4 ka[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int row = 32 * j + c;
                ka[j] = *reinterpret_cast<const f32x4*>(ks + row * HD + 4 * ((8 * h + u) ^ attn_k_swz(row)));
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    s[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[j][e], qv[4 * u + e], s[j], 0, 0, 0);
        }

        // Online softmax for query c over this lane's 32 keys and the partner half's.
        const bool diag = t0 + kAttnKT - 1 > q0;  // some key of the tile follows some query
        float mt = -INFINITY;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float v = s[j][r] * scale_log2;
                if (diag) {
                    const int kpos = t0 + 32 * j + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (kpos > qpos) v = -INFINITY;
                }
                s[j][r] = v;
                mt = fmaxf(mt, v);
            }
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mnew = fmaxf(mrun, mt);  // finite: tile 0 holds key 0 <= every query
        const float corr = exp2f(mrun - mnew);
        mrun = mnew;
        float ls = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = exp2f(s[j][r] - mnew);
                s[j][r] = p;
                ls += p;
            }
        lsum = lsum * corr + ls;
        if (__ballot(corr != 1.0f)) {  // some query's running max moved
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[i][r] *= corr;
        }

        // O^T += V^T P^T: k-step t -> key 32 (t/16) + 8 ((t%16)/4) + 4h + t%4.  Row rho of O^T
        // block i is dim 2 rho + i, so lane (h, c) takes dims 2c and 2c+1 of a key in one 8-byte
        // read; a half tile's 16 reads go out before its 32 MFMAs.
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            f32x2 va[16];
#pragma unroll
            for (int tt = 0; tt < 16; ++tt) {
                const int key = 32 * j + 8 * (tt >> 2) + 4 * h + (tt & 3);
                va[tt] = *reinterpret_cast<const f32x2*>(
                    vs + key * HD + 4 * ((c >> 1) ^ attn_v_swz(key)) + 2 * (c & 1));
            }
#pragma unroll
            for (int tt = 0; tt < 16; ++tt) {
                o[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[tt].x, s[j][tt], o[0], 0, 0, 0);
                o[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[tt].y, s[j][tt], o[1], 0, 0, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);  // LDS reads
            __builtin_amdgcn_sched_group_barrier(0x008, 32, 0);  // MFMA
        }
    }
    if (!wave_live) return;
    const float inv = 1.0f / (lsum + __shfl_xor(lsum, 32));
    if (qpos < rows_per_seq) {
        float* dst = y + ((size_t)b * rows_per_seq + qpos) * y_ld + hh * HD;
        // Register r of block i: dim 2 (8 (r/4) + 4h + r%4) + i.
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float4 lo = make_float4(o[0][4 * u] * inv, o[1][4 * u] * inv,
                                          o[0][4 * u + 1] * inv, o[1][4 * u + 1] * inv);
            const float4 hi = make_float4(o[0][4 * u + 2] * inv, o[1][4 * u + 2] * inv,
                                          o[0][4 * u + 3] * inv, o[1][4 * u + 3] * inv);
            *reinterpret_cast<float4*>(dst + 16 * u + 8 * h) = lo;
            *reinterpret_cast<float4*>(dst + 16 * u + 8 * h + 4) = hi;
        }
    }
}

}  // namespace

bool attn_head_dim_supported(int hd) { return hd == 16 || hd == 32 || hd == 64; }

int attn_prefill(const float* qkv, int qkv_ld, const float* kc, const float* vc, float* y,
                 int y_ld, int batch, int rows_per_seq, int H, int HDv, int T, float scale,
                 hipStream_t s) {
    dim3 grid(batch * H, (rows_per_seq + 63) / 64);
    // head_dim 64 from 256 rows per sequence on: attn_prefill_mfma32_kernel (interleaved A/B on
    // MI355X against the 16x16x4 kernel: c5 prefill 5.80 vs 6.16 ms, c4 equal; at 64 rows, half
    // of its 128-query blocks are empty: 15.1 vs 12.7 us per layer at c3); otherwise the 16x16x4
    // kernel, which FMLH_ATTN_PREFILL=mfma16 selects for every length and FMLH_ATTN_PREFILL=mfma32
    // replaces for every head_dim-64 length; FMLH_ATTN_PREFILL=simt: the per-lane kernel (the
    // one head_dim 16 always uses).  The alternatives serve comparisons.
    const char* env = std::getenv("FMLH_ATTN_PREFILL");
    const bool simt = env && std::strcmp(env, "simt") == 0;
    const bool mfma16 = env && std::strcmp(env, "mfma16") == 0;
    const bool mfma32 = env && std::strcmp(env, "mfma32") == 0;
    if (HDv == 64 && !simt && !mfma16 && (mfma32 || rows_per_seq >= 256)) {
        dim3 g32(batch * H, (rows_per_seq + kAttnQPerWG - 1) / kAttnQPerWG);
        hipLaunchKernelGGL(attn_prefill_mfma32_kernel, g32, dim3(256), kAttnMfma32Lds, s, qkv, qkv_ld,
                           kc, vc, y, y_ld, rows_per_seq, H, T, scale * 1.4426950408889634f);
        FMLH_LAUNCHED("attn_prefill_mfma32_kernel");
        return FMLH_OK;
    }
#define FMLH_PREFILL(HDC)                                                                    \
    hipLaunchKernelGGL(attn_prefill_kernel<HDC>, grid, dim3(64), 0, s, qkv, qkv_ld, kc, vc, y, \
                       y_ld, rows_per_seq, H, T, scale)
#define FMLH_PREFILL_MFMA(HDC)                                                                  \
    hipLaunchKernelGGL(attn_prefill_mfma_kernel<HDC>, grid, dim3(256), 0, s, qkv, qkv_ld, kc, vc, \
                       y, y_ld, rows_per_seq, H, T, scale)
    switch (HDv) {
        case 16: FMLH_PREFILL(16); break;
        case 32: if (simt) FMLH_PREFILL(32); else FMLH_PREFILL_MFMA(32); break;
        case 64: if (simt) FMLH_PREFILL(64); else FMLH_PREFILL_MFMA(64); break;
        default: return set_error(FMLH_E_INVALID, "attention: head_dim %d unsupported", HDv);
    }
#undef FMLH_PREFILL
#undef FMLH_PREFILL_MFMA
    FMLH_LAUNCHED("attn_prefill_kernel");
    return FMLH_OK;
}

// The arrival counts come first, max_batch * H of them (rounded up to 64 floats so that the
// partials stay 256-byte aligned), at the same offsets whatever a call's batch: a count slot is
// never part of another call's partials, so it holds zero between calls.
size_t attn_decode_counts(int max_batch, int H) { return ((size_t)max_batch * H + 63) / 64 * 64; }

size_t attn_decode_workspace(int max_batch, int H, int HDv, int T) {
    const int nchunks = (T + kDecChunk - 1) / kDecChunk;
    return nchunks > 1 ? attn_decode_counts(max_batch, H) + (size_t)max_batch * H * nchunks * (HDv + 2) : 0;
}

int attn_decode(const float* qkv, int qkv_ld, float* kc, float* vc, float* y, int y_ld,
                int batch, int H, int HDv, int T, const int* d_pos, float scale, float* ws,
                int max_batch, hipStream_t s, int qkv_splits) {
    const int nchunks = (T + kDecChunk - 1) / kDecChunk;
    FMLH_REQUIRE(batch >= 1 && batch <= max_batch, "attn_decode: batch %d outside [1, %d]", batch, max_batch);
    FMLH_REQUIRE(nchunks == 1 || ws != nullptr, "attn_decode: %d key chunks need the workspace", nchunks);
    dim3 grid(batch * H, nchunks);
    const size_t plane = (size_t)batch * qkv_ld;
    unsigned* cnt = nchunks > 1 ? reinterpret_cast<unsigned*>(ws) : nullptr;
    float* part = nchunks > 1 ? ws + attn_decode_counts(max_batch, H) : nullptr;
#define FMLH_DECODE_QP(HDC, QPV)                                                                 \
    do {                                                                                         \
        if (nchunks == 1) {                                                                      \
            hipLaunchKernelGGL((attn_decode_kernel<HDC, true, QPV>), grid, dim3(256), 0, s, qkv,   \
                               qkv_ld, kc, vc, y, y_ld, d_pos, H, T, scale, nullptr, nullptr, 1, \
                               qkv_splits, plane);                                               \
        } else {                                                                                 \
            hipLaunchKernelGGL((attn_decode_kernel<HDC, false, QPV>), grid, dim3(256), 0, s, qkv,  \
                               qkv_ld, kc, vc, y, y_ld, d_pos, H, T, scale, part, cnt, nchunks,  \
                               qkv_splits, plane);                                               \
        }                                                                                        \
    } while (0)
#define FMLH_DECODE(HDC)                                   \
    do {                                                   \
        if (qkv_splits > 0) FMLH_DECODE_QP(HDC, true);     \
        else FMLH_DECODE_QP(HDC, false);                   \
    } while (0)
    switch (HDv) {
        case 16: FMLH_DECODE(16); break;
        case 32: FMLH_DECODE(32); break;
        case 64: FMLH_DECODE(64); break;
        default: return set_error(FMLH_E_INVALID, "attention: head_dim %d unsupported", HDv);
    }
#undef FMLH_DECODE
#undef FMLH_DECODE_QP
    FMLH_LAUNCHED("attn_decode");
    return FMLH_OK;
}

}  // namespace fmlh
