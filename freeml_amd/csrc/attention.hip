// Causal self-attention over the device KV cache (CausalSelfAttentionLayer::Forward,
// CausalSelfAttentionLayer.h:424-499: S = Q_h K_h^T * (1/sqrt(hd)) + causal -inf mask,
// row softmax, Y_h = P V_h).  The reference materialises every T x T score matrix; here no
// score matrix is stored:
//   * prefill: one wave per 64 query rows of one (sequence, head), keys streamed through LDS
//     in 64-key tiles up to the diagonal, online softmax (running max / sum) per query row;
//   * decode: one query row per (sequence, head), the cached keys split into 256-position
//     chunks across work-groups; each chunk leaves (max, sum, unnormalised output) and a
//     combine kernel merges the chunks in chunk order.
// Masked positions (j > i) are skipped: in the reference they contribute exp(-inf) = 0.
//
// KV cache layout: [layer][sequence][head][position][head_dim], fp32.
#include "attention.h"

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
    const int qb = blockIdx.x;          // query block
    const int bh = blockIdx.y;          // sequence * H + head
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

// One (sequence, head, chunk).  pos: the query position (keys 0..pos are valid).
template <int HD, bool DIRECT>
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const float* __restrict__ qkv, int qkv_ld, const float* __restrict__ kc,
    const float* __restrict__ vc, float* __restrict__ y, int y_ld, const int* __restrict__ d_pos,
    int H, int T, float scale, float* __restrict__ part, int nchunks) {
    constexpr int G = 256 / HD;  // key groups in the P.V phase
    __shared__ float qs[HD];
    __shared__ float ps[kDecChunk];
    __shared__ float red[256];
    __shared__ float stat[2];
    const int tid = threadIdx.x;
    const int bh = blockIdx.x, chunk = blockIdx.y;
    const int b = bh / H, h = bh % H;
    const int pos = *d_pos;
    const int j0 = chunk * kDecChunk;
    const float* kbase = kc + (size_t)bh * T * HD;
    const float* vbase = vc + (size_t)bh * T * HD;
    float* pslot = DIRECT ? nullptr : part + ((size_t)bh * nchunks + chunk) * (HD + 2);
    if (j0 > pos) {  // chunk entirely beyond the query: empty partial
        if (!DIRECT) {
            if (tid < HD) pslot[2 + tid] = 0.0f;
            if (tid == 0) { pslot[0] = -INFINITY; pslot[1] = 0.0f; }
        }
        return;
    }
    if (tid < HD) qs[tid] = qkv[(size_t)b * qkv_ld + h * HD + tid];
    __syncthreads();
    const int j = j0 + tid;
    float s = -INFINITY;
    if (j <= pos) {
        const float* kr = kbase + (size_t)j * HD;
        float acc = 0.0f;
#pragma unroll
        for (int d = 0; d < HD; d += 4) {
            const float4 kv = *reinterpret_cast<const float4*>(kr + d);
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
    // o[d] = sum_j p_j V[j][d]: thread (g, d) sums keys g, g+G, ...
    const int d = tid % HD, g = tid / HD;
    const int nvalid = min(kDecChunk, pos - j0 + 1);
    float acc = 0.0f;
    for (int jj = g; jj < nvalid; jj += G) acc += ps[jj] * vbase[(size_t)(j0 + jj) * HD + d];
    red[tid] = acc;
    __syncthreads();
    if (tid < HD) {
        float o = 0.0f;
#pragma unroll
        for (int gg = 0; gg < G; ++gg) o += red[gg * HD + tid];
        if (DIRECT) {
            y[(size_t)b * y_ld + h * HD + tid] = o / stat[1];
        } else {
            pslot[2 + tid] = o;
            if (tid == 0) { pslot[0] = m; pslot[1] = stat[1]; }
        }
    }
}

// Merges the chunk partials of one (sequence, head) in chunk order.
template <int HD>
__global__ __launch_bounds__(HD) void attn_combine_kernel(const float* __restrict__ part,
                                                         int nchunks, float* __restrict__ y,
                                                         int y_ld, int H) {
    const int bh = blockIdx.x, d = threadIdx.x;
    const int b = bh / H, h = bh % H;
    const float* base = part + (size_t)bh * nchunks * (HD + 2);
    float m = -INFINITY;
    for (int c = 0; c < nchunks; ++c) m = fmaxf(m, base[(size_t)c * (HD + 2)]);
    float l = 0.0f, o = 0.0f;
    for (int c = 0; c < nchunks; ++c) {
        const float* p = base + (size_t)c * (HD + 2);
        if (p[1] == 0.0f) continue;
        const float w = expf(p[0] - m);
        l += w * p[1];
        o += w * p[2 + d];
    }
    y[(size_t)b * y_ld + h * HD + d] = o / l;
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

bool attn_head_dim_supported(int hd) { return hd == 16 || hd == 32 || hd == 64; }

int attn_prefill(const float* qkv, int qkv_ld, const float* kc, const float* vc, float* y,
                 int y_ld, int batch, int rows_per_seq, int H, int HDv, int T, float scale,
                 hipStream_t s) {
    dim3 grid((rows_per_seq + 63) / 64, batch * H);
#define FMLH_PREFILL(HDC)                                                                    \
    hipLaunchKernelGGL(attn_prefill_kernel<HDC>, grid, dim3(64), 0, s, qkv, qkv_ld, kc, vc, y, \
                       y_ld, rows_per_seq, H, T, scale)
    switch (HDv) {
        case 16: FMLH_PREFILL(16); break;
        case 32: FMLH_PREFILL(32); break;
        case 64: FMLH_PREFILL(64); break;
        default: return set_error(FMLH_E_INVALID, "attention: head_dim %d unsupported", HDv);
    }
#undef FMLH_PREFILL
    FMLH_LAUNCHED("attn_prefill_kernel");
    return FMLH_OK;
}

size_t attn_decode_workspace(int batch, int H, int HDv, int T) {
    const int nchunks = (T + kDecChunk - 1) / kDecChunk;
    return nchunks > 1 ? (size_t)batch * H * nchunks * (HDv + 2) : 0;
}

int attn_decode(const float* qkv, int qkv_ld, const float* kc, const float* vc, float* y, int y_ld,
                int batch, int H, int HDv, int T, const int* d_pos, float scale, float* ws,
                hipStream_t s) {
    const int nchunks = (T + kDecChunk - 1) / kDecChunk;
    dim3 grid(batch * H, nchunks);
#define FMLH_DECODE(HDC)                                                                         \
    do {                                                                                         \
        if (nchunks == 1) {                                                                      \
            hipLaunchKernelGGL((attn_decode_kernel<HDC, true>), grid, dim3(256), 0, s, qkv, qkv_ld, \
                               kc, vc, y, y_ld, d_pos, H, T, scale, nullptr, 1);                 \
        } else {                                                                                 \
            hipLaunchKernelGGL((attn_decode_kernel<HDC, false>), grid, dim3(256), 0, s, qkv,       \
                               qkv_ld, kc, vc, y, y_ld, d_pos, H, T, scale, ws, nchunks);        \
            FMLH_LAUNCHED("attn_decode_kernel");                                                 \
            hipLaunchKernelGGL(attn_combine_kernel<HDC>, dim3(batch * H), dim3(HDC), 0, s, ws,    \
                               nchunks, y, y_ld, H);                                             \
        }                                                                                        \
    } while (0)
    switch (HDv) {
        case 16: FMLH_DECODE(16); break;
        case 32: FMLH_DECODE(32); break;
        case 64: FMLH_DECODE(64); break;
        default: return set_error(FMLH_E_INVALID, "attention: head_dim %d unsupported", HDv);
    }
#undef FMLH_DECODE
    FMLH_LAUNCHED("attn_decode");
    return FMLH_OK;
}

}  // namespace fmlh
