// Training-step ops of the C ABI: the backward, loss and optimiser routines FreeML's layers
// call during Model::Run(input, target) (ModelLibrary/Model.h:790-878), for the MatrixHIP<float>
// overload set.  Each kernel states the reference routine whose result it reproduces.
//
// All of these are memory-bound element or row passes; none has a GEMM shape (the products of
// the backward go through fmlh_mul / fmlh_matmul_strided).
#include "fmlh_internal.h"

namespace fmlh {

namespace {

constexpr unsigned kThreads = 256;

__device__ float block_sum(float v, float* sh) {
    v = wave_sum(v);
    const unsigned w = threadIdx.x / kWave, nw = blockDim.x / kWave;
    __syncthreads();
    if (threadIdx.x % kWave == 0) sh[w] = v;
    __syncthreads();
    float r = 0.0f;
    for (unsigned i = 0; i < nw; ++i) r += sh[i];
    return r;
}

__device__ float block_max(float v, float* sh) {
    v = wave_max(v);
    const unsigned w = threadIdx.x / kWave, nw = blockDim.x / kWave;
    __syncthreads();
    if (threadIdx.x % kWave == 0) sh[w] = v;
    __syncthreads();
    float r = -INFINITY;
    for (unsigned i = 0; i < nw; ++i) r = fmaxf(r, sh[i]);
    return r;
}

// SoftmaxBackwards (MatrixBase_Functions.h:83-111): per row dot = sum(dp * p), then
// out = p * (dp - dot).  One block per row; out may alias dp (each element is read by the
// thread that writes it, after the row's reduction).
__global__ void softmax_backward_kernel(float* out, const float* p, const float* dp, uint32_t cols) {
    __shared__ float sh[kThreads / kWave];
    const size_t base = (size_t)blockIdx.x * cols;
    float s = 0.0f;
    for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) s += dp[base + c] * p[base + c];
    const float dot = block_sum(s, sh);
    for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x)
        out[base + c] = p[base + c] * (dp[base + c] - dot);
}

// LayerNormBackwardsOp, parameter gradients (MatrixBase_Functions.h:595-656): dGamma[c] =
// sum over rows of dY * xHat (xHat recomputed from `in` when not stored), dBeta[c] = sum dY.
// One block per 64 columns; each of the block's waves sums a strided subset of the rows in
// row order and the waves' partial sums are added in wave order.
constexpr unsigned kLnbWaves = 16;

__global__ void layernorm_backward_params_kernel(float* __restrict__ dgamma, float* __restrict__ dbeta,
                                                 const float* __restrict__ dy,
                                                 const float* __restrict__ xhat,
                                                 const float* __restrict__ mean_inv,
                                                 const float* __restrict__ in, uint32_t rows,
                                                 uint32_t cols) {
    __shared__ float pg[kLnbWaves][kWave];
    __shared__ float pb[kLnbWaves][kWave];
    const uint32_t lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
    const uint32_t c = blockIdx.x * kWave + lane;
    float g = 0.0f, b = 0.0f;
    if (c < cols) {
        for (uint32_t r = w; r < rows; r += kLnbWaves) {
            const size_t i = (size_t)r * cols + c;
            const float d = dy[i];
            const float xh = xhat ? xhat[i] : (in[i] - mean_inv[2 * r]) * mean_inv[2 * r + 1];
            g += d * xh;
            b += d;
        }
    }
    pg[w][lane] = g;
    pb[w][lane] = b;
    __syncthreads();
    if (w == 0 && c < cols) {
        float sg = 0.0f, sb = 0.0f;
        for (uint32_t k = 0; k < kLnbWaves; ++k) {
            sg += pg[k][lane];
            sb += pb[k][lane];
        }
        dgamma[c] = sg;
        if (dbeta) dbeta[c] = sb;
    }
}

// LayerNormBackwardsOp, input gradient (MatrixBase_Functions.h:658-705), one wave per row:
// mean, two-pass variance, invStd = 1/sqrt(var + eps), invStd3 = invStd^3; with
// dXhat = dY * gamma: dVar = sum(dXhat * diff * -0.5 * invStd3), dMean = sum(dXhat * -invStd)
// + dVar * -2 * sum(diff) / cols; dX = dXhat * invStd + dVar * 2 * diff / cols + dMean / cols.
// With mean_inv non-null the row's mean and invStd are also stored there (for the parameter
// pass when no xHat is kept).
__global__ void layernorm_backward_input_kernel(float* __restrict__ dx, const float* __restrict__ dy,
                                                const float* __restrict__ in,
                                                const float* __restrict__ gamma,
                                                float* __restrict__ mean_inv, uint32_t rows,
                                                uint32_t cols, float eps) {
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t row = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;
    const float* x = in + (size_t)row * cols;
    const float* g = dy + (size_t)row * cols;
    const float inv_cols = 1.0f / (float)cols;
    float s = 0.0f;
    for (uint32_t c = lane; c < cols; c += kWave) s += x[c];
    const float mean = wave_sum(s) * inv_cols;
    float q = 0.0f;
    for (uint32_t c = lane; c < cols; c += kWave) {
        const float d = x[c] - mean;
        q += d * d;
    }
    const float var = wave_sum(q) * inv_cols;
    const float inv_std = 1.0f / sqrtf(var + eps);
    const float inv_std3 = inv_std * inv_std * inv_std;
    float dvar = 0.0f, dmean = 0.0f, sdiff = 0.0f;
    for (uint32_t c = lane; c < cols; c += kWave) {
        const float diff = x[c] - mean;
        const float dxh = g[c] * gamma[c];
        dvar += dxh * diff * -0.5f * inv_std3;
        dmean += dxh * -inv_std;
        sdiff += diff;
    }
    dvar = wave_sum(dvar);
    dmean = wave_sum(dmean);
    sdiff = wave_sum(sdiff);
    dmean += dvar * -2.0f * sdiff * inv_cols;
    float* o = dx + (size_t)row * cols;
    for (uint32_t c = lane; c < cols; c += kWave) {
        const float diff = x[c] - mean;
        const float dxh = g[c] * gamma[c];
        o[c] = dxh * inv_std + dvar * 2.0f * diff * inv_cols + dmean * inv_cols;
    }
    if (mean_inv && lane == 0) {
        mean_inv[2 * row] = mean;
        mean_inv[2 * row + 1] = inv_std;
    }
}

// ScatterAddRows (MatrixBase_Functions.h:285-327): out[oz][idx[z][r]][:] += src[z][r][:] in
// (z, r) order, oz = 0 when out_batch == 1.  Deterministic: the block of source position i
// works only if i is the first position of its destination row; it then adds that row's
// sources in position order, the reference's order, so the sums are bit-identical to it.
// Ids are float (truncated); one outside [0, out_rows) is skipped (the CPU reference asserts).
__global__ void scatter_add_rows_kernel(float* __restrict__ out, const float* __restrict__ src,
                                        const float* __restrict__ idx, uint32_t width,
                                        uint32_t src_rows, uint32_t out_rows, uint32_t out_batch,
                                        uint32_t n) {
    __shared__ int found;
    __shared__ uint32_t list[kThreads];
    __shared__ uint32_t wave_count[kThreads / kWave];
    const uint32_t i = blockIdx.x;
    auto key = [&](uint32_t j) -> int64_t {
        const float f = idx[j];
        if (!(f >= 0.0f) || !(f < (float)out_rows)) return -1;
        const uint32_t d = (uint32_t)f;
        if (d >= out_rows) return -1;
        const uint32_t oz = out_batch == 1 ? 0u : j / src_rows;
        return (int64_t)oz * out_rows + d;
    };
    const int64_t k = key(i);
    if (k < 0) return;
    if (threadIdx.x == 0) found = 0;
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < i; j += blockDim.x)
        if (key(j) == k) found = 1;
    __syncthreads();
    if (found) return;
    float* dst = out + (size_t)k * width;
    // Running sums live in registers: thread t owns columns t, t + blockDim, ...
    constexpr uint32_t kCols = 8;
    float acc[kCols];
    const uint32_t per = (width + blockDim.x - 1) / blockDim.x;
    for (uint32_t base = 0; base < per; base += kCols) {
#pragma unroll
        for (uint32_t m = 0; m < kCols; ++m) {
            const uint32_t c = threadIdx.x + (base + m) * blockDim.x;
            acc[m] = (base + m < per && c < width) ? dst[c] : 0.0f;
        }
        for (uint32_t j0 = i; j0 < n; j0 += blockDim.x) {
            // Matching positions of this chunk, listed in position order: each wave's matches
            // are ranked by a ballot, after the matches of the waves before it.
            const uint32_t j = j0 + threadIdx.x;
            const bool match = j < n && key(j) == k;
            const uint64_t mask = __ballot(match);
            const uint32_t lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
            __syncthreads();  // the previous chunk's list has been consumed
            if (lane == 0) wave_count[w] = (uint32_t)__popcll(mask);
            __syncthreads();
            uint32_t before = 0, cnt = 0;
            for (uint32_t q = 0; q < blockDim.x / kWave; ++q) {
                if (q < w) before += wave_count[q];
                cnt += wave_count[q];
            }
            if (match) list[before + (uint32_t)__popcll(mask & ((1ull << lane) - 1ull))] = j;
            __syncthreads();
            for (uint32_t a = 0; a < cnt; ++a) {
                const float* s = src + (size_t)list[a] * width;
#pragma unroll
                for (uint32_t m = 0; m < kCols; ++m) {
                    const uint32_t c = threadIdx.x + (base + m) * blockDim.x;
                    if (base + m < per && c < width) acc[m] += s[c];
                }
            }
        }
#pragma unroll
        for (uint32_t m = 0; m < kCols; ++m) {
            const uint32_t c = threadIdx.x + (base + m) * blockDim.x;
            if (base + m < per && c < width) dst[c] = acc[m];
        }
    }
}

// CategoricalCrossEntropyWithLogits::Gradient / ::Loss, index targets (LossLibrary/
// CategoricalCrossEntropyWithLogits.h:117-178, :29-73): rows with target -1 are ignored
// (gradient row 0); valid = number of other rows; per row the stable softmax
// p = exp(z - max) / sum exp(z - max) gives grad = (onehot - p) / valid and
// loss = (max + log(sum)) - z[target].  One block per row (t, z); the valid count is computed
// by every block from the target vector (it is at most a few thousand floats).
__device__ bool cce_target(const float* target, uint32_t steps, uint32_t target_batch, uint32_t row,
                           int32_t* idx_out) {
    const uint32_t z = row / steps, t = row % steps;
    const uint32_t tz = target_batch == 1 ? 0u : z;
    const int32_t idx = (int32_t)target[(size_t)tz * steps + t];
    *idx_out = idx;
    return idx != -1;
}

__global__ void cce_index_kernel(float* __restrict__ grad, float* __restrict__ row_loss,
                                 const float* __restrict__ target, const float* __restrict__ logits,
                                 uint32_t vocab, uint32_t steps, uint32_t batch,
                                 uint32_t target_batch) {
    __shared__ float sh[kThreads / kWave];
    __shared__ uint32_t valid_sh;
    const uint32_t row = blockIdx.x;
    const float* z = logits + (size_t)row * vocab;
    if (grad) {
        // valid count over every (z, t), as the reference counts it before the rows.
        uint32_t v = 0;
        for (uint32_t r = threadIdx.x; r < steps * batch; r += blockDim.x) {
            int32_t id;
            v += cce_target(target, steps, target_batch, r, &id) ? 1u : 0u;
        }
        const float vs = block_sum((float)v, sh);
        if (threadIdx.x == 0) valid_sh = (uint32_t)vs;
        __syncthreads();
    }
    int32_t idx;
    const bool ok = cce_target(target, steps, target_batch, row, &idx);
    if (!ok || idx < 0 || (uint32_t)idx >= vocab) {
        if (grad)
            for (uint32_t c = threadIdx.x; c < vocab; c += blockDim.x) grad[(size_t)row * vocab + c] = 0.0f;
        if (row_loss && threadIdx.x == 0) row_loss[row] = 0.0f;
        return;
    }
    float m = -INFINITY;
    for (uint32_t c = threadIdx.x; c < vocab; c += blockDim.x) m = fmaxf(m, z[c]);
    m = block_max(m, sh);
    float s = 0.0f;
    for (uint32_t c = threadIdx.x; c < vocab; c += blockDim.x) s += expf(z[c] - m);
    s = block_sum(s, sh);
    if (grad) {
        const uint32_t valid = valid_sh;
        const float inv_valid = valid > 0 ? 1.0f / (float)valid : 0.0f;
        for (uint32_t c = threadIdx.x; c < vocab; c += blockDim.x) {
            const float p = expf(z[c] - m) / s;
            const float ti = (uint32_t)idx == c ? 1.0f : 0.0f;
            grad[(size_t)row * vocab + c] = (ti - p) * inv_valid;
        }
    }
    if (row_loss && threadIdx.x == 0) row_loss[row] = (m + logf(s)) - z[idx];
}

// One-hot targets (target dims x == vocab; CategoricalCrossEntropyWithLogits.h:180-208,
// :75-113): grad = t - p without averaging; loss row = lse - z[first i with t_i > 0.5].
__global__ void cce_onehot_kernel(float* __restrict__ grad, float* __restrict__ row_loss,
                                  const float* __restrict__ target, const float* __restrict__ logits,
                                  uint32_t vocab, uint32_t steps, uint32_t target_batch) {
    __shared__ float sh[kThreads / kWave];
    const uint32_t row = blockIdx.x;
    const uint32_t zb = row / steps, t = row % steps;
    const float* tg = target + ((size_t)(target_batch == 1 ? 0u : zb) * steps + t) * vocab;
    const float* z = logits + (size_t)row * vocab;
    float m = -INFINITY;
    for (uint32_t c = threadIdx.x; c < vocab; c += blockDim.x) m = fmaxf(m, z[c]);
    m = block_max(m, sh);
    float s = 0.0f;
    for (uint32_t c = threadIdx.x; c < vocab; c += blockDim.x) s += expf(z[c] - m);
    s = block_sum(s, sh);
    if (grad)
        for (uint32_t c = threadIdx.x; c < vocab; c += blockDim.x)
            grad[(size_t)row * vocab + c] = tg[c] - expf(z[c] - m) / s;
    if (row_loss) {
        // First index with t > 0.5 (the reference breaks at the first one).
        float first = (float)vocab;
        for (uint32_t c = threadIdx.x; c < vocab; c += blockDim.x)
            if (tg[c] > 0.5f) first = fminf(first, (float)c);
        first = -block_max(-first, sh);
        if (threadIdx.x == 0) {
            const uint32_t f = (uint32_t)first;
            row_loss[row] = f < vocab ? (m + logf(s)) - z[f] : 0.0f;
        }
    }
}

// Sum of the per-row losses (the reference accumulates rows sequentially; here a block sums
// them, rounding differently), divided by the valid count for index targets.
__global__ void cce_total_kernel(float* total, const float* row_loss, const float* target,
                                 uint32_t rows, uint32_t steps, uint32_t target_batch, int average) {
    __shared__ float sh[kThreads / kWave];
    float t = 0.0f, valid = 0.0f;
    for (uint32_t r = threadIdx.x; r < rows; r += blockDim.x) {
        if (average) {
            int32_t id;
            if (!cce_target(target, steps, target_batch, r, &id)) continue;
            valid += 1.0f;
        }
        t += row_loss[r];
    }
    t = block_sum(t, sh);
    valid = block_sum(valid, sh);
    if (threadIdx.x == 0) total[0] = average ? (valid > 0.0f ? t / valid : 0.0f) : t;
}

// AdamWUpdate (MatrixBase_Functions.h:1497-1545), element-wise with the reference's operation
// order and no contraction into FMAs, so each element rounds as the x86 reference does:
// m = b1 m + (1-b1) g; v = b2 v + (1-b2) g g; m^ = m / (1-b1^t); v^ = v / (1-b2^t);
// p = (p + lr m^ / (sqrt(v^) + eps)) - lr wd p.  (The loss gradient is the negative
// gradient, CategoricalCrossEntropyWithLogits.h:17-18, hence the '+'.)
__global__ void adamw_kernel(float* __restrict__ param, const float* __restrict__ grad,
                             float* __restrict__ mt, float* __restrict__ vt, size_t n, float lr,
                             float beta1, float beta2, float beta1_pow_t, float beta2_pow_t,
                             float eps, float weight_decay) {
#pragma clang fp contract(off)
    const float inv_b1 = 1.0f - beta1, inv_b2 = 1.0f - beta2;
    const float inv_b1p = 1.0f - beta1_pow_t, inv_b2p = 1.0f - beta2_pow_t;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const float g = grad[i];
        const float m = beta1 * mt[i] + inv_b1 * g;
        const float v = beta2 * vt[i] + inv_b2 * g * g;
        mt[i] = m;
        vt[i] = v;
        const float m_hat = m / inv_b1p;
        const float v_hat = v / inv_b2p;
        const float p = param[i];
        const float update = lr * m_hat / (sqrtf(v_hat) + eps);
        const float decay = lr * weight_decay * p;
        param[i] = p + update - decay;
    }
}

// GeluDerivtiveMat (MatrixBase_Functions.h:1002-1017): 0.5 (1 + erf(x / sqrt 2)) +
// x exp(-0.5 x^2) / sqrt(2 pi), the constants rounded to float as the reference computes them.
__global__ void gelu_derivative_kernel(float* __restrict__ out, const float* __restrict__ in, size_t n) {
    const float sqrt2 = sqrtf(2.0f);
    const float sqrt2pi = sqrtf(2.0f * 3.14159265358979323846f);
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const float x = in[i];
        out[i] = 0.5f * (1.0f + erff(x / sqrt2)) + (x * expf(-0.5f * x * x)) / sqrt2pi;
    }
}

// MergeQKV (MatrixBase_Functions.h:369-431): packed[r][s*C + h*hd + d] = src_s[h][r][d]
// for s = q, k, v.
__global__ void merge_qkv_kernel(float* __restrict__ packed, const float* __restrict__ q,
                                 const float* __restrict__ k, const float* __restrict__ v,
                                 uint32_t head_dim, uint32_t tokens, uint32_t n_head) {
    const uint32_t dC = head_dim * n_head;
    const size_t total = (size_t)tokens * 3 * dC;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const uint32_t r = (uint32_t)(i / (3 * dC));
        const uint32_t col = (uint32_t)(i % (3 * dC));
        const uint32_t s = col / dC, hc = col % dC;
        const uint32_t h = hc / head_dim, d = hc % head_dim;
        const float* src = s == 0 ? q : (s == 1 ? k : v);
        packed[i] = src[((size_t)h * tokens + r) * head_dim + d];
    }
}

// ---- whole-layer attention steps over all heads (CausalSelfAttentionLayer on MatrixHIP) ----

constexpr uint32_t kMaxHeads = 32;
struct HeadPtrs {
    float* p[kMaxHeads];
};

// Per head h and row i (one block each): the reference's ScaleAdd with the causal mask
// (CausalSelfAttentionLayer.h:453; mask 0 on and below the diagonal, -inf above) then Softmax
// (:458; MatrixBase_Functions.h:49-80).  The probabilities go to head h's own matrix (the
// layer's Scratch_AttHead_h, at element offset p_off) and to the contiguous all-heads buffer
// p_all [head][T][T] that the batched P V product reads.
__global__ void attention_softmax_heads_kernel(HeadPtrs heads, size_t p_off, float* __restrict__ p_all,
                                               const float* __restrict__ scores,
                                               const float* __restrict__ scale, uint32_t T) {
    __shared__ float sh[kThreads / kWave];
    const uint32_t i = blockIdx.x, h = blockIdx.y;
    const size_t row = ((size_t)h * T + i) * T;
    const float sc = scale[0];
    float m = -INFINITY;
    for (uint32_t j = threadIdx.x; j <= i && j < T; j += blockDim.x) m = fmaxf(m, scores[row + j] * sc);
    m = block_max(m, sh);
    float s = 0.0f;
    for (uint32_t j = threadIdx.x; j <= i && j < T; j += blockDim.x) s += expf(scores[row + j] * sc - m);
    s = block_sum(s, sh);
    float* ph = heads.p[h] + p_off + (size_t)i * T;
    for (uint32_t j = threadIdx.x; j < T; j += blockDim.x) {
        const float v = j <= i ? expf(scores[row + j] * sc - m) / s : 0.0f;
        ph[j] = v;
        p_all[row + j] = v;
    }
}

// Per head h and row i: SoftmaxBackwards (MatrixBase_Functions.h:83-111), then the layer's
// PerElementMul by the finite causal mask and Scale by 1/sqrt(head_dim)
// (CausalSelfAttentionLayer.h:640-642): ds = ((p (da - sum(da p))) * mask) * scale.
__global__ void attention_softmax_backward_heads_kernel(float* __restrict__ ds_all, HeadPtrs heads,
                                                        const float* __restrict__ datt_all,
                                                        const float* __restrict__ scale, uint32_t T) {
    __shared__ float sh[kThreads / kWave];
    const uint32_t i = blockIdx.x, h = blockIdx.y;
    const size_t row = ((size_t)h * T + i) * T;
    const float* p = heads.p[h] + (size_t)i * T;
    float d = 0.0f;
    for (uint32_t j = threadIdx.x; j < T; j += blockDim.x) d += datt_all[row + j] * p[j];
    const float dot = block_sum(d, sh);
    const float sc = scale[0];
    for (uint32_t j = threadIdx.x; j < T; j += blockDim.x) {
        const float g = p[j] * (datt_all[row + j] - dot);
        ds_all[row + j] = (g * (j <= i ? 1.0f : 0.0f)) * sc;
    }
}

// SumColumns (MatrixBase_Functions.h:1098-1118), the Dense bias gradient: one thread per
// column adds that column's rows in row order, as the reference's loop does, so the sums are
// bit-identical; consecutive threads read consecutive columns of a row.
__global__ void sum_columns_kernel(float* __restrict__ out, const float* __restrict__ in, uint32_t rows,
                                   uint32_t cols) {
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= cols) return;
    float s = 0.0f;
    for (uint32_t r = 0; r < rows; ++r) s += in[(size_t)r * cols + c];
    out[c] = s;
}

// DropoutLayer::UpdateMask (DropoutLayer.h:97-123) for 0 < prob < 1: element i takes draw
// start + i of RandomUtils::random_uniform_buffered (ToolsLibrary/Tools.h:63-69), which reads
// its uniform buffer at (running index) mod count; 0 where the draw is below prob, else 1.
__global__ void dropout_mask_kernel(float* __restrict__ mask, uint64_t n, const float* __restrict__ uniforms,
                                    uint64_t count, uint64_t start, float prob) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        mask[i] = uniforms[(start + i) % count] < prob ? 0.0f : 1.0f;
}

}  // namespace

}  // namespace fmlh

using namespace fmlh;

extern "C" {

int fmlh_sum_columns(float* out, const float* in, uint32_t rows, uint32_t cols) {
    FMLH_REQUIRE(out && in, "fmlh_sum_columns: null pointer");
    FMLH_TRY(ensure_init());
    if (cols == 0) return FMLH_OK;
    hipLaunchKernelGGL(sum_columns_kernel, dim3((cols + kThreads - 1) / kThreads), dim3(kThreads), 0, stream(),
                       out, in, rows, cols);
    FMLH_LAUNCHED("sum_columns_kernel");
    return FMLH_OK;
}

int fmlh_dropout_mask(float* mask, uint64_t n, const float* uniforms, uint64_t count, uint64_t start,
                      float prob) {
    FMLH_REQUIRE(mask && uniforms && count > 0, "fmlh_dropout_mask: null pointer or empty uniform buffer");
    FMLH_TRY(ensure_init());
    if (n == 0) return FMLH_OK;
    hipLaunchKernelGGL(dropout_mask_kernel, dim3(blocks_for(n, kThreads, 8192u)), dim3(kThreads), 0, stream(),
                       mask, n, uniforms, count, start, prob);
    FMLH_LAUNCHED("dropout_mask_kernel");
    return FMLH_OK;
}

int fmlh_softmax_backward(float* out, const float* softmax_out, const float* grad_in, uint32_t rows,
                          uint32_t cols) {
    FMLH_REQUIRE(out && softmax_out && grad_in, "fmlh_softmax_backward: null pointer");
    FMLH_REQUIRE(cols > 0, "fmlh_softmax_backward: cols == 0");
    FMLH_TRY(ensure_init());
    if (rows == 0) return FMLH_OK;
    hipLaunchKernelGGL(softmax_backward_kernel, dim3(rows), dim3(kThreads), 0, stream(), out,
                       softmax_out, grad_in, cols);
    FMLH_LAUNCHED("softmax_backward_kernel");
    return FMLH_OK;
}

int fmlh_layernorm_backward(float* dx, const float* dy, const float* in, const float* gamma,
                            float* dgamma, float* dbeta, const float* xhat, float* ws,
                            uint32_t rows, uint32_t cols, float eps) {
    FMLH_REQUIRE(dx && dy && in && gamma && dgamma, "fmlh_layernorm_backward: null pointer");
    FMLH_REQUIRE(cols > 0, "fmlh_layernorm_backward: cols == 0");
    FMLH_REQUIRE(xhat || ws, "fmlh_layernorm_backward: without xhat a workspace of 2*rows floats is needed");
    FMLH_REQUIRE(dx != dy && dx != in, "fmlh_layernorm_backward: dx may not alias dy or in");
    FMLH_TRY(ensure_init());
    if (rows == 0) {
        FMLH_HIP(hipMemsetAsync(dgamma, 0, cols * sizeof(float), stream()));
        if (dbeta) FMLH_HIP(hipMemsetAsync(dbeta, 0, cols * sizeof(float), stream()));
        return FMLH_OK;
    }
    float* mean_inv = xhat ? nullptr : ws;
    const unsigned waves = 4;
    hipLaunchKernelGGL(layernorm_backward_input_kernel, dim3((rows + waves - 1) / waves),
                       dim3(waves * kWave), 0, stream(), dx, dy, in, gamma, mean_inv, rows, cols, eps);
    FMLH_LAUNCHED("layernorm_backward_input_kernel");
    hipLaunchKernelGGL(layernorm_backward_params_kernel, dim3((cols + kWave - 1) / kWave),
                       dim3(kLnbWaves * kWave), 0, stream(), dgamma, dbeta, dy, xhat, mean_inv, in,
                       rows, cols);
    FMLH_LAUNCHED("layernorm_backward_params_kernel");
    return FMLH_OK;
}

int fmlh_gelu_derivative(float* out, const float* in, size_t n) {
    FMLH_REQUIRE(out && in, "fmlh_gelu_derivative: null pointer");
    FMLH_TRY(ensure_init());
    if (n == 0) return FMLH_OK;
    hipLaunchKernelGGL(gelu_derivative_kernel, dim3(blocks_for(n, kThreads, 8192u)), dim3(kThreads),
                       0, stream(), out, in, n);
    FMLH_LAUNCHED("gelu_derivative_kernel");
    return FMLH_OK;
}

int fmlh_scatter_add_rows(float* out, const float* src, const float* idx, uint32_t width,
                          uint32_t src_rows, uint32_t src_batch, uint32_t out_rows,
                          uint32_t out_batch) {
    FMLH_REQUIRE(out && src && idx, "fmlh_scatter_add_rows: null pointer");
    FMLH_REQUIRE(out_batch == 1 || out_batch == src_batch,
                 "fmlh_scatter_add_rows: out batch %u vs src batch %u", out_batch, src_batch);
    FMLH_TRY(ensure_init());
    const size_t n = (size_t)src_rows * src_batch;
    if (n == 0 || width == 0) return FMLH_OK;
    FMLH_REQUIRE(n <= 0x7fffffffu, "fmlh_scatter_add_rows: too many rows");
    hipLaunchKernelGGL(scatter_add_rows_kernel, dim3((unsigned)n), dim3(kThreads), 0, stream(), out,
                       src, idx, width, src_rows, out_rows, out_batch, (uint32_t)n);
    FMLH_LAUNCHED("scatter_add_rows_kernel");
    return FMLH_OK;
}

int fmlh_cce_logits(float* grad, float* loss, float* ws, const float* target, const float* logits,
                    uint32_t vocab, uint32_t steps, uint32_t batch, uint32_t target_cols,
                    uint32_t target_batch) {
    FMLH_REQUIRE(target && logits, "fmlh_cce_logits: null pointer");
    FMLH_REQUIRE(target_cols == 1 || target_cols == vocab,
                 "fmlh_cce_logits: target width %u is neither 1 nor vocab %u", target_cols, vocab);
    FMLH_REQUIRE(target_batch == 1 || target_batch == batch, "fmlh_cce_logits: target batch %u vs %u",
                 target_batch, batch);
    FMLH_REQUIRE(!loss || ws, "fmlh_cce_logits: the loss needs a workspace of rows + 1 floats");
    FMLH_TRY(ensure_init());
    const uint32_t rows = steps * batch;
    if (rows == 0 || vocab == 0) {
        if (loss) FMLH_HIP(hipMemsetAsync(loss, 0, sizeof(float), stream()));
        return FMLH_OK;
    }
    float* row_loss = loss ? ws : nullptr;
    if (target_cols == 1) {
        hipLaunchKernelGGL(cce_index_kernel, dim3(rows), dim3(kThreads), 0, stream(), grad, row_loss,
                           target, logits, vocab, steps, batch, target_batch);
        FMLH_LAUNCHED("cce_index_kernel");
    } else {
        hipLaunchKernelGGL(cce_onehot_kernel, dim3(rows), dim3(kThreads), 0, stream(), grad,
                           row_loss, target, logits, vocab, steps, target_batch);
        FMLH_LAUNCHED("cce_onehot_kernel");
    }
    if (loss) {
        hipLaunchKernelGGL(cce_total_kernel, dim3(1), dim3(kThreads), 0, stream(), loss, row_loss,
                           target, rows, steps, target_batch, target_cols == 1 ? 1 : 0);
        FMLH_LAUNCHED("cce_total_kernel");
    }
    return FMLH_OK;
}

int fmlh_adamw_update(float* param, const float* grad, float* mt, float* vt, size_t n, float lr,
                      float beta1, float beta2, float beta1_pow_t, float beta2_pow_t, float eps,
                      float weight_decay) {
    FMLH_REQUIRE(param && grad && mt && vt, "fmlh_adamw_update: null pointer");
    FMLH_TRY(ensure_init());
    if (n == 0) return FMLH_OK;
    hipLaunchKernelGGL(adamw_kernel, dim3(blocks_for(n, kThreads, 8192u)), dim3(kThreads), 0,
                       stream(), param, grad, mt, vt, n, lr, beta1, beta2, beta1_pow_t, beta2_pow_t,
                       eps, weight_decay);
    FMLH_LAUNCHED("adamw_kernel");
    return FMLH_OK;
}

int fmlh_merge_qkv(float* packed, const float* q, const float* k, const float* v, uint32_t head_dim,
                   uint32_t tokens, uint32_t n_head) {
    FMLH_REQUIRE(packed && q && k && v, "fmlh_merge_qkv: null pointer");
    FMLH_TRY(ensure_init());
    const size_t total = (size_t)tokens * 3 * head_dim * n_head;
    if (total == 0) return FMLH_OK;
    hipLaunchKernelGGL(merge_qkv_kernel, dim3(blocks_for(total, kThreads, 8192u)), dim3(kThreads), 0,
                       stream(), packed, q, k, v, head_dim, tokens, n_head);
    FMLH_LAUNCHED("merge_qkv_kernel");
    return FMLH_OK;
}

int fmlh_attention_softmax_heads(float* const* p_heads, size_t p_offset, float* p_all, const float* scores,
                                 const float* scale, uint32_t n_head, uint32_t T) {
    FMLH_REQUIRE(p_heads && p_all && scores && scale, "fmlh_attention_softmax_heads: null pointer");
    FMLH_REQUIRE(n_head > 0 && n_head <= kMaxHeads, "fmlh_attention_softmax_heads: %u heads (1..%u)", n_head,
                 kMaxHeads);
    FMLH_TRY(ensure_init());
    if (T == 0) return FMLH_OK;
    HeadPtrs hp{};
    for (uint32_t h = 0; h < n_head; ++h) {
        FMLH_REQUIRE(p_heads[h], "fmlh_attention_softmax_heads: null head pointer %u", h);
        hp.p[h] = p_heads[h];
    }
    hipLaunchKernelGGL(attention_softmax_heads_kernel, dim3(T, n_head), dim3(kThreads), 0, stream(), hp, p_offset,
                       p_all, scores, scale, T);
    FMLH_LAUNCHED("attention_softmax_heads_kernel");
    return FMLH_OK;
}

int fmlh_attention_softmax_backward_heads(float* ds_all, float* const* p_heads, const float* datt_all,
                                          const float* scale, uint32_t n_head, uint32_t T) {
    FMLH_REQUIRE(ds_all && p_heads && datt_all && scale, "fmlh_attention_softmax_backward_heads: null pointer");
    FMLH_REQUIRE(n_head > 0 && n_head <= kMaxHeads, "fmlh_attention_softmax_backward_heads: %u heads (1..%u)",
                 n_head, kMaxHeads);
    FMLH_TRY(ensure_init());
    if (T == 0) return FMLH_OK;
    HeadPtrs hp{};
    for (uint32_t h = 0; h < n_head; ++h) {
        FMLH_REQUIRE(p_heads[h], "fmlh_attention_softmax_backward_heads: null head pointer %u", h);
        hp.p[h] = p_heads[h];
    }
    hipLaunchKernelGGL(attention_softmax_backward_heads_kernel, dim3(T, n_head), dim3(kThreads), 0, stream(), ds_all,
                       hp, datt_all, scale, T);
    FMLH_LAUNCHED("attention_softmax_backward_heads_kernel");
    return FMLH_OK;
}

}  // extern "C"
