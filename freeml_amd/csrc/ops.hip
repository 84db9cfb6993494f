// Element-wise and row-wise matrix ops of the C ABI (the MatrixHIP<float> overload set).
// Each kernel states the reference routine whose result it reproduces.
#include "fmlh_internal.h"

namespace fmlh {

namespace {

constexpr unsigned kThreads = 256;

// ---- element-wise -------------------------------------------------------------------------

template <class F>
__global__ void map_kernel(size_t n, F f) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        f(i);
}

template <class F>
int launch_map(size_t n, F f, const char* name) {
    FMLH_TRY(ensure_init());
    if (n == 0) return FMLH_OK;
    hipLaunchKernelGGL(map_kernel<F>, dim3(blocks_for(n, kThreads, 8192u)), dim3(kThreads), 0,
                       stream(), n, f);
    FMLH_LAUNCHED(name);
    return FMLH_OK;
}

// GeluMat (MatrixBase_Functions.h:988-1000): x / sqrt(2) is a division by sqrtf(2.0f), as the
// reference evaluates it, then erf of that.
__device__ __forceinline__ float gelu_ref(float x) {
    return 0.5f * x * (1.0f + erff(x / 1.41421354f));
}

// ---- row ops -----------------------------------------------------------------------------

// LayerNormOp (MatrixBase_Functions.h:481-549), one wave per row: mean = sum * (1/cols),
// var = sum((x-mean)^2) * (1/cols), invStd = 1 / sqrt(var + eps), out = (x-mean)*invStd*g + b.
// Rows of up to kLnRegCols columns are read once into registers (all loads in flight
// together); longer rows take the three passes over memory.  Same sums, same order.
constexpr uint32_t kLnRegNE = 16, kLnRegCols = kLnRegNE * kWave;

__global__ void layernorm_kernel(float* __restrict__ out, const float* __restrict__ in,
                                 const float* __restrict__ gamma, const float* __restrict__ beta,
                                 float* __restrict__ xhat, uint32_t rows, uint32_t cols,
                                 float eps) {
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t row = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;
    const float* x = in + (size_t)row * cols;
    const float inv_cols = 1.0f / (float)cols;
    if (cols <= kLnRegCols) {
        // gamma / beta are loaded with the row, so the normalisation waits for one round trip.
        float v[kLnRegNE], gv[kLnRegNE], bv[kLnRegNE];
#pragma unroll
        for (uint32_t m = 0; m < kLnRegNE; ++m) {
            const uint32_t c = lane + kWave * m;
            v[m] = c < cols ? x[c] : 0.0f;
            gv[m] = c < cols ? gamma[c] : 0.0f;
            bv[m] = (c < cols && beta) ? beta[c] : 0.0f;
        }
        float s = 0.0f;
#pragma unroll
        for (uint32_t m = 0; m < kLnRegNE; ++m)
            if (lane + kWave * m < cols) s += v[m];
        const float mean = wave_sum(s) * inv_cols;
        float q = 0.0f;
#pragma unroll
        for (uint32_t m = 0; m < kLnRegNE; ++m)
            if (lane + kWave * m < cols) {
                const float d = v[m] - mean;
                q += d * d;
            }
        const float inv_std = 1.0f / sqrtf(wave_sum(q) * inv_cols + eps);
        float* y = out + (size_t)row * cols;
#pragma unroll
        for (uint32_t m = 0; m < kLnRegNE; ++m) {
            const uint32_t c = lane + kWave * m;
            if (c < cols) {
                const float nrm = (v[m] - mean) * inv_std;
                if (xhat) xhat[(size_t)row * cols + c] = nrm;
                y[c] = nrm * gv[m] + bv[m];
            }
        }
        return;
    }
    float s = 0.0f;
    for (uint32_t c = lane; c < cols; c += kWave) s += x[c];
    const float mean = wave_sum(s) * inv_cols;
    float v = 0.0f;
    for (uint32_t c = lane; c < cols; c += kWave) {
        const float d = x[c] - mean;
        v += d * d;
    }
    const float var = wave_sum(v) * inv_cols;
    const float inv_std = 1.0f / sqrtf(var + eps);
    float* y = out + (size_t)row * cols;
    for (uint32_t c = lane; c < cols; c += kWave) {
        const float nrm = (x[c] - mean) * inv_std;
        if (xhat) xhat[(size_t)row * cols + c] = nrm;
        y[c] = nrm * gamma[c] + (beta ? beta[c] : 0.0f);
    }
}

__device__ __forceinline__ float block_reduce_max(float v, float* sh) {
    v = wave_max(v);
    const unsigned w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    __syncthreads();
    if (lane == 0) sh[w] = v;
    __syncthreads();
    float r = sh[0];
    for (unsigned i = 1; i < blockDim.x / kWave; ++i) r = fmaxf(r, sh[i]);
    return r;
}

__device__ __forceinline__ float block_reduce_sum(float v, float* sh) {
    v = wave_sum(v);
    const unsigned w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    __syncthreads();
    if (lane == 0) sh[w] = v;
    __syncthreads();
    float r = 0.0f;
    for (unsigned i = 0; i < blockDim.x / kWave; ++i) r += sh[i];
    return r;
}

// Softmax (MatrixBase_Functions.h:49-80): row max, exp(x - max), sum, then divide.
__global__ void softmax_kernel(float* out, const float* in, uint32_t cols) {
    __shared__ float sh[kThreads / kWave];
    const float* x = in + (size_t)blockIdx.x * cols;
    float* y = out + (size_t)blockIdx.x * cols;
    float m = -INFINITY;
    for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) m = fmaxf(m, x[c]);
    m = block_reduce_max(m, sh);
    float s = 0.0f;
    for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) {
        const float e = expf(x[c] - m);
        y[c] = e;
        s += e;
    }
    s = block_reduce_sum(s, sh);
    for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) y[c] = y[c] / s;
}

// First maximum with strict '>' (NanoLLM.cpp:189-205): ties go to the lowest index.
__global__ void argmax_kernel(int32_t* out_idx, const float* in, uint32_t cols, size_t out_stride) {
    __shared__ float sv[kThreads];
    __shared__ int si[kThreads];
    const float* x = in + (size_t)blockIdx.x * cols;
    float bv = -INFINITY;
    int bi = -1;
    for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) {
        const float v = x[c];
        if (bi < 0 || v > bv) { bv = v; bi = (int)c; }
    }
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (unsigned off = blockDim.x / 2; off > 0; off >>= 1) {
        if (threadIdx.x < off) {
            const float ov = sv[threadIdx.x + off];
            const int oi = si[threadIdx.x + off];
            const float mv = sv[threadIdx.x];
            const int mi = si[threadIdx.x];
            if (oi >= 0 && (mi < 0 || ov > mv || (ov == mv && oi < mi))) {
                sv[threadIdx.x] = ov;
                si[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out_idx[(size_t)blockIdx.x * out_stride] = si[0] < 0 ? 0 : si[0];
}

// GatherRows (MatrixBase_Functions.h:202-242).  An id outside [0, src_rows) yields a zero row,
// as the DX11 backend's gather_rows shader does (the CPU reference asserts instead).
__global__ void gather_rows_kernel(float* out, const float* src, const float* idx, uint32_t width,
                                   uint32_t out_rows, uint32_t src_rows, uint32_t src_batch,
                                   size_t total) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t row = i / width;  // z * out_rows + r
        const uint32_t col = (uint32_t)(i % width);
        const size_t z = row / out_rows;
        const float f = idx[row];
        const uint32_t s = (f >= 0.0f) ? (uint32_t)f : 0xffffffffu;
        const size_t zs = src_batch == 1 ? 0 : z;
        out[i] = (s < src_rows) ? src[(zs * src_rows + s) * width + col] : 0.0f;
    }
}

}  // namespace

int layernorm_rows(float* out, const float* in, const float* gamma, const float* beta,
                   float* xhat, uint32_t rows, uint32_t cols, float eps, hipStream_t s) {
    if (rows == 0) return FMLH_OK;
    const unsigned waves = 4;
    hipLaunchKernelGGL(layernorm_kernel, dim3((rows + waves - 1) / waves), dim3(waves * kWave), 0,
                       s, out, in, gamma, beta, xhat, rows, cols, eps);
    FMLH_LAUNCHED("layernorm_kernel");
    return FMLH_OK;
}

int row_argmax(int32_t* out_idx, const float* in, uint32_t rows, uint32_t cols,
               size_t out_stride, hipStream_t s) {
    if (rows == 0) return FMLH_OK;
    hipLaunchKernelGGL(argmax_kernel, dim3(rows), dim3(kThreads), 0, s, out_idx, in, cols,
                       out_stride);
    FMLH_LAUNCHED("argmax_kernel");
    return FMLH_OK;
}

}  // namespace fmlh

using namespace fmlh;

extern "C" {

int fmlh_softmax(float* out, const float* in, uint32_t rows, uint32_t cols) {
    FMLH_REQUIRE(out && in, "fmlh_softmax: null pointer");
    FMLH_REQUIRE(cols > 0, "fmlh_softmax: cols == 0");
    FMLH_TRY(ensure_init());
    if (rows == 0) return FMLH_OK;
    hipLaunchKernelGGL(softmax_kernel, dim3(rows), dim3(kThreads), 0, stream(), out, in, cols);
    FMLH_LAUNCHED("softmax_kernel");
    return FMLH_OK;
}

int fmlh_layernorm(float* out, const float* in, const float* gamma, const float* beta,
                   float* xhat, uint32_t rows, uint32_t cols, float eps) {
    FMLH_REQUIRE(out && in && gamma, "fmlh_layernorm: null pointer");
    FMLH_REQUIRE(cols > 0, "fmlh_layernorm: cols == 0");
    FMLH_TRY(ensure_init());
    return layernorm_rows(out, in, gamma, beta, xhat, rows, cols, eps, stream());
}

int fmlh_gelu(float* out, const float* in, size_t n) {
    FMLH_REQUIRE(out && in, "fmlh_gelu: null pointer");
    return launch_map(n, [=] __device__(size_t i) { out[i] = gelu_ref(in[i]); }, "gelu");
}

int fmlh_add(float* out, const float* a, const float* b, size_t n) {
    FMLH_REQUIRE(out && a && b, "fmlh_add: null pointer");
    return launch_map(n, [=] __device__(size_t i) { out[i] = a[i] + b[i]; }, "add");
}

int fmlh_copy(float* out, const float* in, size_t n) {
    FMLH_REQUIRE(out && in, "fmlh_copy: null pointer");
    if (out == in || n == 0) return FMLH_OK;
    FMLH_TRY(ensure_init());
    FMLH_HIP(hipMemcpyAsync(out, in, n * sizeof(float), hipMemcpyDeviceToDevice, stream()));
    return FMLH_OK;
}

int fmlh_gather_rows(float* out, const float* src, const float* idx, uint32_t width,
                     uint32_t out_rows, uint32_t out_batch, uint32_t src_rows,
                     uint32_t src_batch) {
    FMLH_REQUIRE(out && src && idx, "fmlh_gather_rows: null pointer");
    FMLH_REQUIRE(src_batch == 1 || src_batch == out_batch,
                 "fmlh_gather_rows: src batch %u vs out batch %u", src_batch, out_batch);
    FMLH_TRY(ensure_init());
    const size_t total = (size_t)width * out_rows * out_batch;
    if (total == 0) return FMLH_OK;
    hipLaunchKernelGGL(gather_rows_kernel, dim3(blocks_for(total, kThreads, 8192u)), dim3(kThreads),
                       0, stream(), out, src, idx, width, out_rows, src_rows, src_batch, total);
    FMLH_LAUNCHED("gather_rows_kernel");
    return FMLH_OK;
}

int fmlh_split_qkv(float* q, float* k, float* v, const float* packed, uint32_t rows,
                   uint32_t dC) {
    FMLH_REQUIRE(q && k && v && packed, "fmlh_split_qkv: null pointer");
    const size_t n = (size_t)rows * dC;
    return launch_map(n, [=] __device__(size_t i) {
        const size_t r = i / dC, c = i % dC;
        const float* p = packed + r * 3 * dC;
        q[i] = p[c];
        k[i] = p[dC + c];
        v[i] = p[2 * dC + c];
    }, "split_qkv");
}

int fmlh_scale_add(float* out, const float* in, const float* scale, const float* add, size_t n) {
    FMLH_REQUIRE(out && in && scale && add, "fmlh_scale_add: null pointer");
    return launch_map(n, [=] __device__(size_t i) { out[i] = in[i] * scale[0] + add[i]; },
                      "scale_add");
}

int fmlh_broadcast_add(float* out, const float* L, const float* R, size_t n, uint32_t dims_x) {
    FMLH_REQUIRE(out && L && R && dims_x, "fmlh_broadcast_add: bad argument");
    return launch_map(n, [=] __device__(size_t i) { out[i] = L[i] + R[i % dims_x]; },
                      "broadcast_add");
}

int fmlh_fill(float* out, float value, size_t n) {
    FMLH_REQUIRE(out, "fmlh_fill: null pointer");
    return launch_map(n, [=] __device__(size_t i) { out[i] = value; }, "fill");
}

int fmlh_fill_from(float* out, const float* value, size_t n) {
    FMLH_REQUIRE(out && value, "fmlh_fill_from: null pointer");
    return launch_map(n, [=] __device__(size_t i) { out[i] = value[0]; }, "fill_from");
}

int fmlh_per_element_mul(float* out, const float* a, const float* b, size_t n) {
    FMLH_REQUIRE(out && a && b, "fmlh_per_element_mul: null pointer");
    return launch_map(n, [=] __device__(size_t i) { out[i] = a[i] * b[i]; }, "per_element_mul");
}

int fmlh_scale(float* out, const float* in, const float* value, size_t n) {
    FMLH_REQUIRE(out && in && value, "fmlh_scale: null pointer");
    return launch_map(n, [=] __device__(size_t i) { out[i] = in[i] * value[0]; }, "scale");
}

int fmlh_scale_scalar(float* out, const float* in, float value, size_t n) {
    FMLH_REQUIRE(out && in, "fmlh_scale_scalar: null pointer");
    return launch_map(n, [=] __device__(size_t i) { out[i] = in[i] * value; }, "scale_scalar");
}

int fmlh_row_argmax(int32_t* out_idx, const float* in, uint32_t rows, uint32_t cols) {
    FMLH_REQUIRE(out_idx && in && cols, "fmlh_row_argmax: bad argument");
    FMLH_TRY(ensure_init());
    return row_argmax(out_idx, in, rows, cols, 1, stream());
}

}  // extern "C"
