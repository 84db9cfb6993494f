// Internal helpers shared by the HIP translation units of libfreeml_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/freeml_hip.h"

namespace fmlh {

// Records the message for fmlh_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Lazily initialises device 0 if fmlh_init was not called; returns FMLH_OK or an error.
int ensure_init();
hipStream_t stream();
int cu_count();
// Failure injection for tests of the error paths.  FMLH_FAULT=alloc:N or launch:N, read at
// each fmlh_init (and at lazy initialisation): the N-th device allocation (device_malloc) or
// kernel launch check (FMLH_LAUNCHED, the persistent launch) after it fails as the runtime
// reports such failures, with a message naming FMLH_FAULT.  One shot; unset: never.
enum FaultKind { kFaultAlloc = 0, kFaultLaunch = 1 };
bool inject_fault(FaultKind kind);
// hipMalloc behind the failure hook; every library allocation goes through it.
int device_malloc(void** p, size_t bytes);
// fmlh_gemm_ex_noalloc's split-K partials: a fixed device array of kNoAllocScratchFloats per
// device (gemm.hip).  setup_noalloc_scratch resolves its address on `device` (current) at
// fmlh_init; noalloc_scratch returns it, nullptr before initialisation.
constexpr size_t kNoAllocScratchFloats = size_t(4) << 20;  // 16 MiB
int setup_noalloc_scratch(int device);
float* noalloc_scratch();
// Floats of split-K partials gemm() needs for this product (0 when it splits nothing).
struct GemmArgs;
size_t gemm_workspace_elems(const GemmArgs& g);
// Teardown steps of fmlh_shutdown, owned by the translation units that allocate: every live
// token-loop engine (nanollm.hip) and the process-wide split-K workspace (gemm.hip).
void destroy_all_engines();
void release_global_workspace();

inline int hip_fail(hipError_t e, const char* what, const char* file, int line) {
    return set_error(FMLH_E_HIP, "%s failed at %s:%d: %s", what, file, line, hipGetErrorString(e));
}

}  // namespace fmlh

#define FMLH_HIP(expr)                                                      \
    do {                                                                    \
        hipError_t fmlh_e_ = (expr);                                        \
        if (fmlh_e_ != hipSuccess) return fmlh::hip_fail(fmlh_e_, #expr, __FILE__, __LINE__); \
    } while (0)

// After a kernel launch: reports launch-configuration errors.
#define FMLH_LAUNCHED(name)                                                  \
    do {                                                                     \
        hipError_t fmlh_e_ = hipGetLastError();                              \
        if (fmlh_e_ != hipSuccess) return fmlh::hip_fail(fmlh_e_, name, __FILE__, __LINE__); \
        if (fmlh::inject_fault(fmlh::kFaultLaunch))                          \
            return fmlh::set_error(FMLH_E_HIP, "%s: launch failed (injected by FMLH_FAULT)", name); \
    } while (0)

#define FMLH_REQUIRE(cond, ...)                                   \
    do {                                                          \
        if (!(cond)) return fmlh::set_error(FMLH_E_INVALID, __VA_ARGS__); \
    } while (0)

#define FMLH_TRY(expr)                 \
    do {                               \
        int fmlh_rc_ = (expr);         \
        if (fmlh_rc_ != FMLH_OK) return fmlh_rc_; \
    } while (0)

namespace fmlh {

constexpr int kWave = 64;

// Wave-wide reductions with DPP lane shifts (no LDS round trips): an inclusive scan inside
// each 16-lane row (row_shr 1, 2, 4, 8), then row_bcast:15 / row_bcast:31 carry the row
// totals upward, so lane 63 holds the wave total, which readlane broadcasts.  Out-of-row
// sources take the identity (old operand), as bound_ctrl is off.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_move(float old, float x) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(x), kCtrl, kRowMask, 0xf, false));
}

template <class Op>
__device__ __forceinline__ float wave_reduce(float v, float identity, Op op) {
    v = op(v, dpp_move<0x111, 0xf>(identity, v));  // row_shr:1
    v = op(v, dpp_move<0x112, 0xf>(identity, v));  // row_shr:2
    v = op(v, dpp_move<0x114, 0xf>(identity, v));  // row_shr:4
    v = op(v, dpp_move<0x118, 0xf>(identity, v));  // row_shr:8
    v = op(v, dpp_move<0x142, 0xa>(identity, v));  // row_bcast:15 -> rows 1, 3
    v = op(v, dpp_move<0x143, 0xc>(identity, v));  // row_bcast:31 -> rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_sum(float v) {
    return wave_reduce(v, 0.0f, [](float a, float b) { return a + b; });
}

__device__ __forceinline__ float wave_max(float v) {
    return wave_reduce(v, -INFINITY, [](float a, float b) { return fmaxf(a, b); });
}

inline unsigned blocks_for(size_t n, unsigned threads, unsigned cap = 65535u * 8u) {
    size_t b = (n + threads - 1) / threads;
    if (b == 0) b = 1;
    return b > cap ? cap : static_cast<unsigned>(b);
}

// ---- GEMM entry points shared between the op layer and the token loop ------------------

enum Epilogue : int {
    kEpiNone = 0,   // C = acc
    kEpiGelu = 1,   // C = gelu(acc)  (GeluMat applied to the Dense output, Dense.h:218-222)
    kEpiResid = 2,  // C = R + acc    (the block's residual Add, TransformerBlock.h:382/:400)
    // Internal (not accepted by fmlh_gemm_ex): the QKV product of a prefill, N = 3 C.  Columns
    // [0, C) go to C (the queries); columns [C, 3C) go straight to the K / V caches (GemmArgs
    // kv), row m being position m % rows_per_seq of sequence m / rows_per_seq.
    kEpiKV = 3,
};

// Destination of kEpiKV's key / value columns: caches [sequence][head][T][head_dim].
struct KvDest {
    float* kc = nullptr;
    float* vc = nullptr;
    int C = 0, H = 0, hd = 0, T = 0, rows_per_seq = 1;
};

// C (M x N, row stride ldc) = A (M x K, row stride lda) * op(B) with op(B) = B (K x N, ldb)
// when b_trans == 0, or B^T for B stored N x K (ldb) when b_trans == 1; epilogue as above
// (R has row stride ldr and may alias C).
struct GemmArgs {
    const float* A = nullptr;
    int lda = 0;
    const float* B = nullptr;
    int ldb = 0;
    int b_trans = 0;
    float* C = nullptr;
    int ldc = 0;
    int M = 0, N = 0, K = 0;
    int epi = kEpiNone;
    const float* R = nullptr;
    int ldr = 0;
    KvDest kv;  // kEpiKV only
    // ln_g != nullptr: A holds rows before a LayerNorm (LayerNormOp, eps ln_eps, gamma ln_g,
    // optional beta ln_b) and the product takes the normalised rows.  Skinny NT products only
    // (gemm_takes_ln); no normalised copy is written.
    const float* ln_g = nullptr;
    const float* ln_b = nullptr;
    float ln_eps = 1e-5f;
    hipStream_t s = nullptr;
};

// Kernel choice for a shape: skinny kernels for M <= 8 (decode), MFMA tiles otherwise, with
// the split-K factor and the workspace (floats) the split partial sums need.
struct GemmPlan {
    enum Kind { kSkinnyNN, kSkinnyNT, kMfma, kMfmaNT } kind = kMfma;
    int bm = 64, bn = 64;
    int splits = 1, k_per_split = 0;
    size_t ws_elems = 0;
};
GemmPlan plan_gemm(int M, int N, int K, int b_trans);

// Runs the product.  ws/ws_elems: caller workspace for split partials (must hold
// plan_gemm(...).ws_elems floats); nullptr uses a process-wide buffer grown on demand, which
// callers that capture HIP graphs must avoid.
int gemm(const GemmArgs& g, float* ws, size_t ws_elems);
// Whether the product runs on gemm_nt_kernel (the kernel that takes kEpiKV): B stored N x K,
// 16-byte aligned K-contiguous rows, K % 16 == 0 and enough 64 x 64 tiles.
bool gemm_runs_nt(const GemmArgs& g);
// Whether the product can take its A rows through a LayerNorm (GemmArgs ln_*): the skinny NT
// kernels (M <= 8, B stored N x K) with K <= 1024.
bool gemm_takes_ln(int M, int N, int K, int b_trans);
// When the plan splits K (batched-decode shapes), launches only the split products: ws holds
// *splits partial M x N sums, [split][row][col], for a caller-side reduction (fused with what
// follows the product).  Otherwise launches nothing and sets *splits = 0.
int gemm_split_partials(const GemmArgs& g, float* ws, size_t ws_elems, int* splits);
// The K-split partial sums of an NT product (B stored N x K) on gemm_nt_kernel's 64 x 64 tiles,
// whatever the plan: split z takes K range [z K / splits, (z + 1) K / splits) and writes
// ws[z][M][N], for a caller-side reduction.  K must be a multiple of 16 splits.
int gemm_nt_partials(const GemmArgs& g, int splits, float* ws, size_t ws_elems);

// General strided product (any transpose mode, element strides, batched planes) used by the
// MatMul_Strided / Mul overloads when the fast layouts do not apply.
int gemm_strided(int mode, float* out, const float* L, const float* R, uint32_t M, uint32_t N,
                 uint32_t K, uint32_t l_rs, uint32_t l_cs, uint32_t r_rs, uint32_t r_cs,
                 uint32_t o_rs, uint32_t o_cs, uint32_t batch, size_t l_plane, size_t r_plane,
                 size_t o_plane, hipStream_t s);

// Row LayerNorm (one wave per row).
int layernorm_rows(float* out, const float* in, const float* gamma, const float* beta,
                   float* xhat, uint32_t rows, uint32_t cols, float eps, hipStream_t s);

int row_argmax(int32_t* out_idx, const float* in, uint32_t rows, uint32_t cols, size_t out_stride,
               hipStream_t s);


// ---- direct-to-LDS tile copies (device code) ----------------------------------------------
// 16 bytes per lane from src_lane into LDS at lds_wave_base + 16 * lane (global_load_lds).
// Issued as inline asm: with the builtin, the compiler's wait insertion treats every later LDS
// read as possibly dependent on the copy and waits for all LDS reads at once (lgkmcnt(0)),
// which serialises the operand reads with the MFMAs.  The caller orders the copies itself
// (copies_barrier).  An LDS DMA that reads M0 must not directly follow the SALU write of M0
// (one wait state: the compiler inserts it for its own code, not inside asm), or it may take
// the previous M0 and write its 1 KB to the previous copy's place.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void copy16_to_lds(float* lds_wave_base, const float* src_lane) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)lds_wave_base);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :: "s"(base), "v"(src_lane) : "memory", "m0");
}
#pragma clang diagnostic pop

// Work-group barrier after this wave's copies have drained to at most N in flight and its
// LDS reads have completed.  One asm statement: the compiler does not see the copies (they
// are asm too), so it must not be left to place or merge this wait; the memory clobber keeps
// LDS accesses from moving across the barrier.
template <int N>
__device__ __forceinline__ void copies_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" :: "n"(N) : "memory");
}

}  // namespace fmlh
