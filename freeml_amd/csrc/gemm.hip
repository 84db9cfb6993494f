// GEMM kernels behind Mul / MatMul_Strided and the token loop's projections.
//
//  * gemm_nt_kernel: fp32 MFMA (v_mfma_f32_32x32x2f32) tiles for B stored N x K (the token
//    loop's weights), operands copied straight into a three-stage LDS ring; used when the
//    product has at least half a device's worth of 64 x 64 tiles (prefill).
//  * gemm_mfma_kernel: the same MFMA tiling with register-staged, double-buffered LDS, for
//    either B layout and M > 8 (batched decode, small products).  Optional split-K writes
//    partial sums that splitk_reduce_kernel adds in a fixed order (deterministic) before the
//    epilogue.
//  * skinny kernels for M <= 8 (single-sequence decode): HBM-bound weight streaming, every
//    weight read once, all M rows accumulated per weight load.
//  * gemm_strided_kernel: any transpose mode and element strides (MatMul_Strided views).
//
// All products accumulate in fp32.  The reference (MatrixBase_Mul.h:521-545) sums each output
// sequentially over k; these kernels sum in other orders, so results differ from it by fp32
// rounding only (compared with a tolerance in the parity tests).
#include "fmlh_internal.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

namespace fmlh {

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float gelu_ref(float x) {
    return 0.5f * x * (1.0f + erff(x / 1.41421354f));
}

template <int EPI>
__device__ __forceinline__ float epilogue(float acc, const float* R, size_t ridx) {
    if constexpr (EPI == kEpiGelu) return gelu_ref(acc);
    else if constexpr (EPI == kEpiResid) return R[ridx] + acc;
    else return acc;
}

// ---------------------------------------------------------------------------------------
// MFMA tile kernel.
//
// v_mfma_f32_32x32x2f32 operand layout (one 64-lane wave, h = lane / 32, c = lane % 32):
//   A (32 x 2):  lane supplies A[c][h]          B (2 x 32): lane supplies B[h][c]
//   D (32 x 32): lane holds D[8*(r/4) + 4*h + r%4][c] in accumulator register r.
// Within a 16-wide K block the k index of MFMA step s for half h is 8*h + s, so each lane
// reads 8 consecutive k values of its A row / B column from LDS (two 16-byte reads).
// ---------------------------------------------------------------------------------------
constexpr int KB = 16;       // K block
constexpr int LDS_STRIDE = KB + 4;  // floats per LDS row (padding spreads banks)

template <int BM, int BN, bool BT, int EPI, bool SPLIT>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(
    const float* __restrict__ A, int lda, const float* __restrict__ B, int ldb,
    float* __restrict__ C, int ldc, int M, int N, int K, const float* R, int ldr,
    float* __restrict__ partial, int k_per_split) {
    static_assert(BM % 64 == 0 && BN % 64 == 0, "tile must be a multiple of 64");
    constexpr int WM = BM / 2, WN = BN / 2;       // wave tile (2 x 2 waves)
    constexpr int MB = WM / 32, NB = WN / 32;     // 32x32 blocks per wave
    constexpr int A_F4 = BM * KB / 4 / 256;       // float4 loads per thread per K block
    constexpr int B_F4 = BN * KB / 4 / 256;

    __shared__ float As[2][BM][LDS_STRIDE];
    __shared__ float Bs[2][BN][LDS_STRIDE];

    const int tid = threadIdx.x;
    const int lane = tid % 64, wave = tid / 64;
    const int wm = wave / 2, wn = wave % 2;
    const int h = lane / 32, c = lane % 32;
    const int row0 = blockIdx.y * BM, col0 = blockIdx.x * BN;
    const int kbeg = SPLIT ? blockIdx.z * k_per_split : 0;
    const int kend = SPLIT ? min(K, kbeg + k_per_split) : K;

    floatx16 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    floatx4 ra[A_F4], rb[B_F4];

    auto load_global = [&](int k0) {
#pragma unroll
        for (int t = 0; t < A_F4; ++t) {
            const int idx = tid + t * 256;          // BM rows x 4 float4
            const int r = idx / 4, q = idx % 4;
            const int gr = row0 + r;
            ra[t] = (gr < M) ? *reinterpret_cast<const floatx4*>(A + (size_t)gr * lda + k0 + 4 * q)
                             : floatx4{0.f, 0.f, 0.f, 0.f};
        }
        if constexpr (BT) {  // B stored N x K: rows of the tile are output columns
#pragma unroll
            for (int t = 0; t < B_F4; ++t) {
                const int idx = tid + t * 256;
                const int r = idx / 4, q = idx % 4;
                const int gc = col0 + r;
                rb[t] = (gc < N) ? *reinterpret_cast<const floatx4*>(B + (size_t)gc * ldb + k0 + 4 * q)
                                 : floatx4{0.f, 0.f, 0.f, 0.f};
            }
        } else {  // B stored K x N: the tile is KB rows of BN contiguous floats
#pragma unroll
            for (int t = 0; t < B_F4; ++t) {
                const int idx = tid + t * 256;
                const int kr = idx / (BN / 4), q = idx % (BN / 4);
                const int gc = col0 + 4 * q;
                const float* src = B + (size_t)(k0 + kr) * ldb + gc;
                if (gc + 3 < N) {
                    rb[t] = *reinterpret_cast<const floatx4*>(src);
                } else {
                    floatx4 v = {0.f, 0.f, 0.f, 0.f};
                    for (int e = 0; e < 4; ++e)
                        if (gc + e < N) v[e] = src[e];
                    rb[t] = v;
                }
            }
        }
    };

    auto store_lds = [&](int buf) {
#pragma unroll
        for (int t = 0; t < A_F4; ++t) {
            const int idx = tid + t * 256;
            const int r = idx / 4, q = idx % 4;
            *reinterpret_cast<floatx4*>(&As[buf][r][4 * q]) = ra[t];
        }
        if constexpr (BT) {
#pragma unroll
            for (int t = 0; t < B_F4; ++t) {
                const int idx = tid + t * 256;
                const int r = idx / 4, q = idx % 4;
                *reinterpret_cast<floatx4*>(&Bs[buf][r][4 * q]) = rb[t];
            }
        } else {
#pragma unroll
            for (int t = 0; t < B_F4; ++t) {
                const int idx = tid + t * 256;
                const int kr = idx / (BN / 4), q = idx % (BN / 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) Bs[buf][4 * q + e][kr] = rb[t][e];
            }
        }
    };

    int buf = 0;
    if (kbeg < kend) {
        load_global(kbeg);
        store_lds(0);
    }
    __syncthreads();
    for (int k0 = kbeg; k0 < kend; k0 += KB) {
        const bool more = k0 + KB < kend;
        if (more) load_global(k0 + KB);
        floatx4 a_lo[MB], a_hi[MB], b_lo[NB], b_hi[NB];
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            const float* p = &As[buf][wm * WM + i * 32 + c][8 * h];
            a_lo[i] = *reinterpret_cast<const floatx4*>(p);
            a_hi[i] = *reinterpret_cast<const floatx4*>(p + 4);
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const float* p = &Bs[buf][wn * WN + j * 32 + c][8 * h];
            b_lo[j] = *reinterpret_cast<const floatx4*>(p);
            b_hi[j] = *reinterpret_cast<const floatx4*>(p + 4);
        }
#pragma unroll
        for (int s = 0; s < 8; ++s) {
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const float av = s < 4 ? a_lo[i][s] : a_hi[i][s - 4];
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const float bv = s < 4 ? b_lo[j][s] : b_hi[j][s - 4];
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc[i][j], 0, 0, 0);
                }
            }
        }
        if (more) store_lds(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }

#pragma unroll
    for (int i = 0; i < MB; ++i) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int gc = col0 + wn * WN + j * 32 + c;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int gr = row0 + wm * WM + i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
                if (gr < M && gc < N) {
                    if constexpr (SPLIT) {
                        partial[((size_t)blockIdx.z * M + gr) * N + gc] = acc[i][j][r];
                    } else {
                        C[(size_t)gr * ldc + gc] =
                            epilogue<EPI>(acc[i][j][r], R, (size_t)gr * ldr + gc);
                    }
                }
            }
        }
    }
}

// Adds the split partial sums in split order, then applies the epilogue.
template <int EPI>
__global__ void splitk_reduce_kernel(const float* __restrict__ partial, int splits, float* C,
                                     int ldc, int M, int N, const float* R, int ldr) {
    const size_t total = (size_t)M * N;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        float s = 0.0f;
        for (int z = 0; z < splits; ++z) s += partial[(size_t)z * total + i];
        const size_t r = i / N, col = i % N;
        C[r * ldc + col] = epilogue<EPI>(s, R, r * ldr + col);
    }
}

// ---------------------------------------------------------------------------------------
// NT tile kernel (B stored N x K: the projections' transposed weights).  Both operands are
// K-contiguous, so a KBT-wide K block of either tile is R rows of KBT/4 float4, which the wave
// copies from global memory straight into LDS (global_load_lds, 16 bytes per lane, 1 KB per
// instruction: 16 rows of a 16-wide block, 8 rows of a 32-wide one) without passing through
// registers.  Three LDS stages: the copies of block k+2 are in flight while block k is
// multiplied, with one barrier per block.  The 64 x 64 tiles take 32-wide blocks: 16 MFMAs per
// wave between barriers (measured on MI355X at the prefill projection shapes, 3 work-groups per
// CU: 10-15 % faster than 16-wide blocks at 6 per CU, whose waves wait at a barrier every 8).
// A copy instruction fills 1 KB of LDS contiguously, so rows cannot be padded; instead float4
// q of row r is stored at position q ^ nt_swz(r), which puts the operand reads of any 8 or 16
// consecutive lanes (one row each, same q) on distinct banks.  Rows past M (columns past N)
// copy row M-1 (N-1): their results are computed and never stored.  Same MFMA operand layout
// as gemm_mfma_kernel; lane half h takes the block's k = h KBT/2 .. + KBT/2 - 1.
// ---------------------------------------------------------------------------------------
// Depends on r % 16 only.  4 quads per row: ((r >> 1) ^ (r >> 3)) & 3; 8 quads per row:
// (r >> 1) & 7 with bit 2 flipped on odd rows (8 consecutive rows: 0 4 1 5 2 6 3 7).
__device__ __forceinline__ int quad_swz(int r) { return ((r >> 1) ^ ((r >> 3) & 1)) & 3; }
template <int KBT>
__device__ __forceinline__ int nt_swz(int r) {
    if constexpr (KBT == 16) return quad_swz(r);
    else return ((r >> 1) & 7) ^ ((r & 1) << 2);
}

constexpr int NT_STAGES = 3;
constexpr int NT_KB64 = 32;  // K block of the 64 x 64 tiles

// Whether the 64 x 64 NT tiles take 32-wide K blocks for a K range of k (FMLH_GEMM_NT_KB=16:
// 16-wide blocks everywhere, for comparison).
bool nt_wide_kb(int k) {
    static const bool narrow = [] {
        const char* e = std::getenv("FMLH_GEMM_NT_KB");
        return e && std::strcmp(e, "16") == 0;
    }();
    return !narrow && k % NT_KB64 == 0;
}

template <int BM, int BN, int KBT = KB>
constexpr size_t nt_lds_bytes() { return (size_t)NT_STAGES * (BM + BN) * KBT * sizeof(float); }

// SPLIT: work-group z of the grid's third dimension takes K range [z K, z K + K) (K is the
// range length) and writes its partial sums to partial[z][M][N] (epilogue by the reduction).
// K must be a multiple of KBT.
template <int BM, int BN, int EPI, bool SPLIT = false, int KBT = KB>
__global__ __launch_bounds__(256) void gemm_nt_kernel(
    const float* __restrict__ A, int lda, const float* __restrict__ B, int ldb,
    float* C, int ldc, int M, int N, int K, const float* R, int ldr, KvDest kv,
    float* __restrict__ partial = nullptr) {
    static_assert(!SPLIT || EPI == kEpiNone, "split partials take no epilogue");
    static_assert(BM % 64 == 0 && BN % 64 == 0, "tile must be a multiple of 64");
    static_assert(KBT == 16 || KBT == 32, "K block of 16 or 32");
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int MB = WM / 32, NB = WN / 32;
    constexpr int A_FL = BM * KBT, ST_FL = (BM + BN) * KBT;
    constexpr int QPR = KBT / 4, RPI = 64 / QPR;   // float4 per row, rows per copy instruction
    constexpr int NQ = QPR / 2;                    // float4 operand reads per row and block
    constexpr int DA = BM / (4 * RPI), DB = BN / (4 * RPI);  // copy instructions per wave per block
    constexpr int D = DA + DB;

    extern __shared__ __attribute__((aligned(16))) float nt_lds[];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int h = lane >> 5, c = lane & 31;
    const int row0 = blockIdx.y * BM, col0 = blockIdx.x * BN;
    const int nk = K / KBT;

    // Copy addressing: lane -> row (lane / QPR) of an RPI-row chunk and stored position
    // lane % QPR, which holds global float4 (lane % QPR) ^ nt_swz(row).
    const int crow = lane / QPR, cpos = lane % QPR;
    const int cq = cpos ^ nt_swz<KBT>(crow);  // chunks start at multiples of 8 rows: r % 16 ...
    const int cq8 = cpos ^ nt_swz<KBT>(crow + 8);  // ... is crow or crow + 8
    const float* asrc[DA];
    const float* bsrc[DB];
    const size_t kofs = SPLIT ? (size_t)blockIdx.z * K : 0;
#pragma unroll
    for (int t = 0; t < DA; ++t) {
        const int r = RPI * (wave + 4 * t);
        const int gr = min(row0 + r + crow, M - 1);
        asrc[t] = A + (size_t)gr * lda + kofs + 4 * ((r & 8) ? cq8 : cq);
    }
#pragma unroll
    for (int t = 0; t < DB; ++t) {
        const int r = RPI * (wave + 4 * t);
        const int gc = min(col0 + r + crow, N - 1);
        bsrc[t] = B + (size_t)gc * ldb + kofs + 4 * ((r & 8) ? cq8 : cq);
    }
    auto issue = [&](int kb, int st) {
        float* sa = nt_lds + st * ST_FL;
        float* sb = sa + A_FL;
#pragma unroll
        for (int t = 0; t < DA; ++t) copy16_to_lds(sa + (wave + 4 * t) * 256, asrc[t] + kb * KBT);
#pragma unroll
        for (int t = 0; t < DB; ++t) copy16_to_lds(sb + (wave + 4 * t) * 256, bsrc[t] + kb * KBT);
    };

    // Operand reads: lane (h, c) takes float4 h NQ .. h NQ + NQ - 1 of its row
    // (k = h KBT/2 .. h KBT/2 + KBT/2 - 1); rows wm WM + 32 i + c have r % 16 = c % 16.
    const int swc = nt_swz<KBT>(c);

    floatx16 acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    issue(0, 0);
    if (nk > 1) issue(1, 1);
    int st = 0;
    for (int kb = 0; kb < nk; ++kb) {
        // This wave's copies of block kb are done once at most those of block kb+1 remain;
        // the barrier makes every wave's part visible and ends all reads of the stage that
        // block kb+2 overwrites (it held block kb-1).
        // (__syncthreads would wait for every copy in flight, block kb+1's included.)
        if (kb + 1 < nk) copies_barrier<D>();
        else copies_barrier<0>();
        if (kb + 2 < nk) issue(kb + 2, st == 0 ? 2 : st - 1);
        const float* sa = nt_lds + st * ST_FL;
        const float* sb = sa + A_FL;
        floatx4 av[NQ][MB], bv[NQ][NB];
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            const int pos = (h * NQ + q) ^ swc;
#pragma unroll
            for (int i = 0; i < MB; ++i)
                av[q][i] = *reinterpret_cast<const floatx4*>(sa + (wm * WM + 32 * i + c) * KBT + 4 * pos);
#pragma unroll
            for (int j = 0; j < NB; ++j)
                bv[q][j] = *reinterpret_cast<const floatx4*>(sb + (wn * WN + 32 * j + c) * KBT + 4 * pos);
        }
#pragma unroll
        for (int s = 0; s < 4 * NQ; ++s) {
#pragma unroll
            for (int i = 0; i < MB; ++i) {
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[s / 4][i][s % 4], bv[s / 4][j][s % 4],
                                                                     acc[i][j], 0, 0, 0);
            }
        }
        // All operand reads first (first quads first: the first MFMAs wait for those only),
        // then the MFMAs, which the later reads overlap.
        __builtin_amdgcn_sched_group_barrier(0x100, NQ * (MB + NB), 0);  // LDS reads
        __builtin_amdgcn_sched_group_barrier(0x008, 4 * NQ * MB * NB, 0);  // MFMA
        st = st == NT_STAGES - 1 ? 0 : st + 1;
    }

    // kEpiKV: cache offset of each row of the tile, (sequence * H * T + position) * head_dim.
    __shared__ size_t kv_row[EPI == kEpiKV ? BM : 1];
    int kv_shift = 0;
    if constexpr (EPI == kEpiKV) {
        kv_shift = 31 - __builtin_clz(kv.hd);
        for (int rr = tid; rr < BM; rr += 256) {
            const int gr = min(row0 + rr, M - 1);
            const int b = gr / kv.rows_per_seq, p = gr - b * kv.rows_per_seq;
            kv_row[rr] = ((size_t)b * kv.H * kv.T + p) << kv_shift;
        }
        __syncthreads();
    }
    if constexpr (BM == 64 && BN == 64) {
        // The tile goes through LDS (the operand ring is free once every wave is past the
        // barrier below: every copy has landed and every read of the ring is done), then out
        // as 16-byte stores of whole row segments (a key/value tile row is one head's cache
        // row for head_dim 64, or 2-4 of them), where the destination's strides and alignment
        // allow it; otherwise the per-element stores below.
        const bool rows_ok = ((uintptr_t)C % 16 == 0) && ldc % 4 == 0 &&
                             (EPI != kEpiResid || ((uintptr_t)R % 16 == 0 && ldr % 4 == 0));
        const bool vec_ok = SPLIT ? (N % 4 == 0 && (uintptr_t)partial % 16 == 0)
                                  : (EPI == kEpiKV || (N % 4 == 0 && rows_ok));
        if (vec_ok) {
            constexpr int TS = BN + 4;  // padded row: the 16-byte reads stay aligned
            float* tile = nt_lds;
            if constexpr (EPI != kEpiKV) __syncthreads();  // (kEpiKV passed one above)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                tile[(wm * 32 + 8 * (r / 4) + 4 * h + (r % 4)) * TS + wn * 32 + c] = acc[0][0][r];
            __syncthreads();
#pragma unroll
            for (int u = 0; u < BM * BN / 4 / 256; ++u) {
                const int idx = tid + 256 * u, rr = idx / (BN / 4), q = idx % (BN / 4);
                const int gr = row0 + rr, gc = col0 + 4 * q;
                if (gr >= M || gc >= N) continue;  // N % 4 == 0: no float4 crosses N
                floatx4 v = *reinterpret_cast<const floatx4*>(tile + rr * TS + 4 * q);
                if constexpr (SPLIT) {
                    *reinterpret_cast<floatx4*>(partial + ((size_t)blockIdx.z * M + gr) * N + gc) = v;
                } else if constexpr (EPI == kEpiKV) {
                    if (gc < kv.C) {
                        *reinterpret_cast<floatx4*>(C + (size_t)gr * ldc + gc) = v;
                    } else {
                        const bool is_v = gc >= 2 * kv.C;
                        const int cc = gc - (is_v ? 2 * kv.C : kv.C);
                        const int hh = cc >> kv_shift, d = cc & (kv.hd - 1);
                        float* cache = is_v ? kv.vc : kv.kc;
                        *reinterpret_cast<floatx4*>(cache + kv_row[rr] + ((size_t)hh * kv.T << kv_shift) + d) = v;
                    }
                } else {
                    if constexpr (EPI == kEpiResid) {
                        const floatx4 rv = *reinterpret_cast<const floatx4*>(R + (size_t)gr * ldr + gc);
                        v += rv;
                    } else if constexpr (EPI != kEpiNone) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = epilogue<EPI>(v[e], R, 0);
                    }
                    *reinterpret_cast<floatx4*>(C + (size_t)gr * ldc + gc) = v;
                }
            }
            return;
        }
    }

#pragma unroll
    for (int i = 0; i < MB; ++i) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int gc = col0 + wn * WN + j * 32 + c;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int gr = row0 + wm * WM + i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
                if (gr < M && gc < N) {
                    if constexpr (SPLIT) {
                        partial[((size_t)blockIdx.z * M + gr) * N + gc] = acc[i][j][r];
                    } else if constexpr (EPI == kEpiKV) {
                        if (gc < kv.C) {
                            C[(size_t)gr * ldc + gc] = acc[i][j][r];
                        } else {
                            // head_dim is a power of two; the row's cache offset comes from LDS
                            const bool is_v = gc >= 2 * kv.C;
                            const int cc = gc - (is_v ? 2 * kv.C : kv.C);
                            const int hh = cc >> kv_shift, d = cc & (kv.hd - 1);
                            float* cache = is_v ? kv.vc : kv.kc;
                            cache[kv_row[gr - row0] + ((size_t)hh * kv.T << kv_shift) + d] = acc[i][j][r];
                        }
                    } else {
                        C[(size_t)gr * ldc + gc] = epilogue<EPI>(acc[i][j][r], R, (size_t)gr * ldr + gc);
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// Split-K NT kernel for short K ranges (batched decode: M <= 64 rows, K-range of at most
// kNtSplitMaxBlocks 16-wide blocks per work-group).  The whole range of both 64 x 64 tiles is
// copied into LDS at once (one stage per block), so the work-group waits for global memory
// once instead of once per block; then every MFMA runs back to back.  Writes the partial sums
// of split blockIdx.z to partial[z][M][N] (added up by the caller).  Same operand layout, LDS
// swizzle and k order as gemm_nt_kernel.
// ---------------------------------------------------------------------------------------
constexpr int kNtSplitMaxBlocks = 8;

__global__ __launch_bounds__(256) void gemm_nt_split_kernel(
    const float* __restrict__ A, int lda, const float* __restrict__ B, int ldb, int M, int N,
    int k_per_split, float* __restrict__ partial) {
    constexpr int BM = 64, BN = 64, A_FL = BM * KB, ST_FL = (BM + BN) * KB;
    extern __shared__ __attribute__((aligned(16))) float nts_lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int h = lane >> 5, c = lane & 31;
    const int row0 = blockIdx.y * BM, col0 = blockIdx.x * BN;
    const int kbeg = blockIdx.z * k_per_split;
    const int nk = k_per_split / KB;  // <= kNtSplitMaxBlocks (host check)

    const int crow = lane >> 2;
    const int cq = (lane & 3) ^ quad_swz(crow);
    const float* asrc = A + (size_t)min(row0 + 16 * wave + crow, M - 1) * lda + kbeg + 4 * cq;
    const float* bsrc = B + (size_t)min(col0 + 16 * wave + crow, N - 1) * ldb + kbeg + 4 * cq;
    for (int kb = 0; kb < nk; ++kb) {
        float* sa = nts_lds + kb * ST_FL;
        copy16_to_lds(sa + wave * 256, asrc + kb * KB);
        copy16_to_lds(sa + A_FL + wave * 256, bsrc + kb * KB);
    }
    const int p0 = (2 * h) ^ quad_swz(c);
    const int p1 = p0 ^ 1;
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    copies_barrier<0>();
    for (int kb = 0; kb < nk; ++kb) {
        const float* sa = nts_lds + kb * ST_FL + (wm * 32 + c) * KB;
        const float* sb = nts_lds + kb * ST_FL + A_FL + (wn * 32 + c) * KB;
        const floatx4 a_lo = *reinterpret_cast<const floatx4*>(sa + 4 * p0);
        const floatx4 b_lo = *reinterpret_cast<const floatx4*>(sb + 4 * p0);
        const floatx4 a_hi = *reinterpret_cast<const floatx4*>(sa + 4 * p1);
        const floatx4 b_hi = *reinterpret_cast<const floatx4*>(sb + 4 * p1);
#pragma unroll
        for (int s = 0; s < 8; ++s)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(s < 4 ? a_lo[s] : a_hi[s - 4],
                                                       s < 4 ? b_lo[s] : b_hi[s - 4], acc, 0, 0, 0);
    }
    const int gc = col0 + wn * 32 + c;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int gr = row0 + wm * 32 + 8 * (r / 4) + 4 * h + (r % 4);
        if (gr < M && gc < N) partial[((size_t)blockIdx.z * M + gr) * N + gc] = acc[r];
    }
}

// ---------------------------------------------------------------------------------------
// Skinny kernels (M <= 8).
// ---------------------------------------------------------------------------------------
constexpr int SK_MAXM = 8;
constexpr int SK_KCHUNK = 16;  // k rows per block of the NN kernel

// NN: B is K x N.  Block (x = 256-column strip, y = k chunk); lane owns 4 columns.  Writes
// partial[y][m][n]; splitk_reduce_kernel sums the chunks in order and applies the epilogue.
__global__ __launch_bounds__(64) void skinny_nn_partial_kernel(
    const float* __restrict__ A, int lda, const float* __restrict__ B, int ldb,
    float* __restrict__ partial, int M, int N, int K) {
    const int col = blockIdx.x * 256 + threadIdx.x * 4;
    const int k0 = blockIdx.y * SK_KCHUNK;
    const int k1 = min(K, k0 + SK_KCHUNK);
    if (col >= N) return;
    float acc[SK_MAXM][4];
#pragma unroll
    for (int m = 0; m < SK_MAXM; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[m][e] = 0.0f;
    const bool full = col + 3 < N;
    for (int k = k0; k < k1; ++k) {
        floatx4 w;
        const float* src = B + (size_t)k * ldb + col;
        if (full) {
            w = *reinterpret_cast<const floatx4*>(src);
        } else {
            w = floatx4{0.f, 0.f, 0.f, 0.f};
            for (int e = 0; e < 4; ++e)
                if (col + e < N) w[e] = src[e];
        }
#pragma unroll
        for (int m = 0; m < SK_MAXM; ++m) {
            if (m < M) {
                const float a = A[(size_t)m * lda + k];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[m][e] += a * w[e];
            }
        }
    }
#pragma unroll
    for (int m = 0; m < SK_MAXM; ++m) {
        if (m < M) {
            float* dst = partial + ((size_t)blockIdx.y * M + m) * N + col;
            for (int e = 0; e < 4; ++e)
                if (col + e < N) dst[e] = acc[m][e];
        }
    }
}

// NT: B is N x K (rows contiguous in k).  16 lanes per output column n, 4 columns per wave.
template <int EPI>
__global__ __launch_bounds__(64) void skinny_nt_kernel(
    const float* __restrict__ A, int lda, const float* __restrict__ B, int ldb, float* C, int ldc,
    int M, int N, int K, const float* R, int ldr) {
    const int sub = threadIdx.x % 16;
    const int n = blockIdx.x * 4 + threadIdx.x / 16;
    float acc[SK_MAXM];
#pragma unroll
    for (int m = 0; m < SK_MAXM; ++m) acc[m] = 0.0f;
    if (n < N) {
        const float* w = B + (size_t)n * ldb;
        for (int k = sub * 4; k < K; k += 64) {
            const floatx4 wv = *reinterpret_cast<const floatx4*>(w + k);
#pragma unroll
            for (int m = 0; m < SK_MAXM; ++m) {
                if (m < M) {
                    const floatx4 av = *reinterpret_cast<const floatx4*>(A + (size_t)m * lda + k);
                    acc[m] += av[0] * wv[0] + av[1] * wv[1] + av[2] * wv[2] + av[3] * wv[3];
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < SK_MAXM; ++m) {
        float v = acc[m];
        v += __shfl_xor(v, 8, 16);
        v += __shfl_xor(v, 4, 16);
        v += __shfl_xor(v, 2, 16);
        v += __shfl_xor(v, 1, 16);
        acc[m] = v;
    }
    if (n < N && sub == 0) {
#pragma unroll
        for (int m = 0; m < SK_MAXM; ++m)
            if (m < M) C[(size_t)m * ldc + n] = epilogue<EPI>(acc[m], R, (size_t)m * ldr + n);
    }
}

// NT, KS waves per output column (KS = 1, 2 or 4): wave j of a column takes float4 chunks
// j, j + KS, ... of each 64-chunk stretch of K (its 64 lanes side by side, four chunks in flight
// per lane) and keeps the M <= 8 row partials; a wave reduction, then the KS waves' sums added in
// wave order through LDS.  4 / KS columns per work-group: small N (the residual projections,
// N = C) still spreads over every CU.
// LN: A holds rows before a LayerNorm; the work-group first forms each row's mean and 1/std
// exactly as layernorm_kernel does (wave per row, lane l holding elements l + 64 i, two-pass
// variance), then normalises the A values it loads: ((a - mean) * inv_std) * gamma + beta.
constexpr int kSkLnNE = 16;  // row elements per lane of the statistics pass (K <= 1024)

template <int EPI, int KS, bool LN = false>
__global__ __launch_bounds__(256) void skinny_nt_wave_kernel(
    const float* __restrict__ A, int lda, const float* __restrict__ B, int ldb, float* C, int ldc,
    int M, int N, int K, const float* R, int ldr, const float* __restrict__ ln_g = nullptr,
    const float* __restrict__ ln_b = nullptr, float ln_eps = 0.0f) {
    constexpr int CPW = 4 / KS;  // columns per work-group
    __shared__ float part[4][SK_MAXM];
    __shared__ float ln_st[LN ? SK_MAXM : 1][2];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = wave / KS, j = wave % KS;
    const int n = blockIdx.x * CPW + col;
    if constexpr (LN) {
        const float inv_cols = 1.0f / (float)K;
        for (int m = wave; m < M; m += 4) {
            const float* xr = A + (size_t)m * lda;
            float v[kSkLnNE];
#pragma unroll
            for (int i = 0; i < kSkLnNE; ++i) {
                const int c = lane + 64 * i;
                v[i] = c < K ? xr[c] : 0.0f;
            }
            float sum = 0.0f;
#pragma unroll
            for (int i = 0; i < kSkLnNE; ++i)
                if (lane + 64 * i < K) sum += v[i];
            const float mean = wave_sum(sum) * inv_cols;
            float q = 0.0f;
#pragma unroll
            for (int i = 0; i < kSkLnNE; ++i)
                if (lane + 64 * i < K) {
                    const float d = v[i] - mean;
                    q += d * d;
                }
            const float inv_std = 1.0f / sqrtf(wave_sum(q) * inv_cols + ln_eps);
            if (lane == 0) {
                ln_st[m][0] = mean;
                ln_st[m][1] = inv_std;
            }
        }
        __syncthreads();
    }
    // The residual's values are loaded now, so the store does not wait for another round trip.
    float rv[SK_MAXM];
    if constexpr (EPI == kEpiResid) {
        if (n < N && j == 0 && lane == 0) {
#pragma unroll
            for (int m = 0; m < SK_MAXM; ++m) rv[m] = m < M ? R[(size_t)m * ldr + n] : 0.0f;
        }
    }
    float acc[SK_MAXM];
#pragma unroll
    for (int m = 0; m < SK_MAXM; ++m) acc[m] = 0.0f;
    if (n < N) {
        const float* w = B + (size_t)n * ldb;
        const int nch = K / 4;
#pragma unroll 4
        for (int e = lane + 64 * j; e < nch; e += 64 * KS) {
            const floatx4 wv = *reinterpret_cast<const floatx4*>(w + 4 * e);
            floatx4 gv, bv;
            if constexpr (LN) {
                gv = *reinterpret_cast<const floatx4*>(ln_g + 4 * e);
                if (ln_b) bv = *reinterpret_cast<const floatx4*>(ln_b + 4 * e);
                else bv = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            }
#pragma unroll
            for (int m = 0; m < SK_MAXM; ++m) {
                if (m < M) {
                    floatx4 av = *reinterpret_cast<const floatx4*>(A + (size_t)m * lda + 4 * e);
                    if constexpr (LN) {
                        const float mean = ln_st[m][0], inv_std = ln_st[m][1];
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            const float nrm = (av[t] - mean) * inv_std;
                            av[t] = nrm * gv[t] + bv[t];
                        }
                    }
                    acc[m] += av[0] * wv[0] + av[1] * wv[1] + av[2] * wv[2] + av[3] * wv[3];
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < SK_MAXM; ++m)
        if (m < M) acc[m] = wave_sum(acc[m]);
    if constexpr (KS > 1) {
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < SK_MAXM; ++m) part[wave][m] = acc[m];
        }
        __syncthreads();
        if (j == 0) {
#pragma unroll
            for (int m = 0; m < SK_MAXM; ++m) {
                float t = part[wave][m];
#pragma unroll
                for (int q = 1; q < KS; ++q) t += part[wave + q][m];
                acc[m] = t;
            }
        }
    }
    if (n < N && j == 0 && lane == 0) {
#pragma unroll
        for (int m = 0; m < SK_MAXM; ++m) {
            if (m < M) {
                if constexpr (EPI == kEpiResid) C[(size_t)m * ldc + n] = rv[m] + acc[m];
                else C[(size_t)m * ldc + n] = epilogue<EPI>(acc[m], R, (size_t)m * ldr + n);
            }
        }
    }
}

// Wide products (N > 4096, e.g. a 50304-row lm_head): one wave per group of NC columns, so
// every activation float4 the wave loads serves NC weight rows (with one column per wave the
// M <= 8 activation rows are re-read from the caches once per column: ~8x the weight bytes).
// Per column the arithmetic is that of skinny_nt_wave_kernel with KS = 1.
template <int EPI, int NC>
__global__ __launch_bounds__(256) void skinny_nt_wide_kernel(
    const float* __restrict__ A, int lda, const float* __restrict__ B, int ldb, float* C, int ldc,
    int M, int N, int K, const float* R, int ldr) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * 4 + wave) * NC;
    if (n0 >= N) return;  // wave-uniform; no barrier follows
    const float* w[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) w[c] = B + (size_t)min(n0 + c, N - 1) * ldb;
    float acc[NC][SK_MAXM];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int m = 0; m < SK_MAXM; ++m) acc[c][m] = 0.0f;
    const int nch = K / 4;
#pragma unroll 2
    for (int e = lane; e < nch; e += 64) {
        floatx4 wv[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) wv[c] = *reinterpret_cast<const floatx4*>(w[c] + 4 * e);
#pragma unroll
        for (int m = 0; m < SK_MAXM; ++m) {
            if (m < M) {
                const floatx4 av = *reinterpret_cast<const floatx4*>(A + (size_t)m * lda + 4 * e);
#pragma unroll
                for (int c = 0; c < NC; ++c)
                    acc[c][m] += av[0] * wv[c][0] + av[1] * wv[c][1] + av[2] * wv[c][2] + av[3] * wv[c][3];
            }
        }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int m = 0; m < SK_MAXM; ++m)
            if (m < M) acc[c][m] = wave_sum(acc[c][m]);
    if (lane == 0) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int n = n0 + c;
            if (n < N) {
#pragma unroll
                for (int m = 0; m < SK_MAXM; ++m)
                    if (m < M) C[(size_t)m * ldc + n] = epilogue<EPI>(acc[c][m], R, (size_t)m * ldr + n);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// Generic strided product: C[i*o_rs + j*o_cs] = sum_k A(i,k) B(k,j), batched over planes.
// A(i,k) = L[i*l_rs + k*l_cs] (TL: L[k*l_rs + i*l_cs]); B(k,j) = R[k*r_rs + j*r_cs]
// (TR: R[j*r_rs + k*r_cs]).  The callers are FreeML's per-head attention products and the
// Dense weight gradients (Mul<Left>): small outputs (e.g. 256 x 64) over K of a few hundred,
// so the tile is 32 x 32 (more work-groups per product) and K is staged in chunks of 64 with
// the next chunk's loads in flight (registers) while the current one is multiplied from LDS.
// Each thread loads with the strided operand's contiguous index fastest across threads.
// ---------------------------------------------------------------------------------------
constexpr uint32_t kStT = 32, kStKC = 64, kStPer = kStT * kStKC / 256;

template <bool TL, bool TR>
__global__ __launch_bounds__(256) void gemm_strided_kernel(
    float* __restrict__ out, const float* __restrict__ L, const float* __restrict__ Rm,
    uint32_t M, uint32_t N, uint32_t K, uint32_t l_rs, uint32_t l_cs, uint32_t r_rs,
    uint32_t r_cs, uint32_t o_rs, uint32_t o_cs, size_t l_plane, size_t r_plane,
    size_t o_plane) {
    __shared__ float As[kStKC][kStT + 1];  // As[k][i]
    __shared__ float Bs[kStKC][kStT + 1];  // Bs[k][j]
    const float* Lp = L + blockIdx.z * l_plane;
    const float* Rp = Rm + blockIdx.z * r_plane;
    float* Op = out + blockIdx.z * o_plane;
    const uint32_t row0 = blockIdx.y * kStT, col0 = blockIdx.x * kStT;
    const uint32_t t = threadIdx.x;
    // Element e = t + 256 r of a chunk: (i, k) of A and (k, j) of B.
    auto a_ik = [&](uint32_t e, uint32_t& i, uint32_t& k) {
        if (TL) { i = e % kStT; k = e / kStT; } else { k = e % kStKC; i = e / kStKC; }
    };
    auto b_kj = [&](uint32_t e, uint32_t& k, uint32_t& j) {
        if (TR) { k = e % kStKC; j = e / kStKC; } else { j = e % kStT; k = e / kStT; }
    };
    float ra[kStPer], rb[kStPer];
    auto load = [&](uint32_t k0) {
#pragma unroll
        for (uint32_t r = 0; r < kStPer; ++r) {
            uint32_t i, k, j, kb;
            a_ik(t + 256 * r, i, k);
            b_kj(t + 256 * r, kb, j);
            const uint32_t gi = row0 + i, gk = k0 + k, gj = col0 + j, gkb = k0 + kb;
            ra[r] = (gi < M && gk < K)
                        ? (TL ? Lp[(size_t)gk * l_rs + (size_t)gi * l_cs] : Lp[(size_t)gi * l_rs + (size_t)gk * l_cs])
                        : 0.0f;
            rb[r] = (gj < N && gkb < K)
                        ? (TR ? Rp[(size_t)gj * r_rs + (size_t)gkb * r_cs] : Rp[(size_t)gkb * r_rs + (size_t)gj * r_cs])
                        : 0.0f;
        }
    };
    const uint32_t tx = t % 16, ty = t / 16;  // outputs (2 ty + a, 2 tx + b)
    float acc[2][2] = {};
    load(0);
    for (uint32_t k0 = 0; k0 < K; k0 += kStKC) {
        __syncthreads();  // the previous chunk has been read out of LDS
#pragma unroll
        for (uint32_t r = 0; r < kStPer; ++r) {
            uint32_t i, k, j, kb;
            a_ik(t + 256 * r, i, k);
            b_kj(t + 256 * r, kb, j);
            As[k][i] = ra[r];
            Bs[kb][j] = rb[r];
        }
        __syncthreads();
        if (k0 + kStKC < K) load(k0 + kStKC);
#pragma unroll 16
        for (uint32_t kk = 0; kk < kStKC; ++kk) {
            const float a0 = As[kk][2 * ty], a1 = As[kk][2 * ty + 1];
            const float b0 = Bs[kk][2 * tx], b1 = Bs[kk][2 * tx + 1];
            acc[0][0] += a0 * b0;
            acc[0][1] += a0 * b1;
            acc[1][0] += a1 * b0;
            acc[1][1] += a1 * b1;
        }
    }
#pragma unroll
    for (uint32_t a = 0; a < 2; ++a) {
        const uint32_t gi = row0 + 2 * ty + a;
#pragma unroll
        for (uint32_t b = 0; b < 2; ++b) {
            const uint32_t gj = col0 + 2 * tx + b;
            if (gi < M && gj < N) Op[(size_t)gi * o_rs + (size_t)gj * o_cs] = acc[a][b];
        }
    }
}

// Same product for K > kStKC: the work-group's four waves each take one K chunk of every pass
// (pass = 4 chunks) for the same TT x TT output tile, with the next pass's operands in flight
// during the multiply; the four partial tiles are then added in wave order (deterministic).
// TT = 16 (chunk 64) spreads small outputs over more work-groups -- a 256 x 64 per-head
// product with K = 256 becomes 64 work-groups that each load all of K at once -- and TT = 32
// (chunk 32) serves larger outputs.  Lane (tx, ty) = (lane % 8, lane / 8) holds the
// MT x MT outputs (MT ty + x, MT tx + y), MT = TT / 8.
constexpr uint32_t kWsWaves = 4;

template <uint32_t MT> struct VecOf;
template <> struct VecOf<2> { using type = float2; };
template <> struct VecOf<4> { using type = float4; };

template <bool TL, bool TR, uint32_t TT>
__global__ __launch_bounds__(256) void gemm_strided_wsplit_kernel(
    float* __restrict__ out, const float* __restrict__ L, const float* __restrict__ Rm,
    uint32_t M, uint32_t N, uint32_t K, uint32_t l_rs, uint32_t l_cs, uint32_t r_rs,
    uint32_t r_cs, uint32_t o_rs, uint32_t o_cs, size_t l_plane, size_t r_plane,
    size_t o_plane) {
    constexpr uint32_t KC = 1024 / TT;        // K chunk per wave
    constexpr uint32_t LD = TT + 4;           // LDS row stride (rows stay 16-byte aligned)
    constexpr uint32_t PER = TT * KC / kWave;  // elements per lane per operand (16)
    constexpr uint32_t MT = TT / 8;           // lane micro-tile
    using Vec = typename VecOf<MT>::type;
    static_assert(TT * TT <= 2 * KC * LD, "partial tile must fit the wave's LDS slice");
    __shared__ __attribute__((aligned(16))) float sm[kWsWaves][2 * KC * LD];
    const float* Lp = L + blockIdx.z * l_plane;
    const float* Rp = Rm + blockIdx.z * r_plane;
    float* Op = out + blockIdx.z * o_plane;
    const uint32_t row0 = blockIdx.y * TT, col0 = blockIdx.x * TT;
    const uint32_t lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
    float* As = sm[w];            // As[k * LD + i]
    float* Bs = sm[w] + KC * LD;  // Bs[k * LD + j]
    auto a_ik = [&](uint32_t e, uint32_t& i, uint32_t& k) {
        if (TL) { i = e % TT; k = e / TT; } else { k = e % KC; i = e / KC; }
    };
    auto b_kj = [&](uint32_t e, uint32_t& k, uint32_t& j) {
        if (TR) { k = e % KC; j = e / KC; } else { j = e % TT; k = e / TT; }
    };
    float ra[PER], rb[PER];
    auto load = [&](uint32_t k0) {
#pragma unroll
        for (uint32_t r = 0; r < PER; ++r) {
            uint32_t i, k, j, kb;
            a_ik(lane + kWave * r, i, k);
            b_kj(lane + kWave * r, kb, j);
            const uint32_t gi = row0 + i, gk = k0 + k, gj = col0 + j, gkb = k0 + kb;
            ra[r] = (gi < M && gk < K)
                        ? (TL ? Lp[(size_t)gk * l_rs + (size_t)gi * l_cs] : Lp[(size_t)gi * l_rs + (size_t)gk * l_cs])
                        : 0.0f;
            rb[r] = (gj < N && gkb < K)
                        ? (TR ? Rp[(size_t)gj * r_rs + (size_t)gkb * r_cs] : Rp[(size_t)gkb * r_rs + (size_t)gj * r_cs])
                        : 0.0f;
        }
    };
    const uint32_t tx = lane % 8, ty = lane / 8;
    float acc[MT][MT] = {};
    constexpr uint32_t kPass = kWsWaves * KC;
    load(w * KC);
    for (uint32_t kp = 0; kp < K; kp += kPass) {
        __syncthreads();  // this wave's previous chunk has been read out of LDS
#pragma unroll
        for (uint32_t r = 0; r < PER; ++r) {
            uint32_t i, k, j, kb;
            a_ik(lane + kWave * r, i, k);
            b_kj(lane + kWave * r, kb, j);
            As[k * LD + i] = ra[r];
            Bs[kb * LD + j] = rb[r];
        }
        __syncthreads();
        if (kp + kPass < K) load(kp + kPass + w * KC);
#pragma unroll 8
        for (uint32_t kk = 0; kk < KC; ++kk) {
            const Vec a = *reinterpret_cast<const Vec*>(&As[kk * LD + MT * ty]);
            const Vec b = *reinterpret_cast<const Vec*>(&Bs[kk * LD + MT * tx]);
            const float* av = reinterpret_cast<const float*>(&a);
            const float* bv = reinterpret_cast<const float*>(&b);
#pragma unroll
            for (uint32_t x = 0; x < MT; ++x)
#pragma unroll
                for (uint32_t y = 0; y < MT; ++y) acc[x][y] += av[x] * bv[y];
        }
    }
    __syncthreads();
    float* part = sm[w];  // this wave's TT x TT partial tile, row-major
#pragma unroll
    for (uint32_t x = 0; x < MT; ++x)
#pragma unroll
        for (uint32_t y = 0; y < MT; ++y) part[(MT * ty + x) * TT + MT * tx + y] = acc[x][y];
    __syncthreads();
    for (uint32_t idx = threadIdx.x; idx < TT * TT; idx += 256) {
        const uint32_t i = idx / TT, j = idx % TT;
        float v = sm[0][idx];
#pragma unroll
        for (uint32_t ww = 1; ww < kWsWaves; ++ww) v += sm[ww][idx];
        const uint32_t gi = row0 + i, gj = col0 + j;
        if (gi < M && gj < N) Op[(size_t)gi * o_rs + (size_t)gj * o_cs] = v;
    }
}

// Process-wide split-K workspace for callers that do not bring their own.
std::mutex g_ws_mu;
float* g_ws = nullptr;
size_t g_ws_elems = 0;

int global_workspace(size_t elems, float** ws) {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    if (elems > g_ws_elems) {
        if (g_ws) {
            FMLH_HIP(hipStreamSynchronize(stream()));
            FMLH_HIP(hipFree(g_ws));
            g_ws = nullptr;
            g_ws_elems = 0;
        }
        FMLH_TRY(device_malloc(reinterpret_cast<void**>(&g_ws), elems * sizeof(float)));
        g_ws_elems = elems;
    }
    *ws = g_ws;
    return FMLH_OK;
}

template <int EPI>
int launch_reduce(const float* partial, int splits, float* C, int ldc, int M, int N,
                  const float* R, int ldr, hipStream_t s) {
    const size_t total = (size_t)M * N;
    hipLaunchKernelGGL(splitk_reduce_kernel<EPI>, dim3(blocks_for(total, 256, 4096u)), dim3(256), 0,
                       s, partial, splits, C, ldc, M, N, R, ldr);
    FMLH_LAUNCHED("splitk_reduce_kernel");
    return FMLH_OK;
}

int reduce_dispatch(int epi, const float* partial, int splits, float* C, int ldc, int M, int N,
                    const float* R, int ldr, hipStream_t s) {
    switch (epi) {
        case kEpiGelu: return launch_reduce<kEpiGelu>(partial, splits, C, ldc, M, N, R, ldr, s);
        case kEpiResid: return launch_reduce<kEpiResid>(partial, splits, C, ldc, M, N, R, ldr, s);
        default: return launch_reduce<kEpiNone>(partial, splits, C, ldc, M, N, R, ldr, s);
    }
}

template <int BM, int BN, bool BT, int EPI>
int launch_mfma(const GemmArgs& g, int splits, int k_per_split, float* ws) {
    dim3 grid((g.N + BN - 1) / BN, (g.M + BM - 1) / BM, splits);
    if (splits > 1) {
        hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, BT, EPI, true>), grid, dim3(256), 0, g.s, g.A,
                           g.lda, g.B, g.ldb, g.C, g.ldc, g.M, g.N, g.K, g.R, g.ldr, ws, k_per_split);
        FMLH_LAUNCHED("gemm_mfma_kernel(split)");
        return reduce_dispatch(g.epi, ws, splits, g.C, g.ldc, g.M, g.N, g.R, g.ldr, g.s);
    }
    hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, BT, EPI, false>), grid, dim3(256), 0, g.s, g.A,
                       g.lda, g.B, g.ldb, g.C, g.ldc, g.M, g.N, g.K, g.R, g.ldr, nullptr, 0);
    FMLH_LAUNCHED("gemm_mfma_kernel");
    return FMLH_OK;
}

template <int BM, int BN, bool BT>
int mfma_epi(const GemmArgs& g, int splits, int kps, float* ws) {
    switch (g.epi) {
        case kEpiGelu: return launch_mfma<BM, BN, BT, kEpiGelu>(g, splits, kps, ws);
        case kEpiResid: return launch_mfma<BM, BN, BT, kEpiResid>(g, splits, kps, ws);
        default: return launch_mfma<BM, BN, BT, kEpiNone>(g, splits, kps, ws);
    }
}

template <int BM, int BN>
int mfma_tile(const GemmArgs& g, int splits, int kps, float* ws) {
    return g.b_trans ? mfma_epi<BM, BN, true>(g, splits, kps, ws)
                     : mfma_epi<BM, BN, false>(g, splits, kps, ws);
}

template <int BM, int BN, int EPI>
int launch_nt_tile(const GemmArgs& g) {
    dim3 grid((g.N + BN - 1) / BN, (g.M + BM - 1) / BM);
    if (BM == 64 && BN == 64 && nt_wide_kb(g.K)) {
        const size_t lds = nt_lds_bytes<BM, BN, NT_KB64>();
        hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, EPI, false, NT_KB64>), grid, dim3(256), lds, g.s,
                           g.A, g.lda, g.B, g.ldb, g.C, g.ldc, g.M, g.N, g.K, g.R, g.ldr, g.kv);
    } else {
        const size_t lds = nt_lds_bytes<BM, BN>();
        hipLaunchKernelGGL((gemm_nt_kernel<BM, BN, EPI>), grid, dim3(256), lds, g.s,
                           g.A, g.lda, g.B, g.ldb, g.C, g.ldc, g.M, g.N, g.K, g.R, g.ldr, g.kv);
    }
    FMLH_LAUNCHED("gemm_nt_kernel");
    return FMLH_OK;
}

// 64 x 64 NT partial sums over `splits` K ranges of k_per_split (multiple of KB) each.
void launch_nt_partials(const GemmArgs& g, int splits, int k_per_split, float* ws) {
    dim3 grid((g.N + 63) / 64, (g.M + 63) / 64, splits);
    if (nt_wide_kb(k_per_split)) {
        const size_t lds = nt_lds_bytes<64, 64, NT_KB64>();
        hipLaunchKernelGGL((gemm_nt_kernel<64, 64, kEpiNone, true, NT_KB64>), grid, dim3(256), lds, g.s,
                           g.A, g.lda, g.B, g.ldb, g.C, g.ldc, g.M, g.N, k_per_split, g.R, g.ldr, g.kv, ws);
    } else {
        const size_t lds = nt_lds_bytes<64, 64>();
        hipLaunchKernelGGL((gemm_nt_kernel<64, 64, kEpiNone, true>), grid, dim3(256), lds, g.s,
                           g.A, g.lda, g.B, g.ldb, g.C, g.ldc, g.M, g.N, k_per_split, g.R, g.ldr, g.kv, ws);
    }
}

// NT tiles with split K (plan splits > 1): partials, then the reduction with the epilogue.
int launch_nt_split_tiles(const GemmArgs& g, const GemmPlan& p, float* ws) {
    launch_nt_partials(g, p.splits, p.k_per_split, ws);
    FMLH_LAUNCHED("gemm_nt_kernel(split)");
    return reduce_dispatch(g.epi, ws, p.splits, g.C, g.ldc, g.M, g.N, g.R, g.ldr, g.s);
}

template <int BM, int BN>
int nt_epi(const GemmArgs& g) {
    switch (g.epi) {
        case kEpiGelu: return launch_nt_tile<BM, BN, kEpiGelu>(g);
        case kEpiResid: return launch_nt_tile<BM, BN, kEpiResid>(g);
        case kEpiKV: return launch_nt_tile<BM, BN, kEpiKV>(g);
        default: return launch_nt_tile<BM, BN, kEpiNone>(g);
    }
}

template <int EPI>
int launch_nt(const GemmArgs& g) {
    const char* env = std::getenv("FMLH_GEMM_SKINNY");  // "quad": 16 lanes per column
    if (g.ln_g != nullptr || !(env && std::strcmp(env, "quad") == 0)) {
        // Waves per column so that the launch has >= ~2048 waves when N is small.
        const int ks = g.N <= 1024 ? 4 : (g.N <= 4096 ? 2 : 1);
        const char* wide = std::getenv("FMLH_SKINNY_WIDE_NC");  // columns per wave, N > 4096
        const int wnc = wide ? std::atoi(wide) : 4;
        if (ks == 1 && g.ln_g == nullptr && (wnc == 2 || wnc == 4)) {
            const unsigned wwgs = (unsigned)((g.N + 4 * wnc - 1) / (4 * wnc));
            if (wnc == 4)
                hipLaunchKernelGGL((skinny_nt_wide_kernel<EPI, 4>), dim3(wwgs), dim3(256), 0, g.s, g.A, g.lda,
                                   g.B, g.ldb, g.C, g.ldc, g.M, g.N, g.K, g.R, g.ldr);
            else
                hipLaunchKernelGGL((skinny_nt_wide_kernel<EPI, 2>), dim3(wwgs), dim3(256), 0, g.s, g.A, g.lda,
                                   g.B, g.ldb, g.C, g.ldc, g.M, g.N, g.K, g.R, g.ldr);
            FMLH_LAUNCHED("skinny_nt_wide_kernel");
            return FMLH_OK;
        }
        const unsigned wgs = (unsigned)((g.N * ks + 3) / 4);
#define FMLH_SKW(KSV, LNV)                                                                        \
    hipLaunchKernelGGL((skinny_nt_wave_kernel<EPI, KSV, LNV>), dim3(wgs), dim3(256), 0, g.s, g.A, g.lda, \
                       g.B, g.ldb, g.C, g.ldc, g.M, g.N, g.K, g.R, g.ldr, g.ln_g, g.ln_b, g.ln_eps)
        if (g.ln_g != nullptr) {
            if (ks == 4) FMLH_SKW(4, true);
            else if (ks == 2) FMLH_SKW(2, true);
            else FMLH_SKW(1, true);
        } else {
            if (ks == 4) FMLH_SKW(4, false);
            else if (ks == 2) FMLH_SKW(2, false);
            else FMLH_SKW(1, false);
        }
#undef FMLH_SKW
        FMLH_LAUNCHED("skinny_nt_wave_kernel");
        return FMLH_OK;
    }
    hipLaunchKernelGGL(skinny_nt_kernel<EPI>, dim3((g.N + 3) / 4), dim3(64), 0, g.s, g.A, g.lda,
                       g.B, g.ldb, g.C, g.ldc, g.M, g.N, g.K, g.R, g.ldr);
    FMLH_LAUNCHED("skinny_nt_kernel");
    return FMLH_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The split-K NT kernel takes B stored N x K, 64 x 64 tiles and K ranges of at most
// kNtSplitMaxBlocks blocks (the callers have checked alignment and K % 16).
bool nt_split_applies(const GemmArgs& g, const GemmPlan& p) {
    const char* env = std::getenv("FMLH_GEMM_NT_SPLIT");  // "0": register-staged split kernel
    if (env && env[0] == '0') return false;
    return g.b_trans && p.kind == GemmPlan::kMfma && p.splits > 1 && p.bm == 64 && p.bn == 64 &&
           p.k_per_split % KB == 0 && p.k_per_split / KB <= kNtSplitMaxBlocks;
}

int launch_nt_split(const GemmArgs& g, const GemmPlan& p, float* ws) {
    dim3 grid((g.N + 63) / 64, (g.M + 63) / 64, p.splits);
    const size_t lds = (size_t)(p.k_per_split / KB) * 128 * KB * sizeof(float);
    hipLaunchKernelGGL(gemm_nt_split_kernel, grid, dim3(256), lds, g.s, g.A, g.lda, g.B, g.ldb, g.M,
                       g.N, p.k_per_split, ws);
    FMLH_LAUNCHED("gemm_nt_split_kernel");
    return FMLH_OK;
}

}  // namespace

GemmPlan plan_gemm(int M, int N, int K, int b_trans) {
    GemmPlan p;
    if (M <= SK_MAXM) {
        if (b_trans) {
            p.kind = GemmPlan::kSkinnyNT;
        } else {
            p.kind = GemmPlan::kSkinnyNN;
            p.splits = (K + SK_KCHUNK - 1) / SK_KCHUNK;
            p.ws_elems = (size_t)p.splits * M * N;
        }
        return p;
    }
    const int cus = cu_count() > 0 ? cu_count() : 256;
    // FMLH_GEMM_NT: "0" puts B-transposed products on gemm_mfma_kernel, "1" on the NT kernel
    // whatever the tile count (for measurement).
    const char* nt_env = std::getenv("FMLH_GEMM_NT");
    const bool nt_forced = nt_env && nt_env[0] == '1';
    if (b_trans && (nt_forced || (long)((M + 63) / 64) * ((N + 63) / 64) * 2 >= cus) &&
        !(nt_env && nt_env[0] == '0')) {
        // NT kernel, 64 x 64 tiles: measured on MI355X at the prefill projection shapes
        // (M 4096-14336, N 384-3072, K 384-3072) within 2% of the best of 64x64, 128x64 and
        // 128x128 everywhere (six work-groups per CU hide the operand-read latency, and small
        // tiles leave no CU idle at the end).  FMLH_GEMM_NT_TILE=128x128|128x64 selects the others.
        p.kind = GemmPlan::kMfmaNT;
        p.bm = 64;
        p.bn = 64;
        // Fewer than two 64 x 64 tiles per CU leaves CUs idle in the last round; with a long K
        // range, two K halves balance the grid (partials + a reduction kernel).
        // FMLH_GEMM_NT_SPLIT_K=0 turns it off.
        const long tiles = (long)((M + 63) / 64) * ((N + 63) / 64);
        const char* sk = std::getenv("FMLH_GEMM_NT_SPLIT_K");
        if (!(sk && sk[0] == '0') && tiles < 2L * cus && K >= 1024 && (K / 2) % KB == 0) {
            p.splits = 2;
            p.k_per_split = K / 2;
            p.ws_elems = (size_t)2 * M * N;
        }
        if (const char* e = std::getenv("FMLH_GEMM_NT_TILE")) {
            int bm = 0, bn = 0;
            if (std::sscanf(e, "%dx%d", &bm, &bn) == 2 &&
                ((bm == 128 && (bn == 128 || bn == 64)) || (bm == 64 && bn == 64))) {
                p.bm = bm; p.bn = bn;
            }
        }
        return p;
    }
    p.kind = GemmPlan::kMfma;
    const long t128 = (long)((M + 127) / 128) * ((N + 127) / 128);
    const long t64 = (long)((M + 63) / 64) * ((N + 63) / 64);
    long tiles;
    if (t128 >= cus) { p.bm = 128; p.bn = 128; tiles = t128; }
    else { p.bm = 64; p.bn = 64; tiles = t64; }
    // Split K when the tile grid cannot fill the device (skinny batched-decode shapes).
    int splits = 1;
    while (tiles * splits * 2 <= cus && K / (splits * 2) >= 64 && (K / (splits * 2)) % KB == 0)
        splits *= 2;
    p.splits = splits;
    p.k_per_split = K / splits;
    p.ws_elems = splits > 1 ? (size_t)splits * M * N : 0;
    return p;
}

bool gemm_takes_ln(int M, int N, int K, int b_trans) {
    return M > 0 && N > 0 && K <= 64 * kSkLnNE && plan_gemm(M, N, K, b_trans).kind == GemmPlan::kSkinnyNT;
}

bool gemm_runs_nt(const GemmArgs& g) {
    const bool vec_ok = aligned16(g.A) && aligned16(g.B) && g.lda % 4 == 0 && g.ldb % 4 == 0 &&
                        g.K % KB == 0;
    return vec_ok && g.M > 0 && g.N > 0 && plan_gemm(g.M, g.N, g.K, g.b_trans).kind == GemmPlan::kMfmaNT;
}

size_t gemm_workspace_elems(const GemmArgs& g) {
    if (g.M == 0 || g.N == 0 || g.K == 0) return 0;
    const bool vec_ok = aligned16(g.A) && aligned16(g.B) && g.lda % 4 == 0 && g.ldb % 4 == 0 &&
                        g.K % KB == 0;
    return vec_ok ? plan_gemm(g.M, g.N, g.K, g.b_trans).ws_elems : 0;  // the strided fallback takes none
}

int gemm(const GemmArgs& g, float* ws, size_t ws_elems) {
    if (g.M == 0 || g.N == 0) return FMLH_OK;
    FMLH_REQUIRE(g.K > 0, "gemm: K == 0");
    FMLH_REQUIRE(g.ln_g == nullptr || gemm_takes_ln(g.M, g.N, g.K, g.b_trans),
                 "gemm: a LayerNorm on A needs the skinny NT path (M <= 8, K <= 1024)");
    FMLH_REQUIRE(g.epi != kEpiKV || (gemm_runs_nt(g) && g.kv.kc && g.kv.vc && g.N == 3 * g.kv.C &&
                                     g.kv.hd > 0 && (g.kv.hd & (g.kv.hd - 1)) == 0),
                 "gemm: the cache-writing epilogue needs the NT kernel, N = 3 C and a power-of-two head_dim");
    const bool vec_ok = aligned16(g.A) && aligned16(g.B) && g.lda % 4 == 0 && g.ldb % 4 == 0 &&
                        g.K % KB == 0;
    FMLH_REQUIRE(g.ln_g == nullptr || (vec_ok && aligned16(g.ln_g) && (g.ln_b == nullptr || aligned16(g.ln_b))),
                 "gemm: a LayerNorm on A needs 16-byte aligned rows and parameters");
    if (!vec_ok) {
        // Fallback: generic strided kernel, then the epilogue through the reduce kernel.
        FMLH_REQUIRE(g.epi == kEpiNone, "gemm: epilogue needs 16-byte aligned rows with K %% 16 == 0");
        return gemm_strided(g.b_trans ? FMLH_TRANSPOSE_RIGHT : FMLH_TRANSPOSE_NONE, g.C, g.A, g.B,
                            g.M, g.N, g.K, g.lda, 1, g.ldb, 1, g.ldc, 1, 1, 0, 0, 0, g.s);
    }
    GemmPlan p = plan_gemm(g.M, g.N, g.K, g.b_trans);
    if (p.ws_elems > ws_elems) {
        if (ws != nullptr) return set_error(FMLH_E_INVALID, "gemm: workspace too small");
        FMLH_TRY(global_workspace(p.ws_elems, &ws));
    }
    switch (p.kind) {
        case GemmPlan::kSkinnyNT:
            switch (g.epi) {
                case kEpiGelu: return launch_nt<kEpiGelu>(g);
                case kEpiResid: return launch_nt<kEpiResid>(g);
                default: return launch_nt<kEpiNone>(g);
            }
        case GemmPlan::kSkinnyNN: {
            dim3 grid((g.N + 255) / 256, p.splits);
            hipLaunchKernelGGL(skinny_nn_partial_kernel, grid, dim3(64), 0, g.s, g.A, g.lda, g.B,
                               g.ldb, ws, g.M, g.N, g.K);
            FMLH_LAUNCHED("skinny_nn_partial_kernel");
            return reduce_dispatch(g.epi, ws, p.splits, g.C, g.ldc, g.M, g.N, g.R, g.ldr, g.s);
        }
        case GemmPlan::kMfmaNT:
            if (p.splits > 1 && g.epi != kEpiKV && p.bm == 64 && p.bn == 64) return launch_nt_split_tiles(g, p, ws);
            if (p.bm == 128 && p.bn == 128) return nt_epi<128, 128>(g);
            if (p.bm == 128) return nt_epi<128, 64>(g);
            return nt_epi<64, 64>(g);
        default:
            if (nt_split_applies(g, p)) {
                FMLH_TRY(launch_nt_split(g, p, ws));
                return reduce_dispatch(g.epi, ws, p.splits, g.C, g.ldc, g.M, g.N, g.R, g.ldr, g.s);
            }
            if (p.bm == 128) return mfma_tile<128, 128>(g, p.splits, p.k_per_split, ws);
            return mfma_tile<64, 64>(g, p.splits, p.k_per_split, ws);
    }
}

int gemm_nt_partials(const GemmArgs& g, int splits, float* ws, size_t ws_elems) {
    const bool vec_ok = aligned16(g.A) && aligned16(g.B) && g.lda % 4 == 0 && g.ldb % 4 == 0;
    FMLH_REQUIRE(g.b_trans && vec_ok && splits >= 1 && g.K % (splits * KB) == 0,
                 "gemm_nt_partials: %dx%dx%d in %d splits needs B stored N x K, 16-byte rows, K %% (16 splits) == 0",
                 g.M, g.N, g.K, splits);
    FMLH_REQUIRE(ws != nullptr && (size_t)splits * g.M * g.N <= ws_elems, "gemm_nt_partials: workspace too small");
    if (g.M == 0 || g.N == 0) return FMLH_OK;
    launch_nt_partials(g, splits, g.K / splits, ws);
    FMLH_LAUNCHED("gemm_nt_kernel(partials)");
    return FMLH_OK;
}

int gemm_split_partials(const GemmArgs& g, float* ws, size_t ws_elems, int* splits) {
    *splits = 0;
    const bool vec_ok = aligned16(g.A) && aligned16(g.B) && g.lda % 4 == 0 && g.ldb % 4 == 0 &&
                        g.K % KB == 0;
    if (g.M == 0 || g.N == 0 || !vec_ok) return FMLH_OK;
    const GemmPlan p = plan_gemm(g.M, g.N, g.K, g.b_trans);
    if (p.kind != GemmPlan::kMfma || p.splits < 2) return FMLH_OK;
    FMLH_REQUIRE(ws != nullptr && p.ws_elems <= ws_elems, "gemm_split_partials: workspace too small");
    if (nt_split_applies(g, p)) {
        *splits = p.splits;
        return launch_nt_split(g, p, ws);
    }
    dim3 grid((g.N + p.bn - 1) / p.bn, (g.M + p.bm - 1) / p.bm, p.splits);
#define FMLH_PARTIALS(BMV, BTV)                                                                  \
    hipLaunchKernelGGL((gemm_mfma_kernel<BMV, BMV, BTV, kEpiNone, true>), grid, dim3(256), 0, g.s, \
                       g.A, g.lda, g.B, g.ldb, g.C, g.ldc, g.M, g.N, g.K, nullptr, 0, ws, p.k_per_split)
    if (p.bm == 128) {
        if (g.b_trans) FMLH_PARTIALS(128, true); else FMLH_PARTIALS(128, false);
    } else {
        if (g.b_trans) FMLH_PARTIALS(64, true); else FMLH_PARTIALS(64, false);
    }
#undef FMLH_PARTIALS
    FMLH_LAUNCHED("gemm_mfma_kernel(split partials)");
    *splits = p.splits;
    return FMLH_OK;
}

int gemm_strided(int mode, float* out, const float* L, const float* R, uint32_t M, uint32_t N,
                 uint32_t K, uint32_t l_rs, uint32_t l_cs, uint32_t r_rs, uint32_t r_cs,
                 uint32_t o_rs, uint32_t o_cs, uint32_t batch, size_t l_plane, size_t r_plane,
                 size_t o_plane, hipStream_t s) {
    if (M == 0 || N == 0 || batch == 0) return FMLH_OK;
    const bool tl = mode == FMLH_TRANSPOSE_LEFT || mode == FMLH_TRANSPOSE_BOTH;
    const bool tr = mode == FMLH_TRANSPOSE_RIGHT || mode == FMLH_TRANSPOSE_BOTH;
    // K within one 64-wide chunk: one chunk per 32 x 32 tile.  Longer K: the wave-split
    // kernel, with 16 x 16 tiles unless 32 x 32 tiles already give a work-group per CU.
    const size_t tiles32 = (size_t)((N + 31) / 32) * ((M + 31) / 32) * batch;
    const int kind = K <= kStKC || std::getenv("FMLH_STRIDED_NO_WSPLIT") ? 0 : (tiles32 >= (size_t)cu_count() ? 32 : 16);
    const uint32_t tt = kind == 16 ? 16u : 32u;
    dim3 grid((N + tt - 1) / tt, (M + tt - 1) / tt, batch);
#define FMLH_STRIDED(TLV, TRV)                                                                             \
    do {                                                                                                    \
        if (kind == 16)                                                                                     \
            hipLaunchKernelGGL((gemm_strided_wsplit_kernel<TLV, TRV, 16>), grid, dim3(256), 0, s, out, L, R,  \
                               M, N, K, l_rs, l_cs, r_rs, r_cs, o_rs, o_cs, l_plane, r_plane, o_plane);       \
        else if (kind == 32)                                                                                \
            hipLaunchKernelGGL((gemm_strided_wsplit_kernel<TLV, TRV, 32>), grid, dim3(256), 0, s, out, L, R,  \
                               M, N, K, l_rs, l_cs, r_rs, r_cs, o_rs, o_cs, l_plane, r_plane, o_plane);       \
        else                                                                                                \
            hipLaunchKernelGGL((gemm_strided_kernel<TLV, TRV>), grid, dim3(256), 0, s, out, L, R, M, N, K,    \
                               l_rs, l_cs, r_rs, r_cs, o_rs, o_cs, l_plane, r_plane, o_plane);               \
    } while (0)
    if (tl && tr) FMLH_STRIDED(true, true);
    else if (tl) FMLH_STRIDED(true, false);
    else if (tr) FMLH_STRIDED(false, true);
    else FMLH_STRIDED(false, false);
#undef FMLH_STRIDED
    FMLH_LAUNCHED("gemm_strided_kernel");
    return FMLH_OK;
}

}  // namespace fmlh

using namespace fmlh;

extern "C" {

int fmlh_mul(int mode, float* out, const float* L, const float* R, uint32_t M, uint32_t N,
             uint32_t K) {
    FMLH_REQUIRE(out && L && R, "fmlh_mul: null pointer");
    FMLH_REQUIRE(mode >= 0 && mode <= 3, "fmlh_mul: bad transpose mode %d", mode);
    FMLH_TRY(ensure_init());
    if (mode == FMLH_TRANSPOSE_NONE || mode == FMLH_TRANSPOSE_RIGHT) {
        GemmArgs g;
        g.A = L; g.lda = (int)K;
        g.B = R; g.ldb = (int)(mode == FMLH_TRANSPOSE_RIGHT ? K : N);
        g.b_trans = mode == FMLH_TRANSPOSE_RIGHT;
        g.C = out; g.ldc = (int)N;
        g.M = (int)M; g.N = (int)N; g.K = (int)K;
        g.s = stream();
        return gemm(g, nullptr, 0);
    }
    const bool tl = true;
    const bool tr = mode == FMLH_TRANSPOSE_BOTH;
    return gemm_strided(mode, out, L, R, M, N, K, tl ? M : K, 1, tr ? K : N, 1, N, 1, 1, 0, 0, 0,
                        stream());
}

int fmlh_gemm_ex(const float* A, int lda, const float* B, int ldb, int b_trans, float* C, int ldc,
                 int M, int N, int K, int epilogue, const float* R, int ldr) {
    FMLH_REQUIRE(A && B && C, "fmlh_gemm_ex: null pointer");
    FMLH_REQUIRE(M >= 0 && N >= 0 && K >= 0, "fmlh_gemm_ex: negative size");
    FMLH_REQUIRE(epilogue >= kEpiNone && epilogue <= kEpiResid, "fmlh_gemm_ex: bad epilogue %d",
                 epilogue);
    FMLH_REQUIRE(epilogue != kEpiResid || R != nullptr, "fmlh_gemm_ex: residual needs R");
    FMLH_REQUIRE(lda >= K && ldc >= N && ldb >= (b_trans ? K : N), "fmlh_gemm_ex: bad leading dim");
    FMLH_TRY(ensure_init());
    GemmArgs g;
    g.A = A; g.lda = lda; g.B = B; g.ldb = ldb; g.b_trans = b_trans ? 1 : 0;
    g.C = C; g.ldc = ldc; g.M = M; g.N = N; g.K = K; g.epi = epilogue; g.R = R; g.ldr = ldr;
    g.s = stream();
    return gemm(g, nullptr, 0);
}

int fmlh_gemm_ex_noalloc(const float* A, int lda, const float* B, int ldb, int b_trans, float* C, int ldc,
                         int M, int N, int K, int epilogue, const float* R, int ldr) {
    FMLH_REQUIRE(A && B && C, "fmlh_gemm_ex_noalloc: null pointer");
    FMLH_REQUIRE(M >= 0 && N >= 0 && K >= 0, "fmlh_gemm_ex_noalloc: negative size");
    FMLH_REQUIRE(epilogue >= kEpiNone && epilogue <= kEpiResid, "fmlh_gemm_ex_noalloc: bad epilogue %d",
                 epilogue);
    FMLH_REQUIRE(epilogue != kEpiResid || R != nullptr, "fmlh_gemm_ex_noalloc: residual needs R");
    FMLH_REQUIRE(lda >= K && ldc >= N && ldb >= (b_trans ? K : N), "fmlh_gemm_ex_noalloc: bad leading dim");
    // No lazy initialisation here (it would create the library stream): fmlh_init set up the
    // scratch address of this device.
    float* ws = noalloc_scratch();
    if (ws == nullptr)
        return set_error(FMLH_E_STATE, "fmlh_gemm_ex_noalloc: call fmlh_init first (it sets up the scratch)");
    GemmArgs g;
    g.A = A; g.lda = lda; g.B = B; g.ldb = ldb; g.b_trans = b_trans ? 1 : 0;
    g.C = C; g.ldc = ldc; g.M = M; g.N = N; g.K = K; g.epi = epilogue; g.R = R; g.ldr = ldr;
    g.s = stream();
    const size_t need = gemm_workspace_elems(g);
    if (need > kNoAllocScratchFloats)
        return set_error(FMLH_E_INVALID,
                         "fmlh_gemm_ex_noalloc: %dx%dx%d needs %zu floats of split-K partials; the fixed "
                         "scratch holds %zu (use fmlh_gemm_ex)", M, N, K, need, kNoAllocScratchFloats);
    return gemm(g, ws, kNoAllocScratchFloats);
}

int fmlh_matmul_strided(int mode, float* out, const float* L, const float* R, uint32_t M,
                        uint32_t N, uint32_t K, uint32_t l_rs, uint32_t l_cs, uint32_t r_rs,
                        uint32_t r_cs, uint32_t o_rs, uint32_t o_cs, uint32_t batch,
                        size_t l_plane, size_t r_plane, size_t o_plane) {
    FMLH_REQUIRE(out && L && R, "fmlh_matmul_strided: null pointer");
    FMLH_REQUIRE(mode >= 0 && mode <= 3, "fmlh_matmul_strided: bad transpose mode %d", mode);
    FMLH_TRY(ensure_init());
    return gemm_strided(mode, out, L, R, M, N, K, l_rs, l_cs, r_rs, r_cs, o_rs, o_cs, batch,
                        l_plane, r_plane, o_plane, stream());
}

}  // extern "C"

namespace fmlh {

// ---- split-K partials of fmlh_gemm_ex_noalloc ------------------------------------------------
// A fixed device array, one copy per device (each device that loads the library holds it until
// the process ends).  In host code `scratch` names a host-side stand-in, not device memory: the
// device address comes from hipGetSymbolAddress, once per device, at fmlh_init.

static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};
int g_scratch_device = -1;  // the device the library runs on (fmlh_init)
}  // namespace

int setup_noalloc_scratch(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0 || device >= kMaxDevices)
        return set_error(FMLH_E_INVALID, "device %d beyond the %d the scratch table holds", device, kMaxDevices);
    if (g_scratch_ptr[device] == nullptr) {
        void* p = nullptr;
        FMLH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        g_scratch_ptr[device] = static_cast<float*>(p);
    }
    g_scratch_device = device;
    return FMLH_OK;
}

float* noalloc_scratch() {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (stream() == nullptr || g_scratch_device < 0) return nullptr;  // not initialised
    return g_scratch_ptr[g_scratch_device];
}

void release_global_workspace() {
    std::lock_guard<std::mutex> lock(g_ws_mu);
    if (g_ws) (void)hipFree(g_ws);
    g_ws = nullptr;
    g_ws_elems = 0;
}

}  // namespace fmlh
