// Host side of the persistent decode kernel (decode_persistent_kernel.h): shape planning,
// dispatch to the per-head-dimension launchers, and the weight transposes it reads.
#include "decode_persistent.h"

#include <algorithm>
#include <cstdlib>

namespace fmlh {
namespace {

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

long ceil_div(long a, long b) { return (a + b - 1) / b; }
long round_up(long a, long b) { return ceil_div(a, b) * b; }

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
    if (B < 1 || B > kMaxPersistBatch * kMaxPersistGroups || L < 1 || V < 1 || hd * H != C) return p;
    if (hd != 16 && hd != 32 && hd != 64) return p;
    if (C > 512 || T > 1024) return p;  // rows of 1-2 LDS chunks; key chunks staged in LDS
    // Sequences in groups of at most kMaxPersistBatch, balanced; each group gets an equal share
    // of the CUs (one WG per CU).  G <= C keeps every all-to-all hop publishing from every WG.
    p.groups = (int)ceil_div(B, kMaxPersistBatch);
    p.Bg = (int)ceil_div(B, p.groups);
    const int cus_per_group = cus / p.groups;
    int G = std::min({C, cus_per_group, kMaxPersistG});  // more WGs: smaller slices (measured faster)
    if (const char* env = std::getenv("FMLH_PERSIST_G")) {
        const int g = std::atoi(env);
        if (g > 0) G = g;
    }
    G = std::min({G, C, cus_per_group, kMaxPersistG / p.groups});
    if (G < 1) return p;
    p.G = G;
    const int Bg = p.Bg;
    p.bt = Bg <= 1 ? 1 : Bg <= 2 ? 2 : Bg <= 4 ? 4 : 8;
    p.nqc = (int)ceil_div(C, 256);
    const long cp = 256L * p.nqc;
    p.h4p = (int)round_up(4L * C, 512);
    const long r3 = ceil_div(3L * C, G), r1 = ceil_div(C, G), r4 = ceil_div(4L * C, G), rv = ceil_div(V, G);
    p.wcap = (int)round_up(std::max({r3 * cp, r1 * cp, r4 * cp, r1 * p.h4p, rv * cp}), 64);
    p.max_chunks = (int)ceil_div(T, kPersistItemKeys);
    const long part = (long)p.max_chunks * p.bt * H * (hd + 2);
    const long kv = 2L * kPersistItemKeys * hd;
    const long fixed = 2L * p.wcap + 2L * p.bt * cp + 4L * 512 + 4L * (hd + 2) + 4;
    // K/V rows either share U with the other per-hop data or (FMLH_PERSIST_KV_AHEAD=1) get a
    // region of their own and are fetched a layer ahead.  Measured on MI355X (c2, bs1): the
    // early fetch is ~2 us/token slower -- the hop-1 polls complete in order behind it.
    const long u_sep = round_up(std::max({(long)p.bt * p.h4p, part, rv * p.bt}), 64);
    const long u_shared = round_up(std::max(u_sep, kv), 64);
    const char* ahead = std::getenv("FMLH_PERSIST_KV_AHEAD");
    if (ahead && ahead[0] == '1' && (size_t)(fixed + u_sep + kv) * sizeof(float) <= smem_limit()) {
        p.kv_sep = true;
        p.ufloats = (int)u_sep;
        p.smem = (size_t)(fixed + u_sep + kv) * sizeof(float);
    } else {
        p.ufloats = (int)u_shared;
        p.smem = (size_t)(fixed + u_shared) * sizeof(float);
    }
    if (p.smem > smem_limit()) return PersistPlan{};
    p.ok = true;
    return p;
}

void persist_group_words(int C, int H, int hd, int max_chunks, int G_max, int Bg_max, size_t out[5]) {
    const size_t Bg = Bg_max;
    out[0] = Bg * C;                                   // q, k_new, v_new (each)
    out[1] = (size_t)max_chunks * Bg * H * (hd + 2);   // attention partials
    out[2] = Bg * C;                                   // dx1, dx2 (each)
    out[3] = Bg * 4 * C;                               // h
    out[4] = (size_t)G_max * Bg * 2;                   // argmax candidates
}

int persist_decode(const PersistArgs& a, const PersistPlan& p, int hd, hipStream_t s) {
    if (!p.ok) return set_error(FMLH_E_INVALID, "persistent decode not planned for this shape");
    if (hd == 64) return persist_launch_hd64(a, p, s);
    if (hd == 32) return persist_launch_hd32(a, p, s);
    if (hd == 16) return persist_launch_hd16(a, p, s);
    return set_error(FMLH_E_INVALID, "persistent decode: head_dim %d unsupported", hd);
}

}  // namespace fmlh
