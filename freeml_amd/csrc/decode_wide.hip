// Wide decode kernel (interface and protocol: decode_wide.h).
//
// Layout of one workgroup (256 threads, 4 waves), per launch:
//   LDS  xs[8][C]  the residual stream of every sequence (rows >= B stay 0)
//        xn[8][C]  the LayerNorm of xs for the next product, or the gathered y rows
//        lnp[4][C] the layer's LayerNorm gains and biases (LN0 g, b, LN1 g, b; ln_f g, b
//                  for the lm_head), copied by LDS DMA with the layer's first weight loads, so
//                  a LayerNorm after a hand-off needs no memory round trip
//        and small scratch for the attention item, the slice merge and the reductions.
//   Products: a WG owns a contiguous, balanced block of R rows of each weight (R = N / G
//   rounded: c4 9 QKV, 3 projection, 12 FC rows); wave v takes local rows v, v + 4, ..., and
//   lane l holds float4 chunks l + 64 m (m < C / 256) of each of its rows, so a row's loads
//   are 1 KB contiguous per wave instruction.  Every lane forms the partial dot products of
//   its rows with all 8 activation rows, and one butterfly reduction (reduce_many) over the
//   wave turns the 32 per-lane partials into 32 row x sequence totals, one per lane pair.
//   Weights are requested from HBM (bounds-checked buffer loads) one hand-off before their
//   product, so they arrive while the WG waits.
//
// Parity: fp32 throughout; products and reductions sum in other orders than the reference's
// sequential k (a few ulp); the attention normalises after P.V; every sum is taken in a fixed
// order, so a launch is deterministic.
#include "decode_wide.h"

#include <algorithm>
#include <cmath>

namespace fmlh {
namespace wide {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxB = kWideMaxBatch;
constexpr int kHD = kWideHD;
constexpr int kMaxParts = 64;                     // attention items (key slices) per pair
constexpr int kTeam = 8;                          // WGs sharing their FC columns in the MLP projection
constexpr int kTeams = 256 / kTeam;
constexpr int kKeyBatch = 8;                      // keys per 16-lane group per load round
constexpr int kMaxLmRows = 256;                   // lm_head rows per WG
constexpr int kLmRowsPerWave = 4;                 // lm_head rows per wave per load round
constexpr int kLmMinRows = 8;                     // small vocabularies: rows per lm_head WG at least
constexpr long kSpinLimit = 1L << 21;             // polls of ~1 us: a few seconds at most
constexpr int kRawBufferFlags = 0x00020000;       // raw buffer: loads past num_records read 0
constexpr int kAuxSc1 = 0x10;                     // sc1: served beyond the per-XCD L2 for clean lines

typedef float floatx4 __attribute__((ext_vector_type(4)));

// The thread index through an empty asm at each use: otherwise the compiler computes every
// per-lane address of the step loop (64-bit pointers of every gathered word) once before the
// loop and keeps them all live, which exhausts the registers and spills to scratch.
__device__ __forceinline__ int thread_id() {
    int t = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(t));
    return t;
}
__device__ __forceinline__ int lane_id() { return thread_id() & 63; }
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(thread_id() >> 6); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const float* base, size_t floats) {
    const size_t bytes = floats * sizeof(float);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0,
                                             static_cast<int>(bytes > 0x7fffffffu ? 0x7fffffffu : bytes),
                                             kRawBufferFlags);
}
template <int AUX = 0>
__device__ __forceinline__ floatx4 ld4(__amdgpu_buffer_rsrc_t r, size_t float_index) {
    return __builtin_bit_cast(floatx4,
                              __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(float_index * 4), 0, AUX));
}
__device__ __forceinline__ float ld1(__amdgpu_buffer_rsrc_t r, size_t float_index) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(float_index * 4), 0, 0));
}
__device__ __forceinline__ float dot4(floatx4 a, floatx4 b) { return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w; }

// ---- exchange words ------------------------------------------------------------------------

__device__ __forceinline__ uint64_t xload(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void xput(uint64_t* p, float v, uint32_t ep) {
    __hip_atomic_store(p, (static_cast<uint64_t>(ep) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void xput_bits(uint64_t* p, uint32_t bits, uint32_t ep) {
    __hip_atomic_store(p, (static_cast<uint64_t>(ep) << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool current(uint64_t v, uint32_t ep) { return static_cast<uint32_t>(v >> 32) == ep; }
__device__ __forceinline__ float payload(uint64_t v) { return __uint_as_float(static_cast<uint32_t>(v)); }

struct Shared {
    int bail;        // this WG gave up waiting (a timeout here or in another wave)
    int token[kMaxB];
};

// Polls the words addr(k) (nullptr: none) until all are current: the first loads of all of
// them go out together, then only stale ones are loaded again, together.  Wave-uniform exit
// (a ballot; a per-lane exit let the compiler reuse registers of words other lanes still
// wait for), bounded: past kSpinLimit polls the WG records the timeout and stops waiting for
// the rest of the launch.  Addresses are recomputed rather than held (registers).
template <int N, class Addr>
__device__ __forceinline__ void poll_words(uint64_t (&v)[N], uint32_t ep, Shared* sh, unsigned* err, Addr addr) {
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const uint64_t* p = addr(k);
        v[k] = p != nullptr ? xload(p) : (static_cast<uint64_t>(ep) << 32);
    }
    int it = 0;
    while (true) {
        bool stale = false;
#pragma unroll
        for (int k = 0; k < N; ++k) stale |= !current(v[k], ep);
        if (__builtin_amdgcn_ballot_w64(stale) == 0) return;
        if ((++it & 255) == 0) {
            if (__hip_atomic_load(&sh->bail, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) return;
            if (it > kSpinLimit) {
                __hip_atomic_store(&sh->bail, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                atomicOr(err, 1u);
                return;
            }
        }
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const bool need = !current(v[k], ep);
            uint64_t nv = v[k];
            if (need) nv = xload(addr(k));
            v[k] = need ? nv : v[k];
        }
    }
}

// poll_words after waiting for one proxy word of the same producer (nullptr: none).
template <int N, class Addr>
__device__ __forceinline__ void poll_words_after(const uint64_t* proxy, uint64_t (&v)[N], uint32_t ep, Shared* sh,
                                                 unsigned* err, Addr addr) {
    uint64_t pv[1];
    poll_words(pv, ep, sh, err, [&](int) { return proxy; });
    poll_words(v, ep, sh, err, addr);
}

// n words (n <= MAXW * 256), word i at where(i), taken by thread i % 256: fn(i, value).
template <int MAXW, class Where, class Fn>
__device__ __forceinline__ void gather_at(int n, uint32_t ep, Shared* sh, unsigned* err, Where where, Fn fn) {
    const int t = thread_id();
    uint64_t v[MAXW];
    poll_words(v, ep, sh, err, [&](int k) -> const uint64_t* {
        const int i = t + k * kThreads;
        return i < n ? where(i) : nullptr;
    });
#pragma unroll
    for (int k = 0; k < MAXW; ++k)
        if (t + k * kThreads < n) fn(t + k * kThreads, payload(v[k]));
}
// Words src[0 .. n).
template <int MAXW, class Fn>
__device__ __forceinline__ void gather(const uint64_t* src, int n, uint32_t ep, Shared* sh, unsigned* err, Fn fn) {
    gather_at<MAXW>(n, ep, sh, err, [&](int i) { return src + i; }, fn);
}

// The same after a proxy round: thread p first waits for one word of producer p (proxy(p), p <
// nprod <= 256), then the WG loads every word once.  While producers are still working, a
// waiting WG then polls nprod words instead of all n (a 256-WG gather of B C words re-polled
// whole ~1.5M loads per round, which slowed the producers still streaming their weights).  A
// word that is still stale when loaded (a producer's other stores can land after its proxy)
// is polled again as before.
template <int MAXW, class Proxy, class Where, class Fn>
__device__ __forceinline__ void gather_after(int nprod, Proxy proxy, int n, uint32_t ep, Shared* sh, unsigned* err,
                                             Where where, Fn fn) {
    uint64_t pv[1];
    poll_words(pv, ep, sh, err, [&](int) -> const uint64_t* {
        const int p = thread_id();
        return p < nprod ? proxy(p) : nullptr;
    });
    __syncthreads();
    gather_at<MAXW>(n, ep, sh, err, where, fn);
}

// ---- wave reductions -----------------------------------------------------------------------

// Butterfly: N values per lane (N a power of two <= 64) summed over the 64 lanes; afterwards
// every lane holds the total of value lane >> (6 - log2 N) (lanes differing only in their low
// 6 - log2 N bits hold the same total).  N - 1 + (6 - log2 N) shuffles instead of 6 N.
template <int N, int MASK = 32>
__device__ __forceinline__ void fold(float (&v)[N], int lane) {
    if constexpr (N > 1) {
        constexpr int kHalf = N / 2;
        const bool hi = (lane & MASK) != 0;
#pragma unroll
        for (int i = 0; i < kHalf; ++i) {
            const float send = hi ? v[i] : v[i + kHalf];
            const float keep = hi ? v[i + kHalf] : v[i];
            v[i] = keep + __shfl_xor(send, MASK);
        }
        float w[kHalf];
#pragma unroll
        for (int i = 0; i < kHalf; ++i) w[i] = v[i];
        fold<kHalf, MASK / 2>(w, lane);
        v[0] = w[0];
    } else {
#pragma unroll
        for (int m = MASK; m >= 1; m /= 2) v[0] += __shfl_xor(v[0], m);
    }
}
template <int N>
__device__ __forceinline__ float reduce_many(float (&v)[N]) {
    fold<N, 32>(v, lane_id());
    return v[0];
}
template <int N>
constexpr int log2c() {
    if constexpr (N <= 1) return 0;
    else return 1 + log2c<N / 2>();
}

// (value, index) first maximum over the wave: larger value, or the lower index on a tie.
__device__ __forceinline__ void wave_first_max(float& v, int& idx) {
#pragma unroll
    for (int m = 32; m >= 1; m /= 2) {
        const float ov = __shfl_xor(v, m);
        const int oi = __shfl_xor(idx, m);
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
}

// ---- rows ----------------------------------------------------------------------------------

__device__ __forceinline__ int split(int n, int parts, int i) { return static_cast<int>((long)n * i / parts); }

// LayerNorm of rows b < B of src into dst (gamma g, beta bt or none: LDS), two-pass mean / variance
// as the reference (LayerNormOp, MatrixBase_Functions.h:481-549).  Wave v takes rows v, v + 4.
template <int NQ>
__device__ __forceinline__ void layernorm(const float* src, float* dst, const float* g, const float* bt, int B) {
    constexpr int C = 256 * NQ;
    const int lane = lane_id(), wv = wave_id();
    floatx4 gv[NQ], bv[NQ];
#pragma unroll
    for (int m = 0; m < NQ; ++m) {
        gv[m] = reinterpret_cast<const floatx4*>(g)[lane + 64 * m];
        bv[m] = bt ? reinterpret_cast<const floatx4*>(bt)[lane + 64 * m] : floatx4{0.f, 0.f, 0.f, 0.f};
    }
    for (int b = wv; b < B; b += 4) {
        const floatx4* x4 = reinterpret_cast<const floatx4*>(src + b * C);
        floatx4 x[NQ];
        float s = 0.f;
#pragma unroll
        for (int m = 0; m < NQ; ++m) {
            x[m] = x4[lane + 64 * m];
            s += (x[m].x + x[m].y) + (x[m].z + x[m].w);
        }
        const float mean = wave_sum(s) * (1.0f / C);
        float q = 0.f;
#pragma unroll
        for (int m = 0; m < NQ; ++m) {
            const floatx4 d = x[m] - mean;
            q += (d.x * d.x + d.y * d.y) + (d.z * d.z + d.w * d.w);
        }
        const float inv = 1.0f / sqrtf(wave_sum(q) * (1.0f / C) + 1e-5f);
        floatx4* y4 = reinterpret_cast<floatx4*>(dst + b * C);
#pragma unroll
        for (int m = 0; m < NQ; ++m) y4[lane + 64 * m] = (x[m] - mean) * inv * gv[m] + bv[m];
    }
}

constexpr int pow2_at_least(int n) { return n <= 1 ? 1 : 2 * pow2_at_least((n + 1) / 2); }

// Weight rows r0 + v + 4 j (j < RPW, local row < R) of a row-major N x C matrix, for wave v.
template <int NQ, int RPW>
__device__ __forceinline__ void load_rows(floatx4 (&w)[RPW][NQ], const float* W, int N, int r0, int R) {
    constexpr int C = 256 * NQ;
    const auto r = rsrc(W, (size_t)N * C);
    const int lane = lane_id(), wv = wave_id();
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        const int i = wv + 4 * j;
#pragma unroll
        for (int m = 0; m < NQ; ++m)
            w[j][m] = i < R ? ld4(r, (size_t)(r0 + i) * C + 4 * (lane + 64 * m)) : floatx4{0.f, 0.f, 0.f, 0.f};
    }
}

// The vectors src[k][0 .. C) (k < NV; a null src[k] is skipped) into dst[k C ..) by LDS DMA:
// 1 KB per wave instruction, chunks spread over the 4 waves.  Complete once a later load of
// the issuing wave has returned (vector memory returns in order) and, for other waves'
// chunks, after a barrier.
template <int NQ, int NV>
__device__ __forceinline__ void stage_vectors(float* dst, const float* const (&src)[NV]) {
    constexpr int C = 256 * NQ;
    const int lane = lane_id(), wv = wave_id();
    for (int c = wv; c < NV * NQ; c += 4) {
        const int k = c / NQ, off = (c % NQ) * 256;
        if (src[k] != nullptr) copy16_to_lds(dst + k * C + off, src[k] + off + 4 * lane);
    }
}

// out(j, b) = row (v + 4 j) . act[b] for the wave's rows and the BT rows of act (LDS, stride C):
// per-lane partials over the lane's chunks, then one butterfly over the wave.  fn(local_row,
// b, value) runs in one lane per (row, sequence) with local_row < R and b < B.
template <int NQ, int BT, int RPW, class Fn>
__device__ __forceinline__ void product(const floatx4 (&w)[RPW][NQ], const float* act, int R, int B, Fn fn) {
    constexpr int C = 256 * NQ;
    constexpr int N = pow2_at_least(RPW * BT);
    constexpr int kShift = 6 - log2c<N>();
    const int lane = lane_id(), wv = wave_id();
    float v[N];
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = 0.f;
#pragma unroll
    for (int b = 0; b < BT; ++b) {
        const floatx4* a4 = reinterpret_cast<const floatx4*>(act + b * C);
#pragma unroll
        for (int m = 0; m < NQ; ++m) {
            const floatx4 a = a4[lane + 64 * m];
#pragma unroll
            for (int j = 0; j < RPW; ++j) v[j * BT + b] += dot4(w[j][m], a);
        }
    }
    const float tot = reduce_many(v);
    const int k = lane >> kShift, j = k / BT, b = k % BT;
    const int i = wv + 4 * j;
    if ((lane & ((1 << kShift) - 1)) == 0 && j < RPW && i < R && b < B) fn(i, b, tot);
}

__device__ __forceinline__ float gelu(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

template <int NQ>
struct Lds {
    static constexpr int C = 256 * NQ;
    float* xs;     // [8][C]
    float* xn;     // [8][C]
    float* lnp;    // [4][C] LayerNorm gains and biases
    float* qkv;    // [3][64] the item's q, k_new, v_new
    float* gm;     // [16] per-group max
    float* gl;     // [16] per-group sum
    float* go;     // [16][64] per-group P.V
    float* part;   // [kMaxParts][66] attention records of a pair
    float* lg;     // [8][kMaxLmRows] this WG's logits
    Shared* sh;
    __device__ explicit Lds(float* base) {
        xs = base;
        xn = xs + kMaxB * C;
        lnp = xn + kMaxB * C;
        qkv = lnp + 4 * C;
        gm = qkv + 3 * kHD;
        gl = gm + 16;
        go = gl + 16;
        part = go + 16 * kHD;
        lg = part + kMaxParts * (kHD + 2);
        sh = reinterpret_cast<Shared*>(lg + kMaxB * kMaxLmRows);
    }
    static constexpr size_t floats() {
        return 2 * kMaxB * C + 4 * C + 3 * kHD + 32 + 16 * kHD + kMaxParts * (kHD + 2) + kMaxB * kMaxLmRows +
               (sizeof(Shared) + 3) / 4;
    }
};

__device__ __forceinline__ uint32_t epoch_of(const WideArgs& a, int step, int layer, int hop) {
    return a.epoch_base + static_cast<uint32_t>(step) * (kWideHops * a.L + 1u) + kWideHops * layer + hop + 1u;
}

// xs[b] = tok[token[b]] + pos_emb[pos] for b < B.
template <int NQ>
__device__ __forceinline__ void embed(const WideArgs& a, const Lds<NQ>& s, int pos) {
    constexpr int C = 256 * NQ;
    const auto rt = rsrc(a.tok, (size_t)a.V * C);
    const auto rp = rsrc(a.pos_emb, (size_t)a.T * C);
    for (int e = thread_id(); e < a.B * C / 4; e += kThreads) {
        const int b = e / (C / 4), c4 = e % (C / 4);
        const floatx4 t = ld4(rt, (size_t)s.sh->token[b] * C + 4 * c4);
        const floatx4 p = ld4(rp, (size_t)pos * C + 4 * c4);
        reinterpret_cast<floatx4*>(s.xs)[e] = t + p;
    }
}


// ---- H2: attention items ----------------------------------------------------------------

// Pair p = (sequence, head) has S items, keys 0 .. pos split into S near-equal slices
// [split(n, S, sl), split(n, S, sl + 1)) (n = pos + 1); item (p, sl) runs on WG p + P sl and
// leaves its (max, sum, P.V) at record p + P sl (an empty slice leaves max -inf, sum 0).
// A flat split of all pairs' keys over every WG measured slower: the WGs whose share spans two
// pairs run two items back to back and the merge waits for them.

// Keys [k0, k1) of pair p (k1 == n: the last of them is key pos, taken from the k_new / v_new
// words and written to the caches here).  Each of the 16 groups of 16 lanes scores keys
// k0 + g, k0 + g + 16, ... (lane j holds dims 4 j .. +3), kKeyBatch keys per load round with
// an online max / sum per group, the next round's rows requested before this round's scores;
// the groups meet in LDS and the partial goes out as hd + 2 words at record `rec`.  The cached
// rows are requested before the item waits for q.
template <int NQ>
__device__ __forceinline__ void attention_item(const WideArgs& a, const Lds<NQ>& s, int l, int step, int pos, int p,
                                               int k0, int k1, int rec) {
    constexpr int C = 256 * NQ;
    const int t = thread_id();
    const int g = t >> 4, j = t & 15;
    const int b = p / a.H, h = p % a.H;
    const bool last = k1 == pos + 1;
    const int kend = last ? k1 - 1 : k1;  // cached keys [k0, kend)
    const size_t slab = (((size_t)l * a.Bmax + b) * a.H + h) * (size_t)a.T * kHD;
    // Rows from kend on read as 0 (num_records), so the loads need no condition.
    const auto rk = rsrc(a.kc + slab, (size_t)kend * kHD);
    const auto rv = rsrc(a.vc + slab, (size_t)kend * kHD);
    floatx4 kb[kKeyBatch], vb[kKeyBatch];
#pragma unroll
    for (int i = 0; i < kKeyBatch; ++i) {
        const size_t key = (size_t)(k0 + g + 16 * i);
        kb[i] = ld4<kAuxSc1>(rk, key * kHD + 4 * j);
        vb[i] = ld4<kAuxSc1>(rv, key * kHD + 4 * j);
    }
    // q (and, for the item holding key pos, k_new and v_new): words part * C + h hd + d of row b.
    const uint64_t* row = a.wq + (size_t)b * 3 * C + h * kHD;
    gather_at<1>(last ? 3 * kHD : kHD, epoch_of(a, step, l, 0), s.sh, a.err,
                 [&](int i) { return row + (size_t)(i / kHD) * C + i % kHD; },
                 [&](int i, float v) { s.qkv[i] = v; });
    __syncthreads();
    if (last && t < 2 * kHD) {  // the step's own key and value into the caches (agent scope)
        float* dst = (t < kHD ? a.kc : a.vc) + slab + (size_t)pos * kHD + t % kHD;
        __hip_atomic_store(dst, s.qkv[kHD + t], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const floatx4 q = reinterpret_cast<const floatx4*>(s.qkv)[j];
    float m = -INFINITY, lsum = 0.f;
    floatx4 o = {0.f, 0.f, 0.f, 0.f};
    for (int base = k0; base < kend; base += 16 * kKeyBatch) {
        floatx4 kc[kKeyBatch], vc[kKeyBatch];
#pragma unroll
        for (int i = 0; i < kKeyBatch; ++i) {
            kc[i] = kb[i];
            vc[i] = vb[i];
        }
        const int nb = base + 16 * kKeyBatch;
        if (nb < kend) {  // the next round's rows (WG-uniform bound: every lane loads)
#pragma unroll
            for (int i = 0; i < kKeyBatch; ++i) {
                const size_t key = (size_t)(nb + g + 16 * i);
                kb[i] = ld4<kAuxSc1>(rk, key * kHD + 4 * j);
                vb[i] = ld4<kAuxSc1>(rv, key * kHD + 4 * j);
            }
        }
        float sc[kKeyBatch];
#pragma unroll
        for (int i = 0; i < kKeyBatch; ++i) {
            float d = dot4(q, kc[i]);
            d += __shfl_xor(d, 8);
            d += __shfl_xor(d, 4);
            d += __shfl_xor(d, 2);
            d += __shfl_xor(d, 1);
            sc[i] = base + g + 16 * i < kend ? d * a.scale : -INFINITY;
        }
        float mb = m;
#pragma unroll
        for (int i = 0; i < kKeyBatch; ++i) mb = fmaxf(mb, sc[i]);
        if (mb != -INFINITY) {
            const float corr = __expf(m - mb);  // m = -inf: 0
            lsum *= corr;
            o *= corr;
#pragma unroll
            for (int i = 0; i < kKeyBatch; ++i) {
                const float e = __expf(sc[i] - mb);  // masked keys: exp(-inf) = 0
                lsum += e;
                o += e * vc[i];
            }
            m = mb;
        }
    }
    if (last && g == 0) {  // key pos, by group 0
        const floatx4 kn = reinterpret_cast<const floatx4*>(s.qkv + kHD)[j];
        const floatx4 vn = reinterpret_cast<const floatx4*>(s.qkv + 2 * kHD)[j];
        float d = dot4(q, kn);
        d += __shfl_xor(d, 8);
        d += __shfl_xor(d, 4);
        d += __shfl_xor(d, 2);
        d += __shfl_xor(d, 1);
        d *= a.scale;
        const float mb = fmaxf(m, d);
        const float corr = __expf(m - mb), e = __expf(d - mb);
        lsum = lsum * corr + e;
        o = o * corr + e * vn;
        m = mb;
    }
    if (j == 0) {
        s.gm[g] = m;
        s.gl[g] = lsum;
    }
    reinterpret_cast<floatx4*>(s.go)[g * 16 + j] = o;
    // Every wave's cache stores have completed (vmcnt) before the barrier, so they are visible
    // at agent scope before the partial goes out; then the groups merge in group order.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t < kHD) {
        float M = -INFINITY;
        for (int k = 0; k < 16; ++k) M = fmaxf(M, s.gm[k]);
        float L = 0.f, O = 0.f;
        if (M != -INFINITY) {
            for (int k = 0; k < 16; ++k) {
                if (s.gl[k] == 0.f) continue;
                const float w = __expf(s.gm[k] - M);
                L += w * s.gl[k];
                O += w * s.go[k * kHD + t];
            }
        }
        const uint32_t ep = epoch_of(a, step, l, 1);
        uint64_t* dst = a.wpart + (size_t)rec * (kHD + 2);
        xput(dst + 2 + t, O, ep);
        if (t == 0) {
            xput(dst, M, ep);
            xput(dst + 1, L, ep);
        }
    }
    __syncthreads();  // LDS scratch free for a second item
}

// ---- H3: pair p merges its records (key order) -> y words --------------------------------

template <int NQ>
__device__ __forceinline__ void combine_pair(const WideArgs& a, const Lds<NQ>& s, int l, int step, int pos, int p) {
    constexpr int C = 256 * NQ;
    const int t = thread_id();
    const int P = a.B * a.H, R = a.S, W = kHD + 2;
    (void)pos;
    auto rec_of = [&](int sl) { return p + P * sl; };
    gather_at<(kMaxParts * (kHD + 2) + kThreads - 1) / kThreads>(
        R * W, epoch_of(a, step, l, 1), s.sh, a.err,
        [&](int i) { return a.wpart + (size_t)rec_of(i / W) * W + i % W; },
        [&](int i, float v) { s.part[i] = v; });
    __syncthreads();
    if (t < kHD) {
        float M = -INFINITY;
        for (int k = 0; k < R; ++k)
            if (s.part[k * W + 1] != 0.f) M = fmaxf(M, s.part[k * W]);
        float L = 0.f, O = 0.f;
        for (int k = 0; k < R; ++k) {
            const float lk = s.part[k * W + 1];
            if (lk == 0.f) continue;
            const float w = __expf(s.part[k * W] - M);
            L += w * lk;
            O += w * s.part[k * W + 2 + t];
        }
        const int b = p / a.H, h = p % a.H;
        xput(a.wy + (size_t)b * C + h * kHD + t, O / L, epoch_of(a, step, l, 2));
    }
}

// ---- the kernel ----------------------------------------------------------------------------

// Rows per wave of each product (G = 256, C = 256 NQ): QKV 3C / G = 3 NQ rows, projection
// C / G = NQ rows (at most 4: one per wave), FC 4C / G = 4 NQ rows.
template <int NQ>
struct Rows {
    static constexpr int kQkv = (3 * NQ + 3) / 4, kProj = 1, kFc = NQ;
};

// BT: the batch tile the products, reductions and gathers are unrolled for (B <= BT <= 8).
template <int NQ, int BT>
__global__ __launch_bounds__(kThreads) void decode_wide_kernel(WideArgs a) {
    constexpr int C = 256 * NQ;
    extern __shared__ float lds_base[];
    const Lds<NQ> s(lds_base);
    const int w = static_cast<int>(blockIdx.x), G = a.G, t = thread_id();
    const int lane = lane_id(), wv = wave_id();
    const int B = a.B, L = a.L, P = B * a.H;
    const int q0 = split(3 * C, G, w), R3 = split(3 * C, G, w + 1) - q0;   // QKV rows
    const int j0 = split(C, G, w), R1 = split(C, G, w + 1) - j0;           // projection rows, reduced outputs
    const int f0 = split(4 * C, G, w), R4 = split(4 * C, G, w + 1) - f0;   // FC rows
    // lm_head rows: over GL = min(G, ceil(V / kLmMinRows)) WGs, so that a small vocabulary's token
    // pick gathers GL candidates, not G (c5: 32 WGs of 8 rows; c4: all 256).
    const int GL = min(G, max(1, (a.V + kLmMinRows - 1) / kLmMinRows));
    const int v0 = w < GL ? split(a.V, GL, w) : a.V, RV = w < GL ? split(a.V, GL, w + 1) - v0 : 0;

    auto stamp = [&](int step, int k) {
        if (a.trace && step == a.trace_step && thread_id() == 0)
            a.trace[(size_t)w * kWideTracePoints + k] = wall_clock64();
    };
    for (int e = t; e < 2 * kMaxB * C; e += kThreads) s.xs[e] = 0.f;  // xs, xn
    if (t == 0) s.sh->bail = 0;
    if (t < kMaxB) {
        int tk = 0;
        if (t < B) tk = a.hist[(size_t)t * a.HS + a.pos0];
        s.sh->token[t] = tk < 0 || tk >= a.V ? 0 : tk;  // a corrupt history must not index past the table
    }
    __syncthreads();

    for (int step = 0; step < a.n_steps; ++step) {
        const int pos = a.pos0 + step;
        embed<NQ>(a, s, pos);
        __syncthreads();
        for (int l = 0; l < L; ++l) {
            const WideLayer lw = a.layers[l];
            stamp(step, 12 * l);
            // H1: x += dx2 of the previous layer, LN0, QKV rows -> q / k_new / v_new words.
            floatx4 wq[Rows<NQ>::kQkv][NQ];
            load_rows<NQ>(wq, lw.wqkvT, 3 * C, q0, R3);
            {
                const float* const ln[4] = {lw.ln0g, lw.ln0b, lw.ln1g, lw.ln1b};
                stage_vectors<NQ, 4>(s.lnp, ln);
            }
            if (l > 0)
                gather_after<BT * NQ>(G, [&](int p) { return a.wdx2 + split(C, G, p); }, B * C,
                                         epoch_of(a, step, l - 1, 6), s.sh, a.err, [&](int i) { return a.wdx2 + i; },
                                         [&](int i, float v) { s.xs[i] += v; });
            copies_barrier<0>();
            layernorm<NQ>(s.xs, s.xn, s.lnp, lw.ln0b ? s.lnp + C : nullptr, B);
            __syncthreads();
            stamp(step, 12 * l + 1);
            {
                const uint32_t ep = epoch_of(a, step, l, 0);
                product<NQ, BT>(wq, s.xn, R3, B,
                            [&](int i, int b, float v) { xput(a.wq + (size_t)b * 3 * C + q0 + i, v, ep); });
            }
            // The projection's weights stream in during the attention hops.
            stamp(step, 12 * l + 2);
            floatx4 wp[Rows<NQ>::kProj][NQ];
            load_rows<NQ>(wp, lw.wproj, C, j0, R1);
            // H2, H3: attention items, then the per-pair merge.
            if (w < P * a.S) {
                const int sl = w / P, n = pos + 1;
                attention_item<NQ>(a, s, l, step, pos, w % P, split(n, a.S, sl), split(n, a.S, sl + 1), w);
            }
            stamp(step, 12 * l + 3);
            // The FC rows stream in during the merge and the y hand-off.
            floatx4 wf[Rows<NQ>::kFc][NQ];
            load_rows<NQ>(wf, lw.wfcT, 4 * C, f0, R4);
            if (w < P) combine_pair<NQ>(a, s, l, step, pos, w);
            stamp(step, 12 * l + 4);
            // H4: y rows, projection rows -> dx1 words.
            __syncthreads();
            gather_after<BT * NQ>(P, [&](int p) { return a.wy + (size_t)(p / a.H) * C + (p % a.H) * kHD; }, B * C,
                                     epoch_of(a, step, l, 2), s.sh, a.err, [&](int i) { return a.wy + i; },
                                     [&](int i, float v) { s.xn[i] = v; });
            __syncthreads();
            stamp(step, 12 * l + 5);
            {
                const uint32_t ep = epoch_of(a, step, l, 3);
                product<NQ, BT>(wp, s.xn, R1, B,
                            [&](int i, int b, float v) { xput(a.wdx1 + (size_t)b * C + j0 + i, v, ep); });
            }
            stamp(step, 12 * l + 6);
            // H5: x += dx1, LN1, FC rows + GELU -> h words.  H6: the MLP projection in teams of
            // kTeam WGs: team tm's FC rows are the h columns [tm TJ, (tm + 1) TJ); each member
            // gathers them (an 8-producer hand-off) and forms the partials of its OM outputs over
            // those columns (threads: output ol, column chunk kc, chunks added in order), so a WG
            // publishes B OM partial words instead of B C.  H7: each owner of NQ outputs adds the
            // NT team partials in team order -> dx2 words.
            constexpr int TJ = 32 * NQ, OM = 32 * NQ, KC = kThreads / OM, CH = TJ / KC;
            static_assert(kTeams * TJ == 4 * 256 * NQ && kTeam * OM == 256 * NQ && KC * CH == TJ, "teams");
            const int tm = w / kTeam, mb = w % kTeam;
            float w2r[CH];  // W_proj2 rows tm TJ + kc CH + jj, column mb OM + ol
            {
                const auto r2 = rsrc(lw.w2, (size_t)4 * C * C);
                const int t = thread_id(), ol = t % OM, kc = t / OM;
#pragma unroll
                for (int jj = 0; jj < CH; ++jj)
                    w2r[jj] = kc < KC ? ld1(r2, (size_t)(tm * TJ + kc * CH + jj) * C + mb * OM + ol) : 0.f;
            }
            gather_after<BT * NQ>(G, [&](int p) { return a.wdx1 + split(C, G, p); }, B * C,
                                     epoch_of(a, step, l, 3), s.sh, a.err, [&](int i) { return a.wdx1 + i; },
                                     [&](int i, float v) { s.xs[i] += v; });
            __syncthreads();
            stamp(step, 12 * l + 7);
            layernorm<NQ>(s.xs, s.xn, s.lnp + 2 * C, lw.ln1b ? s.lnp + 3 * C : nullptr, B);
            __syncthreads();
            {
                const uint32_t ep = epoch_of(a, step, l, 4);
                product<NQ, BT>(wf, s.xn, R4, B,
                            [&](int i, int b, float v) { xput(a.wh + (size_t)b * 4 * C + f0 + i, gelu(v), ep); });
            }
            stamp(step, 12 * l + 8);
            float* hl2 = s.part;  // [8][TJ] the team's h columns (the merge records are free now)
            float* pp = s.lg;     // [KC OM][8] column-chunk partials (the logits rows are free now)
            gather_at<(BT * 32 * NQ + kThreads - 1) / kThreads>(
                B * TJ, epoch_of(a, step, l, 4), s.sh, a.err,
                [&](int i) { return a.wh + (size_t)(i / TJ) * 4 * C + tm * TJ + i % TJ; },
                [&](int i, float v) { hl2[i] = v; });
            __syncthreads();
            {
                const int t = thread_id(), ol = t % OM, kc = t / OM;
                if (kc < KC) {
                    float acc[BT];
#pragma unroll
                    for (int b = 0; b < BT; ++b) acc[b] = 0.f;
#pragma unroll
                    for (int jj = 0; jj < CH; ++jj)
#pragma unroll
                        for (int b = 0; b < BT; ++b) acc[b] += w2r[jj] * hl2[b * TJ + kc * CH + jj];
#pragma unroll
                    for (int b = 0; b < BT; ++b) pp[(kc * OM + ol) * BT + b] = acc[b];
                }
                __syncthreads();
                // Output o = mb OM + ol of sequence b -> owner o / NQ's block [owner][tm][b][o % NQ].
                const uint32_t ep = epoch_of(a, step, l, 5);
                for (int v = t; v < OM * B; v += kThreads) {
                    const int vo = v % OM, b = v / OM;
                    float sum = 0.f;
                    for (int k = 0; k < KC; ++k) sum += pp[(k * OM + vo) * BT + b];
                    const int o = mb * OM + vo;
                    xput(a.wp2 + (((size_t)(o / NQ) * kTeams + tm) * B + b) * NQ + o % NQ, sum, ep);
                }
            }
            stamp(step, 12 * l + 9);
            {
                const int nblk = kTeams * B * NQ;
                const uint64_t* blk = a.wp2 + (size_t)w * nblk;
                gather_at<(kTeams * BT * NQ + kThreads - 1) / kThreads>(
                    nblk, epoch_of(a, step, l, 5), s.sh, a.err, [&](int i) { return blk + i; },
                    [&](int i, float v) { s.xn[i] = v; });
                __syncthreads();
                stamp(step, 12 * l + 10);
                if (t < B * NQ) {
                    const int b = t / NQ, oi = t % NQ;
                    float dx = 0.f;
                    for (int k = 0; k < kTeams; ++k) dx += s.xn[(k * B + b) * NQ + oi];
                    xput(a.wdx2 + (size_t)b * C + j0 + oi, dx, epoch_of(a, step, l, 6));
                }
                stamp(step, 12 * l + 11);
            }
        }
        // x += dx2 of the last layer, ln_f, lm_head rows v0 .. v0 + RV -> logits.  The rows are
        // streamed one round ahead: the first round is requested before the dx2 gather.
        const auto rl = rsrc(a.lm, (size_t)a.V * C);
        auto load_lm = [&](floatx4 (&wn)[kLmRowsPerWave][NQ], int c0) {
#pragma unroll
            for (int jj = 0; jj < kLmRowsPerWave; ++jj) {
                const int row = c0 + wv * kLmRowsPerWave + jj;
#pragma unroll
                for (int m = 0; m < NQ; ++m)
                    wn[jj][m] = row < RV ? ld4(rl, (size_t)(v0 + row) * C + 4 * (lane_id() + 64 * m))
                                         : floatx4{0.f, 0.f, 0.f, 0.f};
            }
        };
        floatx4 wn[kLmRowsPerWave][NQ];
        load_lm(wn, 0);
        {
            const float* const ln[2] = {a.lnf_g, a.lnf_b};
            stage_vectors<NQ, 2>(s.lnp, ln);
        }
        gather_after<BT * NQ>(G, [&](int p) { return a.wdx2 + split(C, G, p); }, B * C,
                                 epoch_of(a, step, L - 1, 6), s.sh, a.err, [&](int i) { return a.wdx2 + i; },
                                 [&](int i, float v) { s.xs[i] += v; });
        copies_barrier<0>();
        layernorm<NQ>(s.xs, s.xn, s.lnp, a.lnf_b ? s.lnp + C : nullptr, B);
        __syncthreads();
        stamp(step, 12 * L);
        {
            const bool keep = a.logit_hist && (size_t)(a.gen0 + step) < a.hist_slots;
            float* hrow = keep ? a.logit_hist + (size_t)(a.gen0 + step) * a.B * a.V : nullptr;
            for (int c0 = 0; c0 < RV; c0 += 4 * kLmRowsPerWave) {
                floatx4 wl[kLmRowsPerWave][NQ];
#pragma unroll
                for (int jj = 0; jj < kLmRowsPerWave; ++jj)
#pragma unroll
                    for (int m = 0; m < NQ; ++m) wl[jj][m] = wn[jj][m];
                if (c0 + 4 * kLmRowsPerWave < RV) load_lm(wn, c0 + 4 * kLmRowsPerWave);
                float val[kLmRowsPerWave * BT];
#pragma unroll
                for (int k = 0; k < kLmRowsPerWave * BT; ++k) val[k] = 0.f;
#pragma unroll
                for (int b = 0; b < BT; ++b) {
                    const floatx4* a4 = reinterpret_cast<const floatx4*>(s.xn + b * C);
#pragma unroll
                    for (int m = 0; m < NQ; ++m) {
                        const floatx4 xv = a4[lane + 64 * m];
#pragma unroll
                        for (int jj = 0; jj < kLmRowsPerWave; ++jj) val[jj * BT + b] += dot4(wl[jj][m], xv);
                    }
                }
                constexpr int kShift = 6 - log2c<kLmRowsPerWave * BT>();
                const float tot = reduce_many(val);
                const int k = lane >> kShift;
                const int row = c0 + wv * kLmRowsPerWave + k / BT, b = k % BT;
                if ((lane & ((1 << kShift) - 1)) == 0 && row < RV && b < B) {
                    s.lg[b * kMaxLmRows + row] = tot;
                    a.logits[(size_t)b * a.V + v0 + row] = tot;
                    if (keep) hrow[(size_t)b * a.V + v0 + row] = tot;
                }
            }
        }
        __syncthreads();
        stamp(step, 12 * L + 1);
        // First maximum of this WG's rows per sequence (rows ascending, strict '>').
        const uint32_t epc = epoch_of(a, step, L, 0);
        for (int b = wv; b < B; b += 4) {
            float bv = -INFINITY;
            int bi = 0x7fffffff;
            for (int r = lane; r < RV; r += 64) {
                const float x = s.lg[b * kMaxLmRows + r];
                if (x > bv) {
                    bv = x;
                    bi = v0 + r;
                }
            }
            wave_first_max(bv, bi);
            if (lane == 0 && w < GL) {
                uint64_t* dst = a.wcand + ((size_t)w * B + b) * 2;
                xput(dst, bv, epc);
                xput_bits(dst + 1, static_cast<uint32_t>(bi), epc);
            }
        }
        stamp(step, 12 * L + 2);
        // Every WG picks the tokens from the GL candidates itself: the [GL][B][2] words read
        // coalesced into xn (free after the lm_head rows), then wave v scans producers in WG
        // order (= row order) for sequences v, v + 4 with the first-maximum rule.
        {
            gather<2 * BT>(a.wcand, GL * B * 2, epc, s.sh, a.err, [&](int i, float v) { s.xn[i] = v; });
            __syncthreads();
            for (int b = wv; b < B; b += 4) {
                float bv = -INFINITY;
                int bi = 0x7fffffff;
                for (int g = lane; g < GL; g += 64) {
                    const float v = s.xn[(g * B + b) * 2];
                    const int vi = __float_as_int(s.xn[(g * B + b) * 2 + 1]);
                    if (v > bv || (v == bv && vi < bi)) {
                        bv = v;
                        bi = vi;
                    }
                }
                wave_first_max(bv, bi);
                if (lane == 0) {
                    const int tk = bi < 0 || bi >= a.V ? 0 : bi;
                    s.sh->token[b] = tk;
                    if (w == 0) a.hist[(size_t)b * a.HS + pos + 1] = tk;
                }
            }
            __syncthreads();
            stamp(step, 12 * L + 3);
        }
    }
    if (w == 0 && t == 0) {
        a.st_pos[0] = a.pos0 + a.n_steps;
        a.st_pos[1] = a.gen0 + a.n_steps;
    }
}

template <int NQ, int BT>
int launch(const WideArgs& a, const WidePlan& p, hipStream_t st) {
    auto kern = decode_wide_kernel<NQ, BT>;
    FMLH_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                 static_cast<int>(p.smem)));
    if (inject_fault(kFaultLaunch)) return set_error(FMLH_E_HIP, "decode_wide_kernel: launch failed (injected by FMLH_FAULT)");
    WideArgs args = a;
    void* params[] = {&args};
    const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kern), dim3(p.G), dim3(kThreads),
                                                    params, static_cast<unsigned>(p.smem), st);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        set_error(FMLH_E_HIP, "wide decode: cooperative launch refused (%s)", hipGetErrorString(e));
        return kPersistRefused;
    }
    return FMLH_OK;
}

template <int NQ>
size_t smem_bytes() { return Lds<NQ>::floats() * sizeof(float); }

}  // namespace
}  // namespace wide

WidePlan wide_plan(int B, int C, int H, int L, int V, int T, int cus) {
    WidePlan p;
    if (B < 1 || B > kWideMaxBatch || H < 1 || C != H * kWideHD || L < 1 || V < 1) return p;
    if (C % 256 != 0 || C > 1024 || T < 2 || T > kWideMaxT) return p;
    if (cus != 256) return p;  // row blocks per WG are compile-time bounded for 256 WGs
    const int G = cus, P = B * H;
    if (P > G || (V + G - 1) / G > wide::kMaxLmRows) return p;
    p.G = G;
    p.S = std::min(wide::kMaxParts, G / P);
    const int nq = C / 256;
    p.smem = nq == 1 ? wide::smem_bytes<1>() : nq == 2 ? wide::smem_bytes<2>() : nq == 3 ? wide::smem_bytes<3>()
                                                                                        : wide::smem_bytes<4>();
    if (p.smem > smem_limit()) return WidePlan{};
    p.ok = true;
    return p;
}

void wide_words(int C, int H, int Bmax, int G, int S_max, size_t out[6]) {
    const size_t B = std::min(Bmax, kWideMaxBatch);
    out[0] = B * 3 * C;                                  // wq
    out[1] = B * H * (size_t)S_max * (kWideHD + 2);      // wpart
    out[2] = B * C;                                      // wy, wdx1, wdx2 (each)
    out[3] = (size_t)wide::kTeams * B * C;               // wp2: G owners x 32 teams x B x C / G
    out[4] = (size_t)G * B * 2;                          // wcand
    out[5] = B * 4 * C;                                  // wh
}

int wide_decode(const WideArgs& a, const WidePlan& p, hipStream_t s) {
    if (!p.ok) return set_error(FMLH_E_INVALID, "wide decode not planned for this shape");
    const bool b4 = a.B <= 4;  // batch tile 4 or 8
    switch (a.C) {
        case 256: return b4 ? wide::launch<1, 4>(a, p, s) : wide::launch<1, 8>(a, p, s);
        case 512: return b4 ? wide::launch<2, 4>(a, p, s) : wide::launch<2, 8>(a, p, s);
        case 768: return b4 ? wide::launch<3, 4>(a, p, s) : wide::launch<3, 8>(a, p, s);
        case 1024: return b4 ? wide::launch<4, 4>(a, p, s) : wide::launch<4, 8>(a, p, s);
        default: return set_error(FMLH_E_INVALID, "wide decode: n_embed %d not compiled", a.C);
    }
}

}  // namespace fmlh
