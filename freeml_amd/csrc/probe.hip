// fmlh_probe_exchange: the latency of a hand-off through exchange words (exchange.h) between
// the workgroups of one resident launch -- the cost the persistent decode kernels pay per hop.
// Built into its own library (libfreeml_probe.so), not the product one.
//
// One cooperative launch of one WG per CU (the placement the decode kernels get).  Every WG
// records its XCD.  Group A (and, in the two-group form, group B) then run `rounds` timed
// rounds after 8 untimed ones:
//   * all-to-all (nb = 0): every WG of A publishes its share of `words` words and gathers all of
//     them; one hop per round.  Words alternate between two buffers by round parity, so a WG
//     that starts round r + 1 never overwrites a word another WG still waits for in round r.
//   * A -> B -> A (nb > 0): A publishes `words` words (shared out over its WGs), every WG of B
//     gathers them all and publishes `words` words back, every WG of A gathers those; two hops
//     per round.  A publishes round r + 1 only after reading all of B's round-r words, which B
//     writes after its own reads, so single buffers suffice.
// Every poll is bounded (kSpinLimit); a WG that gives up sets the error word and stops.
#include "exchange.h"
#include "fmlh_internal.h"
#include "../../include/freeml_probe.h"

#include <vector>

namespace fmlh {
namespace {

constexpr int kThreads = 256;
constexpr long kSpinLimit = 1L << 21;
constexpr int kWarmRounds = 8;
constexpr int kProbeLds = 96 * 1024;  // more than half a CU's LDS: one WG per CU

struct ProbeArgs {
    int scope;  // 0 device, 1 XCD (buffer sc0), 2-5 global-instruction variants (get/put),
                // 6-8 device scope with pipelined polls (gather_any), 9-12 forms whose loads
                // skip the CU's L1 but may be served by the XCD's L2 (get/put)
    const int* ga;
    int na;
    const int* gb;
    int nb;
    int words, rounds;
    uint64_t* buf;  // 3 * words: A's two parity buffers (all-to-all) or A's and B's words
    uint32_t epoch;
    int* xcc;                  // per WG
    unsigned long long* t;     // [0] first timed round starts, [1] last round ends (A's first WG)
    unsigned* err;
};

// Word i of buffer `base` (word offset into a.buf) published with `epoch`.
__device__ __forceinline__ void put(const ProbeArgs& a, xchg::XcdBuf xb, int base, int i, uint32_t bits,
                                    uint32_t epoch) {
    const uint64_t w = xchg::pack(bits, epoch);
    uint64_t* p = a.buf + base + i;
    switch (a.scope) {
        case 1: xchg::xcd_store(xb, static_cast<uint32_t>(base + i), w); break;
        case 2: asm volatile("global_store_dwordx2 %0, %1, off sc0" :: "v"(p), "v"(w) : "memory"); break;
        case 3: asm volatile("global_store_dwordx2 %0, %1, off" :: "v"(p), "v"(w) : "memory"); break;
        case 4: asm volatile("global_store_dwordx2 %0, %1, off sc1" :: "v"(p), "v"(w) : "memory"); break;
        case 5: asm volatile("global_store_dwordx2 %0, %1, off sc0" :: "v"(p), "v"(w) : "memory"); break;
        case 9:
        case 11: asm volatile("global_store_dwordx2 %0, %1, off" :: "v"(p), "v"(w) : "memory"); break;
        default: xchg::dev_store(p, w); break;  // 0, 6-8, 10, 12: agent-scope (sc1) store
    }
}

// One word as the scope's consumer loads it.  Scopes 2-5 are single-instruction variants of
// the XCD-scope form (cache policy bits on global loads and stores) used to find which of them
// is coherent between the CUs of one XCD.
__device__ __forceinline__ uint64_t get(const ProbeArgs& a, xchg::XcdBuf xb, int idx) {
    const uint64_t* p = a.buf + idx;
    uint64_t v;
    switch (a.scope) {
        case 1: return xchg::xcd_load(xb, static_cast<uint32_t>(idx));
        case 2:
        case 3:
        case 4:
            asm volatile("global_load_dwordx2 %0, %1, off sc0\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
            return v;
        case 5:
            asm volatile("buffer_inv sc0\n\tglobal_load_dwordx2 %0, %1, off\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
            return v;
        case 9:  // plain store, device-scope (sc1) load: does an sc1 load see a line held in L2?
            asm volatile("global_load_dwordx2 %0, %1, off sc1\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
            return v;
        case 10:  // sc1 store, then an agent-scope invalidate and a plain load
            asm volatile("buffer_inv sc1\n\tglobal_load_dwordx2 %0, %1, off\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
            return v;
        case 11:
        case 12: {
            // Scalar load with glc (it misses the scalar cache and is served by the XCD's L2).
            // The address must be uniform over the active lanes: the host allows these scopes
            // for one-word hand-offs only, where one lane of the WG polls.  The index is taken
            // from the first active lane and clamped to the buffer (3 * words words), so the
            // load stays in bounds even where the compiler runs it with no lane active.
            const int i0 = min(__builtin_amdgcn_readfirstlane(idx), 3 * a.words - 1);
            const uint64_t* sp = a.buf + max(i0, 0);
            asm volatile("s_load_dwordx2 %0, %1, 0x0 glc\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(sp) : "memory");
            return v;
        }
        default: return xchg::dev_load(p);
    }
}

// All n words of buffer `base` at `epoch` into LDS (all threads; 8 words per thread per batch,
// stale words polled again).  False once the spin limit was reached.
__device__ bool gather(const ProbeArgs& a, xchg::XcdBuf xb, int base, int n, uint32_t epoch, float* lds) {
    constexpr int kB = 8;
    for (int b0 = 0; b0 < n; b0 += kB * kThreads) {
        uint64_t v[kB];
        int idx[kB];
#pragma unroll
        for (int k = 0; k < kB; ++k) {
            idx[k] = b0 + k * kThreads + static_cast<int>(threadIdx.x);
            v[k] = xchg::pack(0, epoch);
            if (idx[k] < n) v[k] = get(a, xb, base + idx[k]);
        }
        long it = 0;
        while (true) {
            bool stale = false;
#pragma unroll
            for (int k = 0; k < kB; ++k) stale |= !xchg::current(v[k], epoch);
            if (!stale) break;
            if (++it > kSpinLimit) {
                atomicOr(a.err, 1u);
                return false;
            }
#pragma unroll
            for (int k = 0; k < kB; ++k)
                if (!xchg::current(v[k], epoch))
                    v[k] = get(a, xb, base + idx[k]);
        }
#pragma unroll
        for (int k = 0; k < kB; ++k)
            if (idx[k] < n) lds[idx[k]] = xchg::payload(v[k]);
    }
    return true;
}

// Device scope with pipelined polls: each thread keeps D loads of each of its (at most 2) words
// in flight, issued `gap` s_sleep units apart, and checks the oldest; a new load replaces each
// checked one.  The store is then seen about one load latency after it lands instead of up to
// a whole round trip later.  The loop body names the D slots explicitly so that no pending load
// result is ever moved between registers (which would force a wait for it).
template <int D>
__device__ bool gather_pipelined(const ProbeArgs& a, int base, int n, uint32_t epoch, float* lds, int gap) {
    const int t = static_cast<int>(threadIdx.x);
    // Lanes past n poll a valid word too (word n - 1), so every load is unconditional and the
    // compiler can count the loads in flight exactly.
    const uint64_t* q0 = a.buf + base + min(t, n - 1);
    const uint64_t* q1 = a.buf + base + min(t + kThreads, n - 1);
    uint64_t r0[D], r1[D];
    bool ok0 = false, ok1 = false;
    uint64_t f0 = 0, f1 = 0;
#pragma unroll
    for (int k = 0; k < D; ++k) {
        r0[k] = xchg::dev_load(q0);
        r1[k] = xchg::dev_load(q1);
        if (gap) __builtin_amdgcn_s_sleep(1);
    }
    long it = 0;
    while (true) {
        bool all = false;
#pragma unroll
        for (int k = 0; k < D; ++k) {
            const bool c0 = xchg::current(r0[k], epoch), c1 = xchg::current(r1[k], epoch);
            f0 = (c0 && !ok0) ? r0[k] : f0;
            f1 = (c1 && !ok1) ? r1[k] : f1;
            ok0 = ok0 || c0;
            ok1 = ok1 || c1;
            all = __all(ok0 && ok1);
            if (all) break;
            r0[k] = xchg::dev_load(q0);
            r1[k] = xchg::dev_load(q1);
            if (gap) __builtin_amdgcn_s_sleep(1);
        }
        if (all) break;
        if (++it > kSpinLimit / D) {
            atomicOr(a.err, 1u);
            return false;
        }
    }
    if (t < n) lds[t] = xchg::payload(f0);
    if (t + kThreads < n) lds[t + kThreads] = xchg::payload(f1);
    return true;
}

__device__ __forceinline__ bool gather_any(const ProbeArgs& a, xchg::XcdBuf xb, int base, int n, uint32_t epoch,
                                           float* lds) {
    if (a.scope == 6) return gather_pipelined<4>(a, base, n, epoch, lds, 1);
    if (a.scope == 7) return gather_pipelined<4>(a, base, n, epoch, lds, 0);
    if (a.scope == 8) return gather_pipelined<8>(a, base, n, epoch, lds, 1);
    return gather(a, xb, base, n, epoch, lds);
}

__global__ __launch_bounds__(kThreads) void probe_kernel(ProbeArgs a) {
    extern __shared__ float lds[];
    __shared__ int ok;
    const int wg = static_cast<int>(blockIdx.x), tid = static_cast<int>(threadIdx.x);
    if (tid == 0) {
        a.xcc[wg] = xchg::xcc_id();
        ok = 1;
    }
    int ia = -1, ib = -1;
    for (int i = 0; i < a.na; ++i)
        if (a.ga[i] == wg) ia = i;
    for (int i = 0; i < a.nb; ++i)
        if (a.gb[i] == wg) ib = i;
    if (ia < 0 && ib < 0) return;
    const xchg::XcdBuf xb = xchg::xcd_buf(a.buf);
    const int W = a.words;
    const int total = a.rounds + kWarmRounds;
    __syncthreads();
    for (int r = 0; r < total; ++r) {
        if (ia == 0 && tid == 0 && r == kWarmRounds) a.t[0] = wall_clock64();
        const uint32_t ep = a.epoch + static_cast<uint32_t>(r);
        if (a.nb == 0) {
            const int base = (r & 1) * W;
            const int lo = (W * ia) / a.na, hi = (W * (ia + 1)) / a.na;
            for (int i = lo + tid; i < hi; i += kThreads) put(a, xb, base, i, static_cast<uint32_t>(i), ep);
            if (!gather_any(a, xb, base, W, ep, lds)) ok = 0;
        } else if (ia >= 0) {
            const int lo = (W * ia) / a.na, hi = (W * (ia + 1)) / a.na;
            for (int i = lo + tid; i < hi; i += kThreads) put(a, xb, 0, i, static_cast<uint32_t>(i), ep);
            if (!gather_any(a, xb, W, W, ep, lds)) ok = 0;
        } else {
            if (!gather_any(a, xb, 0, W, ep, lds)) ok = 0;
            __syncthreads();
            const int lo = (W * ib) / a.nb, hi = (W * (ib + 1)) / a.nb;
            for (int i = lo + tid; i < hi; i += kThreads) put(a, xb, W, i, static_cast<uint32_t>(i), ep);
        }
        __syncthreads();
        if (!ok) return;
    }
    if (ia == 0 && tid == 0) a.t[1] = wall_clock64();
}

// Epochs grow across calls so that words left by an earlier call never match.
uint32_t g_probe_epoch = 1;

}  // namespace
}  // namespace fmlh

using namespace fmlh;

extern "C" int fmlh_probe_exchange(int scope, const int32_t* group_a, uint32_t na, const int32_t* group_b,
                                   uint32_t nb, uint32_t words, uint32_t rounds, int32_t* xcc_out,
                                   double* ns_per_hop) {
    FMLH_TRY(ensure_init());
    const int G = cu_count();
    FMLH_REQUIRE(scope >= 0 && scope <= 12, "fmlh_probe_exchange: scope must be 0..12");
    FMLH_REQUIRE(scope < 11 || (words == 1 && na == 1 && nb == 1),
                 "fmlh_probe_exchange: scalar-load scopes take one-word ping-pongs only");
    FMLH_REQUIRE(scope < 6 || words <= 2 * kThreads, "fmlh_probe_exchange: pipelined polls take at most %d words", 2 * kThreads);
    FMLH_REQUIRE(group_a && na >= 1 && na <= (uint32_t)G, "fmlh_probe_exchange: group A needs 1..%d WGs", G);
    FMLH_REQUIRE(nb == 0 || (group_b && nb <= (uint32_t)G), "fmlh_probe_exchange: group B has more WGs than CUs");
    FMLH_REQUIRE(words >= na && words >= nb && words <= (uint32_t)kProbeLds / 4,
                 "fmlh_probe_exchange: words must cover every WG of a group and fit the WG's LDS (%d)", kProbeLds / 4);
    FMLH_REQUIRE(rounds >= 1 && rounds <= 1000000, "fmlh_probe_exchange: rounds must be 1..1e6");
    std::vector<int> ids(group_a, group_a + na);
    for (uint32_t i = 0; i < nb; ++i) ids.push_back(group_b[i]);
    for (size_t i = 0; i < ids.size(); ++i) {
        FMLH_REQUIRE(ids[i] >= 0 && ids[i] < G, "fmlh_probe_exchange: WG id %d outside 0..%d", ids[i], G - 1);
        for (size_t j = 0; j < i; ++j)
            FMLH_REQUIRE(ids[i] != ids[j], "fmlh_probe_exchange: WG %d listed twice", ids[i]);
    }
    const uint32_t span = rounds + kWarmRounds;
    if (g_probe_epoch > 0xffffffffu - span - 1) g_probe_epoch = 1;  // new buffers below: no stale words
    hipStream_t s = stream();
    int* d_ids = nullptr;
    uint64_t* d_buf = nullptr;
    int* d_xcc = nullptr;
    unsigned long long* d_t = nullptr;
    unsigned* d_err = nullptr;
    int rc = FMLH_OK;
    auto fail = [&](hipError_t e, const char* what) {
        if (rc == FMLH_OK && e != hipSuccess) rc = hip_fail(e, what, __FILE__, __LINE__);
    };
    fail(hipMalloc(&d_ids, ids.size() * sizeof(int)), "hipMalloc");
    fail(hipMalloc(&d_buf, 3ull * words * sizeof(uint64_t)), "hipMalloc");
    fail(hipMalloc(&d_xcc, G * sizeof(int)), "hipMalloc");
    fail(hipMalloc(&d_t, 2 * sizeof(unsigned long long)), "hipMalloc");
    fail(hipMalloc(&d_err, sizeof(unsigned)), "hipMalloc");
    if (rc == FMLH_OK) {
        fail(hipMemcpyAsync(d_ids, ids.data(), ids.size() * sizeof(int), hipMemcpyHostToDevice, s), "copy");
        fail(hipMemsetAsync(d_buf, 0, 3ull * words * sizeof(uint64_t), s), "memset");
        fail(hipMemsetAsync(d_t, 0, 2 * sizeof(unsigned long long), s), "memset");
        fail(hipMemsetAsync(d_err, 0, sizeof(unsigned), s), "memset");
    }
    if (rc == FMLH_OK) {
        ProbeArgs a{scope, d_ids, (int)na, d_ids + na, (int)nb, (int)words, (int)rounds, d_buf, g_probe_epoch,
                    d_xcc, d_t, d_err};
        g_probe_epoch += span;
        fail(hipFuncSetAttribute(reinterpret_cast<const void*>(probe_kernel),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, kProbeLds), "hipFuncSetAttribute");
        void* params[] = {&a};
        if (rc == FMLH_OK)
            fail(hipLaunchCooperativeKernel(reinterpret_cast<const void*>(probe_kernel), dim3(G), dim3(kThreads),
                                            params, kProbeLds, s), "hipLaunchCooperativeKernel");
    }
    unsigned err = 0;
    unsigned long long t[2] = {0, 0};
    std::vector<int> xcc(G, -1);
    if (rc == FMLH_OK) {
        fail(hipMemcpyAsync(&err, d_err, sizeof(unsigned), hipMemcpyDeviceToHost, s), "copy");
        fail(hipMemcpyAsync(t, d_t, sizeof(t), hipMemcpyDeviceToHost, s), "copy");
        fail(hipMemcpyAsync(xcc.data(), d_xcc, G * sizeof(int), hipMemcpyDeviceToHost, s), "copy");
        fail(hipStreamSynchronize(s), "hipStreamSynchronize");
    }
    int clock_khz = 0;
    if (rc == FMLH_OK) fail(hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeWallClockRate, 0), "attribute");
    (void)hipFree(d_ids);
    (void)hipFree(d_buf);
    (void)hipFree(d_xcc);
    (void)hipFree(d_t);
    (void)hipFree(d_err);
    if (rc != FMLH_OK) return rc;
    if (xcc_out)
        for (int i = 0; i < G; ++i) xcc_out[i] = xcc[i];
    if (err) return set_error(FMLH_E_STATE, "fmlh_probe_exchange: a wait gave up (words never observed at scope %d)", scope);
    const double hops = (double)rounds * (nb ? 2 : 1);
    if (ns_per_hop) *ns_per_hop = clock_khz > 0 ? (double)(t[1] - t[0]) * 1e6 / clock_khz / hops : 0.0;
    return FMLH_OK;
}
