// Host side of the relay decode kernel (decode_relay_kernel.h): team sizes and dispatch.
#include "decode_relay_kernel.h"

#include <algorithm>

namespace fmlh {

namespace {

// Smallest team (at most 16 workgroups) whose per-workgroup slice of `rows` rows of K floats
// is a multiple of `unit` rows and fits the weight area.
int team(int rows, int K, int unit) {
    for (int n = 1; n <= 16; ++n)
        if (rows % n == 0 && (rows / n) % unit == 0 && (long)(rows / n) * K <= kRelayWeightFloats) return n;
    return 0;
}

}  // namespace

RelayPlan relay_plan(int B, int C, int H, int L, int V, int T, int cus) {
    RelayPlan p;
    if (B != 1 || H < 1 || C != H * relay::kHD || C % 64 != 0 || C / 64 != 6) return p;  // compiled: C = 384
    if (L < 1 || V < 1 || V > 128 || (long)V * C > kRelayWeightFloats || (long)C * relay::kHD > kRelayWeightFloats)
        return p;
    if (T > kRelayMaxT || T % 16 != 0) return p;
    p.nq = team(3 * C, C, 16);
    p.nf = team(4 * C, C, 16);
    p.np = team(C, 4 * C, 4);
    if (!p.nq || !p.nf || !p.np) return RelayPlan{};
    if (3 * C / p.nq != kRelayTeamRows || 4 * C / p.nf != kRelayTeamRows || C / p.np != kRelayPRows)
        return RelayPlan{};  // compiled row counts
    p.roles = L * (p.nq + H + p.nf + p.np) + 1;
    p.G = std::min(cus, p.roles);
    if (p.G < 1 || 2L * p.G < p.roles) return RelayPlan{};  // at most two roles per workgroup
    p.smem = (size_t)(kRelayWeightFloats + H * C + 2 * C + 4) * sizeof(float);
    if (p.smem > smem_limit()) return RelayPlan{};
    p.ok = true;
    return p;
}

void relay_words(int C, int H, int L, size_t out[4]) {
    out[0] = (size_t)(L + 1) * C;
    out[1] = (size_t)L * 3 * C;
    out[2] = (size_t)L * H * C;
    out[3] = (size_t)L * 4 * C;
}

int relay_decode(const RelayArgs& a, const RelayPlan& p, int C, int hd, hipStream_t s) {
    if (!p.ok) return set_error(FMLH_E_INVALID, "relay decode not planned for this shape");
    if (hd == relay::kHD && C == 384) return relay::launch<6>(a, p, s);
    return set_error(FMLH_E_INVALID, "relay decode: head_dim %d, n_embed %d not compiled", hd, C);
}

}  // namespace fmlh
