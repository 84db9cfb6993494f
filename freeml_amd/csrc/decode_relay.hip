// Host side of the relay decode kernel (decode_relay_kernel.h): team sizes and dispatch.
#include "decode_relay_kernel.h"

#include <algorithm>
#include <cstdlib>

namespace fmlh {

RelayPlan relay_plan(int B, int C, int H, int L, int V, int T, int cus) {
    RelayPlan p;
    // compiled: C = 256, 384, 512 (head_dim 64)
    if (B < 1 || B > kRelayMaxBatch || H < 1 || C != H * relay::kHD || (C != 256 && C != 384 && C != 512)) return p;
    if (L < 1 || V < 1 || V > kRelayMaxVocab) return p;
    if (T > kRelayMaxT || T % 16 != 0) return p;
    // Each head's q in its attention role (the Q team then holds the k and v rows only) for small
    // batches, where it shortens a layer's critical path; for larger ones the attention roles
    // are the busiest and the Q team forms q as well.  FMLH_RELAY_QA=0 / 1 forces either.
    const char* qa_env = std::getenv("FMLH_RELAY_QA");
    p.qa = qa_env && (qa_env[0] == '0' || qa_env[0] == '1') ? qa_env[0] == '1' : B <= kRelayQaMaxBatch;
    p.qa = p.qa && 2 * C % kRelayTeamRows == 0;  // the k / v rows in whole Q slices (C = 384)
    // From kRelayBigBatch sequences the FC team is the busiest and its row sums tie its
    // workgroups together: they move to a team of their own, paid for with half the Q team.
    // FMLH_RELAY_BIG=0 / 1 forces either (not together with qa).
    const char* big_env = std::getenv("FMLH_RELAY_BIG");
    p.big = !p.qa && (big_env && (big_env[0] == '0' || big_env[0] == '1') ? big_env[0] == '1' : B >= kRelayBigBatch);
    p.big = p.big && C <= 384;  // 192-row Q slices: 48 weight registers per lane and NE
    // From kRelaySplitBatch sequences the attention roles are the busiest: two per head, and two
    // lm_head roles, each taking every other sequence; at C = 384 paid for with 96-row FC slices.
    // FMLH_RELAY_SPLIT=0 / 1 forces either (with big).
    const char* split_env = std::getenv("FMLH_RELAY_SPLIT");
    p.split = p.big && (C == 256 || C == 384) &&
              (split_env && (split_env[0] == '0' || split_env[0] == '1') ? split_env[0] == '1' : B >= kRelaySplitBatch);
    // From kRelayHBatch sequences (split, n_embed 384) the FC team is the busiest again: the h cut
    // gives it 128-row slices that publish h, and the F2 team (32 rows of x_{l+1} each) the MLP
    // projection's rows (a row split over all of h) in place of adding the FC team's column-split
    // partials, so the two teams share the MLP's work.  FMLH_RELAY_HCUT=0 / 1 forces either (with
    // split).
    const char* h_env = std::getenv("FMLH_RELAY_HCUT");
    p.hcut = p.split && C == 384 &&
             (h_env && (h_env[0] == '0' || h_env[0] == '1') ? h_env[0] == '1' : B >= kRelayHBatch);
    p.nq = p.big ? 3 * C / kRelayBigTeamRows : (p.qa ? 2 : 3) * C / kRelayTeamRows;
    p.nf = 4 * C / (p.hcut ? kRelayHRows : p.split && C == 384 ? kRelaySplitFRows : kRelayFRows);
    p.nf2 = p.big ? C / (p.hcut ? kRelayHF2Rows : kRelayF2Rows) : 0;
    p.nA = p.nlm = p.split ? 2 : 1;
    if (C % p.nf != 0 || (C / p.nf) * p.nf > relay::kThreads) return RelayPlan{};  // F's rows of x
    p.roles = L * (p.nq + p.nA * H + p.nf + p.nf2) + p.nlm;
    p.G = std::min(cus, p.roles);
    if (p.G < 1 || 2L * p.G < p.roles) return RelayPlan{};  // at most two roles per workgroup
    p.smem = (size_t)(relay::kScratch + 2 * C + 4 + (size_t)V * C + C) * sizeof(float);  // lm: token table + position row
    if (p.smem > smem_limit()) return RelayPlan{};
    p.ok = true;
    return p;
}

void relay_words(int C, int H, int L, int B, size_t out[5]) {
    out[0] = (size_t)(L + 1) * B * C;
    out[1] = (size_t)L * B * (4 * C / kRelayFRows) * C;
    out[2] = (size_t)L * B * 3 * C;
    out[3] = (size_t)L * B * H * C;
    out[4] = (size_t)L * B * C;
}

int relay_decode(const RelayArgs& a, const RelayPlan& p, int C, int hd, hipStream_t s) {
    if (!p.ok) return set_error(FMLH_E_INVALID, "relay decode not planned for this shape");
    if (hd == relay::kHD && C == 384)
        return p.qa      ? relay::launch<6, true, false, 0>(a, p, s)
               : p.hcut  ? relay::launch<6, false, true, 2>(a, p, s)
               : p.split ? relay::launch<6, false, true, 1>(a, p, s)
               : p.big   ? relay::launch<6, false, true, 0>(a, p, s)
                         : relay::launch<6, false, false, 0>(a, p, s);
    if (hd == relay::kHD && C == 256)
        return p.split ? relay::launch<4, false, true, 1>(a, p, s)
               : p.big ? relay::launch<4, false, true, 0>(a, p, s)
                       : relay::launch<4, false, false, 0>(a, p, s);
    if (hd == relay::kHD && C == 512) return relay::launch<8, false, false, 0>(a, p, s);
    return set_error(FMLH_E_INVALID, "relay decode: head_dim %d, n_embed %d not compiled", hd, C);
}

}  // namespace fmlh
