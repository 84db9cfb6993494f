// Host side of the grouped persistent decode kernel (decode_grouped_kernel.h): shape planning
// and dispatch to the instantiated (head_dim, n_embed) variants.
#include "decode_grouped_kernel.h"

#include <algorithm>

namespace fmlh {
namespace {

long ceil_div(long a, long b) { return (a + b - 1) / b; }

// The (head_dim, n_embed / 64) pairs compiled: the 384-wide c2/c3 model and the small test shapes.
bool instantiated(int hd, int ne) {
    return (hd == 64 && ne == 6) || (hd == 16 && ne == 1) || (hd == 32 && ne == 1) || (hd == 32 && ne == 4);
}

}  // namespace

GroupedPlan grouped_plan(int B, int C, int H, int L, int V, int T, int cus) {
    GroupedPlan p;
    const int hd = H > 0 ? C / H : 0;
    if (B < 1 || B > kGroupBatch * kMaxGroups || L < 1 || V < 1 || hd * H != C || C % 64 != 0) return p;
    // T a multiple of 16: attention reads whole 16-row groups of the cache
    if (!instantiated(hd, C / 64) || T > kGroupedMaxT || T % 16 != 0) return p;
    p.groups = (int)ceil_div(B, kGroupBatch);
    p.Bg = (int)ceil_div(B, p.groups);
    // One WG per CU.  G <= C: every WG then owns rows of each C-row product, which the
    // single-buffer safety argument needs.  G <= kMaxGroupWGs: past that the wait for the
    // slowest of G producers and the G-way proj2 gather cost more than the smaller row share
    // saves (c3 on MI355X, 16 sequences: 163 us/step at G = 48, 170 at 64, 180 at 128).
    // Rows split evenly: C / G proj2 outputs per WG (hop 5 adds G partials of each), and FC rows
    // in multiples of 4 (each WG's proj2 partial reads W_proj2 columns of its FC rows as float4):
    // the largest such G that fits.
    p.G = std::min({cus / p.groups, C, kMaxGroupWGs});
    while (p.G > 0 && (C % p.G != 0 || (4 * C / p.G) % 4 != 0)) --p.G;
    if (p.G < 1) return GroupedPlan{};
    p.tq = (int)ceil_div(4L * C / p.G, grouped::kTile);
    if (p.tq > 3 || ceil_div(C, p.G) > grouped::kTile || ceil_div(V, p.G) > grouped::kTile) return GroupedPlan{};
    const long u = std::max(8L * C + 8L * grouped::h_row(p.tq) + 8L * C + 4L * p.tq * 256, 2L * T * hd);
    const long floats = grouped::grouped_scratch_floats(hd) + u;
    p.smem = (size_t)floats * sizeof(float);
    if (p.smem > smem_limit()) return GroupedPlan{};
    p.ok = true;
    return p;
}

void grouped_group_words(int C, int G_max, size_t out[2]) {
    out[0] = (size_t)kGroupBatch * C;
    out[1] = (size_t)G_max * kGroupBatch * 2;
}

int grouped_decode(const GroupedArgs& a, const GroupedPlan& p, int C, int hd, hipStream_t s) {
    if (!p.ok) return set_error(FMLH_E_INVALID, "grouped decode not planned for this shape");
    const int ne = C / 64;
    if (hd == 64 && ne == 6) return grouped::launch_tq<64, 6>(a, p, s);
    if (hd == 16 && ne == 1) return grouped::launch_tq<16, 1>(a, p, s);
    if (hd == 32 && ne == 1) return grouped::launch_tq<32, 1>(a, p, s);
    if (hd == 32 && ne == 4) return grouped::launch_tq<32, 4>(a, p, s);
    return set_error(FMLH_E_INVALID, "grouped decode: head_dim %d, n_embed %d not compiled", hd, C);
}

}  // namespace fmlh
