// Group descriptors of a KVMap slice (host C++; format documented with
// kvp_attn_forward_frames_gd in kvp_c_api.h).
//
// A frame's key range [b, e) is cut into 16-row groups g (rows
// [b + 16 g, b + 16 g + 16) below e), the copy groups of the bf16 attention
// kernel. Entry g says which rows of group g the map sends to the arena:
//   (0, 0)   none;
//   (1, 0)   general: the kernel reads the group's map entries;
//   (A, B)   A a sub-run word, B a second one or 0. A sub-run word with
//            bit 31 set says rows r0 .. r0 + n - 1 of the group map to arena
//            rows l .. l + n - 1: l in bits 0-22, r0 in bits 23-26, n - 1 in
//            bits 27-30.
// Rows of the group outside every sub-run map to no arena row.
#pragma once

#include <algorithm>
#include <vector>

namespace kvp {
namespace gd {

// One sub-run: rows [r0, r0 + n) of group g map to arena rows [l, l + n).
struct Sub {
    long g;
    int r0;
    int n;
    long l;
};

// Entry of a frame's table: group g holds words w0, w1.
struct Ent {
    long g;
    unsigned w0, w1;
};

constexpr long kMaxArenaRow = (1L << 23) - 1;

inline unsigned word(const Sub& s) {
    return 0x80000000u | ((unsigned)(s.n - 1) << 27) | ((unsigned)s.r0 << 23) | (unsigned)s.l;
}

// Adds the sub-runs of key rows [j0, j0 + n) mapped to arena rows
// [l0, l0 + n), clipped to the range [b, e), group by group.
inline void add_rows(std::vector<Sub>& subs, long j0, long n, long l0, long b, long e) {
    const long lo = std::max(j0, b);
    const long hi = std::min(j0 + n, e);
    for (long s = lo; s < hi;) {
        const long g = (s - b) / 16;
        const long gs = b + 16 * g;
        const long t = std::min(hi, gs + 16);
        subs.push_back(Sub{g, (int)(s - gs), (int)(t - s), l0 + (s - j0)});
        s = t;
    }
}

// Entries of the groups the sub-runs touch, in group order: adjacent
// sub-runs that continue each other in rows and arena rows merge; a group
// left with more than two, or with an arena row past kMaxArenaRow, is
// general. `subs` is reordered.
inline void encode(std::vector<Sub>& subs, std::vector<Ent>& out) {
    out.clear();
    std::sort(subs.begin(), subs.end(), [](const Sub& x, const Sub& y) {
        return x.g != y.g ? x.g < y.g : x.r0 < y.r0;
    });
    size_t i = 0;
    while (i < subs.size()) {
        const long g = subs[i].g;
        Sub run[2];
        int nr = 0;
        bool general = false;
        for (; i < subs.size() && subs[i].g == g; ++i) {
            const Sub& s = subs[i];
            if (nr > 0 && run[nr - 1].r0 + run[nr - 1].n == s.r0 &&
                run[nr - 1].l + run[nr - 1].n == s.l) {
                run[nr - 1].n += s.n;
            } else if (nr < 2) {
                run[nr++] = s;
            } else {
                general = true;
            }
        }
        for (int r = 0; r < nr; ++r)
            if (run[r].l < 0 || run[r].l + run[r].n - 1 > kMaxArenaRow) general = true;
        if (general)
            out.push_back(Ent{g, 1u, 0u});
        else
            out.push_back(Ent{g, word(run[0]), nr > 1 ? word(run[1]) : 0u});
    }
}

}  // namespace gd
}  // namespace kvp
