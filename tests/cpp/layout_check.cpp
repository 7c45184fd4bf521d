// Host check of the grid and workspace layout helpers the kernels use (csrc/layout.hpp),
// built with a plain C++ compiler.  Prints "ok" and exits 0 when every check holds.
//
// - div_uniform against integer division.
// - The XCD-local designated grid (xcd_slot over a grid padded to whole rounds of 8 heads) as
//   a bijection onto the real (head, segment) slots, every segment of a head on one XCD,
//   whatever XCD the dispatch starts on.
// - Every workgroup of a designated grid (XCD-local from 8 heads, dense below), for
//   B in {1, 2, 3, 17}, NH in 1..40, S in 1..64: a padding slot (a head beyond B * NH) must
//   exit before any load (no speculative tile, no segment), and a live slot's speculative
//   K/V rows, q row, partial index and tagged-word indices must stay inside the cache slot,
//   qkv and the workspace (the reference grid these replace: attention_kvcache.cuh:185-207).
// - Workspace layouts (ws_layout): every region inside the buffer and disjoint from the
//   others, the counters covering every head, and two plans on one buffer never placing
//   counters or tags where the other left partials.
// - Planted mistakes must fail: the shortcut that decoded every slot of a one-sequence call as
//   sequence 0 (padding heads 12-15 of a GPT-2 layer then read V rows past the cache and wrote
//   past the workspace), a missing guess guard, a counter region sized by the plan.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "layout.hpp"

using namespace kvattn_layout;

static int g_fail = 0;
static bool g_quiet = false;   // planted runs: count failures without printing

static bool check(bool ok, const char* what, long long a, long long b, long long c) {
    if (!ok) {
        if (!g_quiet && g_fail < 20) std::printf("FAIL %s (%lld, %lld, %lld)\n", what, a, b, c);
        ++g_fail;
    }
    return ok;
}

// ---------------------------------------------------------------------------------------
// Grid decode under test: the kernels' functions, or a planted variant.
// ---------------------------------------------------------------------------------------
struct Decode {
    bool (*slot)(int v, int S, int B, int NH, int& b, int& h, int& s);
    bool (*guess_live)(int bh0, int BNH);
};

static bool real_slot(int v, int S, int B, int NH, int& b, int& h, int& s) {
    return dense_slot(v, S, B * NH, NH, b, h, s);
}
static bool real_guess(int bh0, int BNH) { return guess_slot_live(bh0, BNH); }

// The faulting shortcut: one sequence -> b = 0 for every slot (padding slots become live).
static bool planted_slot(int v, int S, int B, int NH, int& b, int& h, int& s) {
    const int bh = v / S;
    s = v - bh * S;
    b = B == 1 ? 0 : bh / NH;
    h = bh - b * NH;
    return b < B;
}
static bool planted_guess(int, int) { return true; }

constexpr int kMl = 16, kCh = 64, kW = 4;

// Every workgroup of the designated grid of (B, NH, S) slots, for a cache slot of maxT rows
// and `nom` nominal rows per segment (the speculative tile's window).
static void check_grid(const Decode& d, int B, int NH, int S, int maxT, int nom, int tile_rows) {
    const int BNH = B * NH;
    const bool xl = BNH >= 8;
    const long long grid = xl ? 8ll * ((BNH + 7) / 8) * S : (long long)BNH * S;
    const long long slots = (long long)BNH * S;
    std::vector<int> seen(slots, 0);
    for (long long x = 0; x < grid; ++x) {
        const int v = xl ? xcd_slot((int)x, S) : (int)x;
        const int bh0 = div_uniform(v, S), s0 = v - bh0 * S;
        int b = -1, h = -1, s = -1;
        const bool live = d.slot(v, S, B, NH, b, h, s);
        const bool guess = d.guess_live(bh0, BNH);
        if (bh0 >= BNH) {
            // Padding: exits before any load.
            check(!live && !guess, "padding slot does not exit", BNH, S, x);
            continue;
        }
        if (!check(live, "real slot exits", BNH, S, x)) continue;
        check(b >= 0 && b < B && h >= 0 && h < NH && s >= 0 && s < S, "slot decode out of range", b, h, s);
        const long long pidx = ((long long)b * NH + h) * S + s;
        check(pidx == v && pidx < slots, "partial index", pidx, v, slots);
        if (pidx >= 0 && pidx < slots) seen[pidx]++;
        check((long long)kMl * pidx + 1 < slots * kMl, "tag_ml index", pidx, S, BNH);
        check(pidx * kCh + kCh - 1 < slots * kCh, "tag_out index", pidx, S, BNH);
        if (guess) {
            // Speculative tile of every wave: rows clamped into [w0, w1) as load_tile does.
            for (int w = 0; w < kW; ++w) {
                int nend, w0, w1;
                guess_rows(s0, nom, nom, maxT, false, kW, tile_rows, w, nend, w0, w1);
                if (s0 * nom >= nend) continue;   // the kernel guesses only while j0 < nend
                // The clamp is monotone, so the tile's first and last rows bound all of them.
                for (int r : {w0, w0 + tile_rows - 1}) {
                    int row = r < w1 - 1 ? r : w1 - 1;
                    row = row > 0 ? row : 0;
                    const long long krow = (long long)bh0 * maxT + row;
                    check(row < maxT && krow < (long long)BNH * maxT, "guessed K/V row outside the cache", bh0, row, maxT);
                }
            }
            const int b0 = BNH == NH ? 0 : bh0 / NH;
            const long long qrow = ((long long)b0 * 3 * NH + (bh0 - b0 * NH)) * kCh;
            check(qrow + kCh - 1 < (long long)B * 3 * NH * kCh, "q row outside qkv", b0, bh0, NH);
        }
    }
    for (long long i = 0; i < slots; ++i) check(seen[i] == 1, "slot not taken exactly once", BNH, S, i);
}

static void check_grids(const Decode& d) {
    const int Bs[] = {1, 2, 3, 17};
    for (int B : Bs)
        for (int NH = 1; NH <= 40; ++NH)
            for (int S = 1; S <= 64; ++S) {
                if (g_quiet && g_fail) return;   // a planted mistake: one failure is enough
                const int maxT = S * 128 - (S > 1 ? 37 : 0);   // the last segment's window clipped
                check_grid(d, B, NH, S, maxT, 128, 32);
            }
}

// ---------------------------------------------------------------------------------------
// Workspace layouts.
// ---------------------------------------------------------------------------------------
struct Region {
    size_t lo, hi;
};
static bool overlap(Region a, Region b) { return a.lo < b.hi && b.lo < a.hi; }

static void regions(const WsLayout& l, long long heads, long long S, Region& ctr, Region& parts, Region& tags) {
    const size_t slots = (size_t)heads * S;
    ctr = {l.counters, l.counters + heads * 4};
    parts = {l.part_max, l.part_out + slots * kCh * 4};
    tags = {l.tag_ml, l.tag_out + slots * kCh * 8};
}

typedef WsLayout (*LayoutFn)(long long heads, long long S, size_t avail);
static WsLayout real_layout(long long heads, long long S, size_t avail) { return ws_layout(heads, S, avail); }
// Planted: a counter region sized by the plan (the layout before), not by the buffer.
static WsLayout planted_layout(long long heads, long long S, size_t avail) {
    WsLayout w = ws_layout(heads, S, avail);
    const size_t own = ws_align((size_t)heads * 4);
    const long long shift = (long long)own - (long long)w.counter_bytes;
    w.counter_bytes = own;
    w.part_max += shift;
    w.part_lse += shift;
    w.part_out += shift;
    w.bytes += shift;
    return w;
}

static void check_one_layout(LayoutFn f, long long heads, long long S, size_t avail) {
    const WsLayout l = f(heads, S, avail);
    check(l.bytes <= avail, "plan does not fit a buffer of the reported size", heads, S, (long long)avail);
    Region c, p, t;
    regions(l, heads, S, c, p, t);
    check(l.counters == kWsStatusBytes && c.hi <= l.counters + l.counter_bytes, "counters", heads, S, (long long)avail);
    check(l.part_max >= l.counters + l.counter_bytes && p.hi <= t.lo && t.hi <= avail, "regions out of order",
          heads, S, (long long)avail);
    check(l.part_max % 256 == 0 && l.part_out % 256 == 0 && l.tag_ml % 256 == 0 && l.tag_out % 256 == 0,
          "region alignment", heads, S, (long long)avail);
}

static void check_layouts(LayoutFn f) {
    const long long heads_list[] = {1, 2, 12, 24, 63, 64, 65, 96, 768, 1000, 16384};
    const long long S_list[] = {1, 2, 8, 9, 16, 64, 128};
    for (long long H : heads_list)
        for (long long S : S_list) {
            if (g_quiet && g_fail) return;
            if (H * S > (1ll << 22)) continue;
            const size_t X = ws_layout(H, S, 0).bytes;
            for (size_t extra = 0; extra < 4096; extra += 4) check_one_layout(f, H, S, X + extra);
            for (size_t extra = 4096; extra < (size_t)64 << 20; extra = extra * 3 + 1) check_one_layout(f, H, S, X + extra);
        }
    // Two plans on one buffer sized for the larger: the second plan's counters and tags never
    // sit on the first plan's partials, and its counters never on the first plan's tags.
    for (long long H1 : heads_list)
        for (long long S1 : S_list)
            for (long long H2 : heads_list)
                for (long long S2 : S_list) {
                    if (H1 * S1 > (1ll << 20) || H2 * S2 > (1ll << 20)) continue;
                    const size_t X1 = ws_layout(H1, S1, 0).bytes, X2 = ws_layout(H2, S2, 0).bytes;
                    for (size_t extra : {(size_t)0, (size_t)1000, (size_t)123456}) {
                        const size_t avail = (X1 > X2 ? X1 : X2) + extra;
                        const WsLayout a = f(H1, S1, avail), b = f(H2, S2, avail);
                        if (a.bytes > avail || b.bytes > avail) continue;
                        Region ca, pa, ta, cb, pb, tb;
                        regions(a, H1, S1, ca, pa, ta);
                        regions(b, H2, S2, cb, pb, tb);
                        check(!overlap(cb, pa) && !overlap(cb, ta), "counters on another plan's partials or tags",
                              H1 * 1000 + S1, H2 * 1000 + S2, (long long)avail);
                        check(!overlap(tb, pa), "tags on another plan's partials", H1 * 1000 + S1, H2 * 1000 + S2,
                              (long long)avail);
                    }
                }
}

int main() {
    for (int d = 1; d <= 130; ++d)
        for (int x = 0; x <= 20000; x += (x < 600 ? 1 : 37))
            check(div_uniform(x, d) == x / d, "div_uniform", x, d, div_uniform(x, d));
    const int heads_list[] = {1, 2, 7, 8, 9, 12, 16, 17, 24, 40, 96, 192, 768};
    const int seg_list[] = {1, 2, 3, 4, 6, 8, 16, 33, 64};
    for (int heads : heads_list) {
        if (heads < 8) continue;   // below 8 heads the grid keeps the dense order
        for (int S : seg_list) {
            const int grid = 8 * ((heads + 7) / 8) * S;
            std::vector<int> seen(heads * S, 0), xcd(heads, -1);
            for (int x = 0; x < grid; ++x) {
                const int v = xcd_slot(x, S);
                if (!check(v >= 0 && v < grid, "slot out of the grid", heads, S, x)) continue;
                const int bh = v / S, s = v % S;
                if (bh >= heads) continue;   // padding: the kernel's slot exits
                check(seen[bh * S + s]++ == 0, "slot taken twice", heads, S, x);
                if (xcd[bh] < 0) xcd[bh] = x & 7;
                else check(xcd[bh] == (x & 7), "head spans two XCDs", heads, S, x);
            }
            for (int i = 0; i < heads * S; ++i) check(seen[i] != 0, "slot never taken", heads, S, i);
        }
    }
    check_grids(Decode{real_slot, real_guess});
    check_layouts(real_layout);
    if (g_fail) {
        std::printf("%d failures\n", g_fail);
        return 1;
    }
    // Planted mistakes must be caught.
    g_quiet = true;
    check_grids(Decode{planted_slot, real_guess});
    const int f1 = g_fail;
    g_fail = 0;
    check_grids(Decode{real_slot, planted_guess});
    const int f2 = g_fail;
    g_fail = 0;
    check_layouts(planted_layout);
    const int f3 = g_fail;
    g_fail = 0;
    g_quiet = false;
    if (!f1 || !f2 || !f3) {
        std::printf("FAIL planted mistakes not caught: one-sequence shortcut %d, guess guard %d, plan-sized counters %d\n",
                    f1, f2, f3);
        return 1;
    }
    std::printf("ok\n");
    return 0;
}
