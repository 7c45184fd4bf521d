// Host check of the grid layout helpers the kernels use (csrc/layout.hpp): div_uniform
// against integer division, and the XCD-local designated grid (xcd_slot over a grid padded
// to whole rounds of 8 heads) as a bijection onto the real (head, segment) slots with
// every segment of a head on one XCD, whatever XCD the dispatch starts on.  Prints "ok".
#include <cstdio>
#include <vector>

#include "layout.hpp"

using kvattn_layout::div_uniform;
using kvattn_layout::xcd_slot;

static int fail(const char* what, int a, int b, int c) {
    std::printf("FAIL %s (%d, %d, %d)\n", what, a, b, c);
    return 1;
}

int main() {
    for (int d = 1; d <= 130; ++d)
        for (int x = 0; x <= 20000; x += (x < 600 ? 1 : 37))
            if (div_uniform(x, d) != x / d) return fail("div_uniform", x, d, div_uniform(x, d));
    const int heads_list[] = {1, 2, 7, 8, 9, 12, 16, 17, 24, 40, 96, 192, 768};
    const int seg_list[] = {1, 2, 3, 4, 6, 8, 16, 33, 64};
    for (int heads : heads_list) {
        if (heads < 8) continue;   // below 8 heads the grid keeps the dense order
        for (int S : seg_list) {
            const int grid = 8 * ((heads + 7) / 8) * S;
            std::vector<int> seen(heads * S, 0), xcd(heads, -1);
            for (int x = 0; x < grid; ++x) {
                const int v = xcd_slot(x, S);
                if (v < 0 || v >= grid) return fail("slot out of the grid", heads, S, x);
                const int bh = v / S, s = v % S;
                if (bh >= heads) continue;   // padding: the kernel's slot exits
                if (seen[bh * S + s]++) return fail("slot taken twice", heads, S, x);
                if (xcd[bh] < 0) xcd[bh] = x & 7;
                else if (xcd[bh] != (x & 7)) return fail("head spans two XCDs", heads, S, x);
            }
            for (int i = 0; i < heads * S; ++i)
                if (!seen[i]) return fail("slot never taken", heads, S, i);
        }
    }
    std::printf("ok\n");
    return 0;
}
