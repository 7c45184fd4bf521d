// layout.hpp -- integer helpers of the grid layout, shared by the kernels (device) and by
// host code that checks the layout (built with a plain C++ compiler as well).
#pragma once

#if defined(__HIPCC__)
#define KVATTN_LAYOUT_FN __host__ __device__ __forceinline__
#else
#define KVATTN_LAYOUT_FN inline
#endif

namespace kvattn_layout {

// x / d for x >= 0 and a wave-uniform d > 0: a shift when d is a power of two (the planned
// segment counts are), else the division.  Integer division by a run-time value expands to
// ~25 instructions, which at kernel start delay the first K/V request.
KVATTN_LAYOUT_FN int div_uniform(int x, int d) {
    return (d & (d - 1)) == 0 ? x >> __builtin_ctz((unsigned)d) : x / d;
}

// XCD placement.  The hardware hands consecutive workgroups of a dispatch to the 8 XCDs in
// turn (workgroup x to XCD (x + c) % 8, c fixed per dispatch), so workgroups x and x + 8
// share an XCD.  With groups of S consecutive logical workgroups that must share an XCD,
// workgroup x takes logical index xcd_slot(x, S): member s of group 8k + r is workgroup
// 8 (S k + s) + r.  A grid of 8 * ceil(groups / 8) * S covers every group.
KVATTN_LAYOUT_FN int xcd_slot(int x, int S) {
    const int r = x & 7, j = x >> 3;
    const int k = div_uniform(j, S), s = j - k * S;
    return ((k << 3) + r) * S + s;
}

}  // namespace kvattn_layout
