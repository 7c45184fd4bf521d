// layout.hpp -- integer helpers of the grid layout, shared by the kernels (device) and by
// host code that checks the layout (built with a plain C++ compiler as well).
#pragma once
#include <stddef.h>

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

// xcd_slot with the non-first members of each group moved `rot` XCDs on (mod 8): member
// s > 0 of group 8k + r is workgroup 8 (S k + s) + (r + rot) % 8, member 0 stays at
// 8 S k + r.  Still a bijection, and member 0 of a group still comes before its other
// members in dispatch order; with rot != 0 those members run on another XCD than member 0.
// A test setting: it puts a designated merger and its producers on different XCDs on purpose.
KVATTN_LAYOUT_FN int xcd_slot_rotated(int x, int S, int rot) {
    const int r = x & 7, j = x >> 3;
    const int k = div_uniform(j, S), s = j - k * S;
    const int rr = s == 0 ? r : ((r - rot) & 7);
    return ((k << 3) + rr) * S + s;
}

// Slot v of a dense grid of S slots per (b,h) (head bh = v / S, segment s = v % S, sequence
// b = bh / NH) of BNH = B * NH heads: false for the slots beyond the last head (b >= B),
// which a designated grid padded to whole rounds of 8 heads holds and whose workgroups must
// exit before any load.
KVATTN_LAYOUT_FN bool dense_slot(int v, int S, int BNH, int NH, int& b, int& h, int& s) {
    const int bh = v / S;
    s = v - bh * S;
    b = bh / NH;
    h = bh - b * NH;
    return bh < BNH;
}

// The speculative first tile of a slot whose head is bh0 (= v / S) is requested only for a
// real head: padding heads (bh0 >= B * NH) request nothing.
KVATTN_LAYOUT_FN bool guess_slot_live(int bh0, int BNH) { return bh0 < BNH; }

// Rows of the speculative first tile of segment s0 of a head, requested before the length is
// known: the segment's nominal rows [s0 * nom, nend), nend = min(s0 * nom + span, maxT), where
// span is nom or, for segment 0 of a device plan, the longer first share; wave `wave` of kW
// takes [w0, w1): one tile of tile_rows rows each when `first`, else an even split.  Rows are
// relative to the head's slot; every one is below maxT.
KVATTN_LAYOUT_FN void guess_rows(int s0, int nom, int span, int maxT, bool first, int kW, int tile_rows, int wave,
                                 int& nend, int& w0, int& w1) {
    const int j0 = s0 * nom;
    nend = j0 + span < maxT ? j0 + span : maxT;
    const int per = first ? tile_rows : (nend - j0 + kW - 1) / kW;
    w0 = j0 + wave * per < nend ? j0 + wave * per : nend;
    w1 = w0 + per < nend ? w0 + per : nend;
}

// ------------------------------------------------------------------------------------
// A kvattn_decode workspace (host side), every region 256-byte aligned:
//   status words (256 bytes), last-block counters (u32), part_max, part_lse (f32, one per
//   slot), part_out (64 f32 per slot), tag_ml (16 u64 per slot: the designated merger's
//   {max, exp-sum} words, one 128-byte line), tag_out (64 u64 per slot).
// One buffer may serve calls of different plans (heads = B*NH, S slots per head):
// - the counter region's size follows from the buffer's size alone (a counter for each head
//   of the largest plan the buffer can hold), so every plan finds its counters at the same
//   place, and never on another plan's partials;
// - counters and partials are laid out from the front, the tagged words from the end, so a
//   tag word never sits where another call left a float partial.
// ------------------------------------------------------------------------------------
constexpr size_t kWsStatusBytes = 256;
constexpr size_t kWsMlWords = 16;      // u64 words per slot in tag_ml
constexpr size_t kWsChannels = 64;     // head size
// Partial and tag bytes of one slot: a plan of H heads needs at least H times this much.
constexpr size_t kWsMinHeadBytes = 2 * 4 + kWsChannels * 4 + (kWsMlWords + kWsChannels) * 8;   // 904

KVATTN_LAYOUT_FN size_t ws_align(size_t x) { return (x + 255) / 256 * 256; }

// Counter bytes of a buffer of `bytes`.
KVATTN_LAYOUT_FN size_t ws_counter_bytes(size_t bytes) { return ws_align(bytes / kWsMinHeadBytes * 4); }

// Smallest buffer size reported for a plan whose status words, partials and tags take `fixed`
// bytes: every buffer at least this large holds them beside its own counter region, since
// ws_counter_bytes(x) <= 4 x / 904 + 255, and x - 4 x / 904 - 255 >= fixed once
// x >= (fixed + 255) * 904 / 900.
KVATTN_LAYOUT_FN size_t ws_sized_for(size_t fixed) {
    return ws_align(((fixed + 255) * kWsMinHeadBytes + kWsMinHeadBytes - 5) / (kWsMinHeadBytes - 4));
}

struct WsLayout {
    size_t counters, part_max, part_lse, part_out, tag_ml, tag_out;   // byte offsets
    size_t counter_bytes;
    size_t bytes;   // what the plan needs of the buffer (the size query: the size to allocate)
};

// Layout of a plan of `heads` heads and S slots in a buffer of `avail` bytes (0: the size
// query, a buffer exactly as large as reported).  The plan fits iff bytes <= avail.
// fixed_counters > 0: a counter region of that size whatever the buffer's (the static
// scratch array, whose plans are limited to that many counters).
KVATTN_LAYOUT_FN WsLayout ws_layout(long long heads, long long S, size_t avail, size_t fixed_counters = 0) {
    const size_t slots = (size_t)heads * (size_t)S;
    const size_t nm = ws_align(slots * 4), no = ws_align(slots * kWsChannels * 4);
    const size_t ntm = ws_align(slots * kWsMlWords * 8), nto = ws_align(slots * kWsChannels * 8);
    const size_t body = 2 * nm + no + ntm + nto;
    const size_t reported =
        fixed_counters ? kWsStatusBytes + fixed_counters + body : ws_sized_for(kWsStatusBytes + body);
    const bool query = avail == 0;
    if (query) avail = reported;
    WsLayout w;
    w.counters = kWsStatusBytes;
    w.counter_bytes = fixed_counters ? fixed_counters : ws_counter_bytes(avail);
    const size_t head = kWsStatusBytes + w.counter_bytes;
    w.part_max = head;
    w.part_lse = head + nm;
    w.part_out = head + 2 * nm;
    // The tags end at the last 256-byte boundary of the buffer, or right after the partials
    // when the buffer is too small (then bytes > avail and the call is refused).
    const size_t end = avail >= head + body ? avail / 256 * 256 : head + body;
    w.tag_out = end - nto;
    w.tag_ml = end - nto - ntm;
    w.bytes = query ? reported : head + body;
    return w;
}

}  // namespace kvattn_layout
