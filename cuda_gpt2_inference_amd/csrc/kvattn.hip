// kvattn.hip -- decode-phase KV-cache attention for MI355X (gfx950, CDNA4, wave64).
//
// One head row (hs = 64 elements) is spread over the lanes of one 64-lane wavefront so
// that every lane issues one 16-byte load per row chunk:
//   FP32 row = 256 B -> 16 lanes per row, 4 rows per wave load instruction
//   BF16 row = 128 B ->  8 lanes per row, 8 rows per wave load instruction
//   8-bit row = 64 B ->  4 lanes per row, 16 rows per wave load instruction
// A lane keeps the q values of its own channel slice in registers, forms a partial dot
// product, and the lanes of a row finish it with DPP row permutations.  V rows use the
// same lane mapping, so each lane accumulates its channel slice of the weighted V sum;
// the slices of different rows are combined once per segment.  Everything is bandwidth
// bound (1 flop per BF16 byte), so no matrix cores are involved.
//
// Strategies (host side at the bottom of this file):
//   fused_single     one workgroup per (b,h); when every wave holds one tile the scores
//                    stay in registers, otherwise they are staged in LDS, then a V pass
//                    with the exact maximum (reference strategy 1)
//   split            one workgroup per (b,h,segment); per-lane-group online softmax
//                    (m, l, acc) in base 2, then a workgroup merge into the reference's
//                    partial format (max in natural-log units, exp-sum, weighted V sum)
//   merge            one wave per (b,h) combining the segment partials
//   split+lastblock  split whose last finishing segment of a (b,h) merges; partials travel
//                    through coherent (sc1) stores and loads and a counter atomic; one
//                    ordinary, graph-capturable launch
//   split+coop       split + grid barrier + merge by segment 0 (cooperative launch)
//   split+graph      split and merge kernel nodes in a hipGraph, one hipGraphLaunch
// Workgroup size and tile depth are template parameters (the "latency" and "streaming"
// shapes picked per call by the host plan; both are 4 waves in this build).
#include <hip/hip_runtime.h>

#include <float.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>

#include "kvattn.h"
#include "lanes.hpp"

namespace {

constexpr int kHeadDim = 64;
constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kQScale = 0.125f * kLog2e;   // 1/sqrt(hs) * log2(e) for hs = 64 (exact: 0.125 = 2^-3)
constexpr float kLn2 = 0.69314718055994531f;
constexpr float kEmptyMax = -FLT_MAX;   // max of an empty segment (reference sentinel)
constexpr float kStartMax = -1.0e30f;   // finite start value of every running max
constexpr int kMinSegRows = 64;         // smallest automatic segment length
constexpr int kMaxSegRows = 512;        // largest automatic segment length up to kMaxMergeSegments segments
constexpr int kMaxMergeSegments = 64;   // beyond that many 512-row segments (AUTO's hinted and device plans), rows grow
constexpr int kFusedMaxRows = 256;      // automatic plans keep up to this many positions in one workgroup
constexpr int kStridedMaxSeqs = 256;    // ragged batches up to this size take the strided grid
constexpr int kStridedFactor = 2;       // segments per workgroup bound of the strided grid
constexpr int kMaxPagedSegRows = 4096;  // paged caches: at most 64 tiles per wave and segment
constexpr int kMaxSegments = 1 << 16;   // upper bound on segments per (b,h)
constexpr int kMaxT = 1 << 23;          // keeps per-slot byte offsets inside 32 bits
constexpr size_t kFusedMaxLds = 64 * 1024;  // dynamic LDS of fused_single (scores)
constexpr int kMaxDesignatedSegments = 64;  // the designated merger follows one segment per lane
// Workspace status words (the first 256 bytes of a kvattn_decode workspace).
constexpr int kWsStatusMergeTimeouts = 0;   // merges that stopped waiting (a sticky count)
constexpr int kWsStatusBarrier = 2;         // u64 {generation, count} of the cooperative grid barrier
// Designated producers of an XCD-local grid that published write-through because their
// merger's XCD word named another XCD (a count), or was not there yet when they looked.
constexpr int kWsStatusXcdRemote = 4;
constexpr int kWsStatusXcdUnseen = 5;
constexpr size_t kWsStatusBytes = 256;

// ------------------------------------------------------------------------------------
// Per-dtype row geometry.
// ------------------------------------------------------------------------------------
template <int DT> struct Row;
template <> struct Row<KVATTN_KV_F32> {
    static constexpr int kLanes = 16, kElems = 4, kBytes = 256;
    static constexpr bool k8bit = false, kActF32 = true;
};
template <> struct Row<KVATTN_KV_BF16> {
    static constexpr int kLanes = 8, kElems = 8, kBytes = 128;
    static constexpr bool k8bit = false, kActF32 = false;
};
template <> struct Row<KVATTN_KV_INT8> {
    static constexpr int kLanes = 4, kElems = 16, kBytes = 64;
    static constexpr bool k8bit = true, kActF32 = false;
};
template <> struct Row<KVATTN_KV_FP8_E4M3> {
    static constexpr int kLanes = 4, kElems = 16, kBytes = 64;
    static constexpr bool k8bit = true, kActF32 = false;
};
template <int DT> constexpr int kRowsPerLoad = kWave / Row<DT>::kLanes;
// Row chunks per lane and tile in the unrolled main loops (8-bit rows are 4x denser).
#ifndef KVATTN_UNROLL_WIDE
#define KVATTN_UNROLL_WIDE 8
#endif
#ifndef KVATTN_UNROLL_BYTE
#define KVATTN_UNROLL_BYTE 4
#endif
template <int DT> constexpr int kUnroll = Row<DT>::k8bit ? KVATTN_UNROLL_BYTE : KVATTN_UNROLL_WIDE;
// Latency-bound calls (the "latency" shape) take KVATTN_LAT_ROWS rows per wave per tile, so
// that a GPT-2 head of up to 256 positions is one tile per wave of a 4-wave workgroup.
#ifndef KVATTN_LAT_WAVES
#define KVATTN_LAT_WAVES 4
#endif
#ifndef KVATTN_LAT_ROWS
#define KVATTN_LAT_ROWS 64
#endif
template <int DT> constexpr int kUnrollLat = KVATTN_LAT_ROWS / kRowsPerLoad<DT> > 0 ? KVATTN_LAT_ROWS / kRowsPerLoad<DT> : 1;
constexpr int kWavesLat = KVATTN_LAT_WAVES;
// fused_single: a head of up to kFusedMaxRows positions is one tile per wave.  A wave's
// arithmetic over its tile is the call's critical path while the heads leave CUs idle, and a
// 4-wave workgroup puts one wave on each SIMD of its CU.  So:
// - Hinted lengths up to 128 (the longest, with per-sequence lengths) take 4 waves of 32-row
//   tiles (every wave holds rows).  Measured
//   (12 calls per graph, B·NH from 12 to 768): 10-17 % faster than 4 waves of 64-row tiles at
//   12-96 heads, 10-33 % at 384-768 heads.
// - Otherwise FP32 rows, the widest (four lanes' arithmetic per row of bf16), take 8 waves of
//   32-row tiles up to 256 heads (12-layer graphs, A/B both orders: -0.15 us at 256 positions
//   against 4 × 64; INT8 +0.23 and BF16 within ±0.04 with 8 × 32), and 4 waves of 64-row tiles
//   beyond: once the heads outnumber the CUs, the 8-wave workgroups lose 9-21 % (B·NH from 288
//   to 768, 160-256 positions).  The other caches take 4 waves of KVATTN_LAT_ROWS-row tiles.
template <int DT> constexpr int kFusedWaves = DT == KVATTN_KV_F32 ? 8 : KVATTN_LAT_WAVES;
template <int DT> constexpr int kFusedRows = DT == KVATTN_KV_F32 ? 32 : KVATTN_LAT_ROWS;
constexpr int kFusedShortWaves = 4;
constexpr int kFusedShortRows = 32;
constexpr int kFusedF32WideRows = 64;
constexpr long long kFusedF32WideHeads = 256;   // B * NH beyond which FP32 takes 4 waves of 64-row tiles
template <int DT> constexpr int unroll_for(int rows) {
    return rows / kRowsPerLoad<DT> > 0 ? rows / kRowsPerLoad<DT> : 1;
}
// The split kernels' latency shape takes KVATTN_SPLIT_LAT_ROWS rows per wave per tile: a
// 128-row designated segment is then one full tile per wave of a 4-wave workgroup.  Each
// tile's arithmetic runs over all its row slots, valid or masked, and at GPT-2's sizes it is
// on the call's critical path: 64-row tiles, half of them masked, cost C2 0.24 µs per call.
// The device-planned designated instance takes them too: its segment 0, up to kFusedMaxRows
// rows, gives each wave up to two tiles, both requested before the first is consumed.
#ifndef KVATTN_SPLIT_LAT_ROWS
#define KVATTN_SPLIT_LAT_ROWS 32
#endif
template <int DT> constexpr int kUnrollSplitLat =
    KVATTN_SPLIT_LAT_ROWS / kRowsPerLoad<DT> > 0 ? KVATTN_SPLIT_LAT_ROWS / kRowsPerLoad<DT> : 1;

// Decode one lane's 16-byte chunk of a row into kElems floats.
template <int DT>
__device__ __forceinline__ void decode(const uint4& d, float (&x)[Row<DT>::kElems]) {
    const uint32_t w[4] = {d.x, d.y, d.z, d.w};
    if constexpr (DT == KVATTN_KV_F32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = __uint_as_float(w[i]);
    } else if constexpr (DT == KVATTN_KV_BF16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) { x[2 * i] = bf16_lo(w[i]); x[2 * i + 1] = bf16_hi(w[i]); }
    } else {
        decode_codes<DT == KVATTN_KV_FP8_E4M3>(d, x);
    }
}

// A lane's share of a score: q slice . row chunk.  kHw (the latency-bound kernels): BF16
// rows take the hardware bf16 dot (v_dot2_f32_bf16: two bf16 products, exact in fp32, added
// to an fp32 accumulator) on the packed q pairs that convert_q<DT, true> leaves in q[0..3],
// then the scale in q[4].  The streaming kernel keeps the fma form: measured, the dot costs
// its 64-sequence call 2 % (A/B, both the one-chain and the two-chain form).
typedef __bf16 Bf16x2 __attribute__((ext_vector_type(2)));
template <int DT, bool kHw = false>
__device__ __forceinline__ float dot_chunk(const float (&q)[Row<DT>::kElems], const uint4& d) {
    if constexpr (kHw && DT == KVATTN_KV_BF16) {
        auto pair = [](uint32_t u) { return __builtin_bit_cast(Bf16x2, u); };
        auto qp = [&](int i) { return pair(__float_as_uint(q[i])); };
        float s = __builtin_amdgcn_fdot2_f32_bf16(pair(d.x), qp(0), 0.0f, false);
        s = __builtin_amdgcn_fdot2_f32_bf16(pair(d.y), qp(1), s, false);
        s = __builtin_amdgcn_fdot2_f32_bf16(pair(d.z), qp(2), s, false);
        s = __builtin_amdgcn_fdot2_f32_bf16(pair(d.w), qp(3), s, false);
        return s * q[4];
    } else {
        float x[Row<DT>::kElems];
        decode<DT>(d, x);
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < Row<DT>::kElems; ++e) s = fmaf(q[e], x[e], s);
        return s;
    }
}

// Attended positions of sequence b: device length clamped to [0, maxT-1], plus one.
__device__ __forceinline__ int seq_total(const int* cur_len, int lens_per_seq, int b, int maxT) {
    int cl = cur_len[lens_per_seq ? b : 0];
    cl = cl < 0 ? 0 : (cl > maxT - 1 ? maxT - 1 : cl);
    return cl + 1;
}

// seq_total for a wave-uniform b, read with a scalar load: the lengths are written by earlier
// dispatches or the host, never during a launch, so the constant address space applies.  A
// scalar load is waited for on its own counter, so waiting for the length does not wait for
// the vector loads (K/V tiles, q) or stores issued before it, as it would on the in-order
// vector memory counter.
typedef const __attribute__((address_space(4))) int* ConstIntPtr;
__device__ __forceinline__ int seq_total_uniform(const int* cur_len, int lens_per_seq, int b, int maxT) {
    int cl = ((ConstIntPtr)cur_len)[lens_per_seq ? b : 0];
    cl = cl < 0 ? 0 : (cl > maxT - 1 ? maxT - 1 : cl);
    return cl + 1;
}

// This lane's q slice (channels slice*kElems ..) as raw bytes: 16 bytes, or 32 for the
// 8-bit caches whose lanes cover 16 bf16 channels.  Converting is deferred until the first
// K/V tile has been requested so that the q load and the K/V loads overlap.
template <int DT> struct QRaw {
    uint4 w[Row<DT>::k8bit ? 2 : 1];
};

template <int DT>
__device__ __forceinline__ QRaw<DT> load_q(const void* qkv, int b, int h, int NH, int slice) {
    constexpr int kActBytes = Row<DT>::kActF32 ? 4 : 2;
    const size_t q0 = (((size_t)b * 3 * NH + h) * kHeadDim + (size_t)slice * Row<DT>::kElems) * kActBytes;
    const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(qkv) + q0);
    QRaw<DT> r;
#pragma unroll
    for (int i = 0; i < (Row<DT>::k8bit ? 2 : 1); ++i) r.w[i] = p[i];
    return r;
}

// q as float, multiplied by scale*log2(e) so dot products come out in base-2 units.  With
// kHw, BF16 caches keep q as the raw packed bf16 pairs in q[0..3] (bit patterns) and the
// scale in q[4]: dot_chunk<DT, true> takes the hardware bf16 dot and scales the lane's sum.
template <int DT, bool kHw = false>
__device__ __forceinline__ void convert_q(const QRaw<DT>& r, float qscale, float (&q)[Row<DT>::kElems]) {
    if constexpr (kHw && DT == KVATTN_KV_BF16) {
        q[0] = __uint_as_float(r.w[0].x);
        q[1] = __uint_as_float(r.w[0].y);
        q[2] = __uint_as_float(r.w[0].z);
        q[3] = __uint_as_float(r.w[0].w);
        q[4] = qscale;
        q[5] = q[6] = q[7] = 0.0f;
    } else if constexpr (Row<DT>::kActF32) {
        q[0] = __uint_as_float(r.w[0].x) * qscale;
        q[1] = __uint_as_float(r.w[0].y) * qscale;
        q[2] = __uint_as_float(r.w[0].z) * qscale;
        q[3] = __uint_as_float(r.w[0].w) * qscale;
    } else {
#pragma unroll
        for (int i = 0; i < (Row<DT>::k8bit ? 2 : 1); ++i) {
            const uint32_t w[4] = {r.w[i].x, r.w[i].y, r.w[i].z, r.w[i].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                q[8 * i + 2 * k] = bf16_lo(w[k]) * qscale;
                q[8 * i + 2 * k + 1] = bf16_hi(w[k]) * qscale;
            }
        }
    }
}

template <int DT>
__device__ __forceinline__ void store_out(void* out, size_t i, float v) {
    if constexpr (Row<DT>::kActF32) reinterpret_cast<float*>(out)[i] = v;
    else reinterpret_cast<uint16_t*>(out)[i] = f32_to_bf16(v);
}

// Byte pointers of one (b,h) cache slot, already offset to this lane's 16-byte slice.
struct Slot {
    const uint8_t* k;
    const uint8_t* v;
    const float* ks;   // row scales (8-bit) or nullptr
    const float* vs;
};

template <int DT>
__device__ __forceinline__ Slot make_slot(const uint8_t* kv, const float* kv_scale, int B, int NH,
                                          int maxT, int bh, int slice) {
    const size_t rows = (size_t)B * NH * maxT;
    const size_t base = (size_t)bh * maxT;
    Slot s;
    s.k = kv + base * Row<DT>::kBytes + slice * 16;
    s.v = kv + (rows + base) * Row<DT>::kBytes + slice * 16;
    s.ks = Row<DT>::k8bit ? kv_scale + base : nullptr;
    s.vs = Row<DT>::k8bit ? kv_scale + rows + base : nullptr;
    return s;
}

// ------------------------------------------------------------------------------------
// The current token's K and V rows, for the kernels that append and attend in one launch.
// Every lane loads its own channel slice from qkv (like q); the slice is brought to the
// cache format (8-bit: row amax over the 4 lanes of the row, then the append's
// quantisation), written to column cur_len by one row group of the owning workgroup, and
// substituted for the cache row in the tile that holds position cur_len, so no workgroup
// reads that cache row.
// ------------------------------------------------------------------------------------
template <int DT> struct FreshRaw {
    uint4 k[Row<DT>::k8bit ? 2 : 1], v[Row<DT>::k8bit ? 2 : 1];
};
template <int DT> struct Fresh {
    uint4 k, v;        // this lane's 16-byte slice of the K and V rows, cache format
    float ks, vs;      // 8-bit row scales
};

template <int DT>
__device__ __forceinline__ FreshRaw<DT> load_fresh(const void* qkv, int b, int h, int NH, int slice) {
    constexpr int kActBytes = Row<DT>::kActF32 ? 4 : 2;
    constexpr int kN = Row<DT>::k8bit ? 2 : 1;
    const uint8_t* base = reinterpret_cast<const uint8_t*>(qkv);
    const size_t off = (size_t)slice * Row<DT>::kElems * kActBytes;
    const uint4* pk = reinterpret_cast<const uint4*>(base + (((size_t)b * 3 + 1) * NH + h) * kHeadDim * kActBytes + off);
    const uint4* pv = reinterpret_cast<const uint4*>(base + (((size_t)b * 3 + 2) * NH + h) * kHeadDim * kActBytes + off);
    FreshRaw<DT> r;
#pragma unroll
    for (int i = 0; i < kN; ++i) { r.k[i] = pk[i]; r.v[i] = pv[i]; }
    return r;
}

// 16 bf16 channels -> 16 codes of one row whose other 48 channels sit in the other three
// lanes of this lane's quad.
template <int DT>
__device__ __forceinline__ uint4 quantise_slice(const uint4 (&w)[2], float& scale) {
    float x[16];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t u[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            x[8 * i + 2 * k] = bf16_lo(u[k]);
            x[8 * i + 2 * k + 1] = bf16_hi(u[k]);
        }
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(x[e]));
    amax = fmaxf(amax, dpp<kDppQuadXor1>(amax));
    amax = fmaxf(amax, dpp<kDppQuadXor2>(amax));
    scale = amax / kW8Limit<DT>;
    uint32_t c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        c[i] = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) c[i] |= (uint32_t)w8_code<DT>(x[4 * i + k], scale) << (8 * k);
    }
    return make_uint4(c[0], c[1], c[2], c[3]);
}

template <int DT>
__device__ __forceinline__ Fresh<DT> finish_fresh(const FreshRaw<DT>& r) {
    Fresh<DT> f;
    if constexpr (Row<DT>::k8bit) {
        f.k = quantise_slice<DT>(r.k, f.ks);
        f.v = quantise_slice<DT>(r.v, f.vs);
    } else {
        f.k = r.k[0];
        f.v = r.v[0];
        f.ks = f.vs = 0.0f;
    }
    return f;
}

// Where the fresh row goes: column `cur` of slot bh.
struct FreshDst {
    uint8_t* kv;
    float* kv_scale;
    size_t rk, rv;     // cache row indices of the K and V rows
    int slice;
};

__device__ __forceinline__ FreshDst fresh_dst(uint8_t* kv, float* kv_scale, int B, int NH, int maxT, int bh,
                                              int slice, int cur) {
    FreshDst d;
    d.kv = kv;
    d.kv_scale = kv_scale;
    d.rk = (size_t)bh * maxT + cur;
    d.rv = (size_t)B * NH * maxT + d.rk;
    d.slice = slice;
    return d;
}

// This lane's K and V slices of the row, and (slice 0) the row scales.
template <int DT>
__device__ __forceinline__ void store_fresh(const FreshDst& d, const Fresh<DT>& f) {
    *reinterpret_cast<uint4*>(d.kv + d.rk * Row<DT>::kBytes + d.slice * 16) = f.k;
    *reinterpret_cast<uint4*>(d.kv + d.rv * Row<DT>::kBytes + d.slice * 16) = f.v;
    if constexpr (Row<DT>::k8bit) {
        if (d.slice == 0) { d.kv_scale[d.rk] = f.ks; d.kv_scale[d.rv] = f.vs; }
    }
}

// ------------------------------------------------------------------------------------
// Online softmax over rows [r0, r1) of a slot by one wave.  Each group of kLanes lanes
// owns one row per load instruction and keeps its own running (m, l, acc) in base-2
// units; the groups are combined later.  A tile holds U K and U V row chunks per lane,
// all requested before any of them is used.
// ------------------------------------------------------------------------------------
template <int DT, int U>
struct Tile {
    uint4 k[U], v[U];
    float ks[U], vs[U];
};

// kChecked (a wave's first and last tile, which may reach past the rows it owns): every row
// slot is loaded unconditionally, rows at or beyond r1 clamped to r1 - 1 (r1 is at most the
// slot's maxT, and at least 1), so no load sits behind a branch and all of them issue back
// to back.  Those rows hold another row's data: consume_tile<kChecked>, and fused_single's
// one-tile path, mask them by selection (score -inf, V chunk and V scale zero).
template <int DT, int U, bool kChecked>
__device__ __forceinline__ void load_tile(Tile<DT, U>& t, const Slot& sl, int r, int r1, int slot_row) {
    using R = Row<DT>;
    constexpr int kRPL = kRowsPerLoad<DT>;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        int row = r + u * kRPL + slot_row;
        if (kChecked) row = max(min(row, r1 - 1), 0);
        t.k[u] = load16(sl.k + (uint32_t)row * R::kBytes);
        t.v[u] = load16(sl.v + (uint32_t)row * R::kBytes);
        if constexpr (R::k8bit) { t.ks[u] = sl.ks[row]; t.vs[u] = sl.vs[row]; }
    }
    // INT8 full tiles (the walk past a segment's first tile): keep every load of the tile
    // ahead of its use.  The INT8 decode (a convert per byte) widens each 16-byte chunk into
    // 16 live floats, and to save registers the scheduler otherwise sinks each load to its
    // converts with a full wait in between: one memory round trip per chunk instead of one
    // per tile (measured: INT8 segments of several tiles per wave 8-49 % slower).
    if constexpr (DT == KVATTN_KV_INT8 && !kChecked) __builtin_amdgcn_sched_barrier(0);
}

// In a tile whose rows start at r: the lanes holding row `cur` take the fresh row in place
// of what they loaded from the cache and write it to the cache.
template <int DT, int U>
__device__ __forceinline__ void patch_tile(Tile<DT, U>& t, const FreshRaw<DT>& fr, const FreshDst& d, int r,
                                           int slot_row, int cur) {
    constexpr int kRPL = kRowsPerLoad<DT>;
    const Fresh<DT> f = finish_fresh<DT>(fr);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (r + u * kRPL + slot_row == cur) {
            t.k[u] = f.k;
            t.v[u] = f.v;
            if constexpr (Row<DT>::k8bit) { t.ks[u] = f.ks; t.vs[u] = f.vs; }
            store_fresh<DT>(d, f);
        }
    }
}

// Rows at or beyond r1 of a tile may hold anything: a speculative first tile is requested
// before the length is known, and a cache is never cleared past its length (NaN or Inf
// bits, FP8 NaN codes 0x7F/0xFF, garbage 8-bit scales).  Their scores are replaced by
// -inf, which makes p = 0, but 0 * NaN is NaN: so their V chunks and V scales are replaced
// by zeros as well (a select on the loaded bits), and a masked row contributes exactly
// nothing to l and acc.
template <int DT, int U>
__device__ __forceinline__ void mask_tile_v(Tile<DT, U>& t, int r, int r1, int slot_row) {
    constexpr int kRPL = kRowsPerLoad<DT>;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (r + u * kRPL + slot_row >= r1) {
            t.v[u] = make_uint4(0u, 0u, 0u, 0u);
            if constexpr (Row<DT>::k8bit) t.vs[u] = 0.0f;
        }
    }
}

template <int DT, int U, bool kChecked, bool kHw = false>
__device__ __forceinline__ void consume_tile(const Tile<DT, U>& t, int r, int r1, int slot_row,
                                             const float (&q)[Row<DT>::kElems], float& m, float& l,
                                             float (&acc)[Row<DT>::kElems]) {
    using R = Row<DT>;
    constexpr int kRPL = kRowsPerLoad<DT>;
    float s[U];
    float mt = m;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        s[u] = row_sum<R::kLanes>(dot_chunk<DT, kHw>(q, t.k[u]));
        if constexpr (R::k8bit) s[u] *= t.ks[u];
        if (kChecked && r + u * kRPL + slot_row >= r1) s[u] = -INFINITY;
        mt = fmaxf(mt, s[u]);
    }
    const float corr = exp2_fast(m - mt);
    l *= corr;
#pragma unroll
    for (int e = 0; e < R::kElems; ++e) acc[e] *= corr;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const float p = exp2_fast(s[u] - mt);
        l += p;
        const bool live = !kChecked || r + u * kRPL + slot_row < r1;
        const uint4 vd = live ? t.v[u] : make_uint4(0u, 0u, 0u, 0u);
        const float pv = R::k8bit ? p * (live ? t.vs[u] : 0.0f) : p;
        float x[R::kElems];
        decode<DT>(vd, x);
#pragma unroll
        for (int e = 0; e < R::kElems; ++e) acc[e] = fmaf(pv, x[e], acc[e]);
    }
    m = mt;
}

// Online softmax over rows [r0, r1) of a slot by one wave, given the first tile (rows
// [r0, r0 + kTile) clipped to a bound >= r1) and this lane's q slice already requested;
// rows of that tile at or beyond r1 are masked.  The q slice is requested after the tile's
// K/V loads, so nothing that depends on q is scheduled ahead of them.  kFresh: the row
// `cur` (if inside [r0, r1)) is taken from f instead of the cache.
template <int DT, int kU, bool kFresh, bool kHw = false>
__device__ __forceinline__ void online_rows_from(Tile<DT, kU>& t0, const QRaw<DT>& qr,
                                                 const Slot& sl, int r0, int r1, int slot_row, float qscale,
                                                 const FreshRaw<DT>& fr, const FreshDst& fd, int cur,
                                                 float& m, float& l, float (&acc)[Row<DT>::kElems]) {
    constexpr int kTile = kRowsPerLoad<DT> * kU;
    if (r0 >= r1) return;
    float q[Row<DT>::kElems];
    convert_q<DT, kHw>(qr, qscale, q);
    // Only the wave whose rows [r, min(r + kTile, r1)) contain cur patches (and stores).
    auto holds = [&](int r) { return kFresh && cur >= r && cur < min(r + kTile, r1); };
    if (holds(r0)) patch_tile<DT, kU>(t0, fr, fd, r0, slot_row, cur);
    consume_tile<DT, kU, true, kHw>(t0, r0, r1, slot_row, q, m, l, acc);
    Tile<DT, kU> t;
    int r = r0 + kTile;
    for (; r + kTile <= r1; r += kTile) {
        load_tile<DT, kU, false>(t, sl, r, r1, slot_row);
        if (holds(r)) patch_tile<DT, kU>(t, fr, fd, r, slot_row, cur);
        consume_tile<DT, kU, false, kHw>(t, r, r1, slot_row, q, m, l, acc);
    }
    if (r < r1) {
        load_tile<DT, kU, true>(t, sl, r, r1, slot_row);
        if (holds(r)) patch_tile<DT, kU>(t, fr, fd, r, slot_row, cur);
        consume_tile<DT, kU, true, kHw>(t, r, r1, slot_row, q, m, l, acc);
    }
}

// ------------------------------------------------------------------------------------
// Paged caches.  A page holds page_rows positions (a multiple of 64) of one sequence for
// all heads: [2][NH][page_rows] rows, K block then V block.  Tiles of kTile rows (which
// divides page_rows) start at multiples of kTile and so never cross a page; within a
// segment the waves take tiles round-robin.  Each wave loads the page ids of all its tiles
// with one vector load (lane i: tile i) before its first tile, so the table costs one
// memory round trip, not one per tile.  A page id outside [0, num_pages) is never
// dereferenced: its rows are skipped.
// ------------------------------------------------------------------------------------
struct PagedView {
    const uint8_t* pool;
    const float* scale_pool;
    const int* table;
    int max_pages, page_rows, num_pages, NH;
};

// Slot pointers of head h inside page `page` (rows counted from the page's first row).
template <int DT>
__device__ __forceinline__ Slot page_slot(const PagedView& pv, int page, int h, int slice) {
    const size_t rk = ((size_t)page * 2 * pv.NH + h) * pv.page_rows;
    const size_t rv = rk + (size_t)pv.NH * pv.page_rows;
    Slot s;
    s.k = pv.pool + rk * Row<DT>::kBytes + slice * 16;
    s.v = pv.pool + rv * Row<DT>::kBytes + slice * 16;
    s.ks = Row<DT>::k8bit ? pv.scale_pool + rk : nullptr;
    s.vs = Row<DT>::k8bit ? pv.scale_pool + rv : nullptr;
    return s;
}

// Page ids of one wave's tiles of rows [j0, j1) of sequence b: lane i gets the page of the
// wave's tile i (tiles go round-robin to the kW waves), -1 past j1.
template <int DT, int kU, int kW>
__device__ __forceinline__ int paged_tile_ids(const PagedView& pv, int b, int j0, int j1, int wave) {
    constexpr int kTile = kRowsPerLoad<DT> * kU;
    const int lane = threadIdx.x & (kWave - 1);
    const int tr = j0 + (wave + lane * kW) * kTile;     // first row of this lane's tile
    return tr < j1 ? pv.table[(size_t)b * pv.max_pages + tr / pv.page_rows] : -1;
}

// Online softmax over rows [j0, j1) of (b, h) (j0 a multiple of kTile) by one wave of kW.
// kFresh: the row `cur` is taken from fr and written through the table.
// kAhead: the wave's first two tiles are both requested before the first is consumed (the
// paged latency shape of the 8-bit caches, whose waves walk one or a few tiles).
template <int DT, int kU, int kW, bool kFresh, bool kHw = false, bool kAhead = false>
__device__ __forceinline__ void online_tiles_paged(const PagedView& pv, int b, int h, int j0, int j1, int wave,
                                                   int slot_row, int slice, const QRaw<DT>& qr, float qscale,
                                                   const FreshRaw<DT>& fr, uint8_t* kv_out, float* kv_scale_out,
                                                   int cur, float& m, float& l, float (&acc)[Row<DT>::kElems],
                                                   int pid_in = -1, bool have_pid = false) {
    constexpr int kTile = kRowsPerLoad<DT> * kU;
    const int P = pv.page_rows;
    // Lane i: the page of this wave's tile i (requested here, or earlier by the caller:
    // paged_tile_ids with the same arguments).
    const int pid = have_pid ? pid_in : paged_tile_ids<DT, kU, kW>(pv, b, j0, j1, wave);
    float q[Row<DT>::kElems];
    convert_q<DT, kHw>(qr, qscale, q);
    Tile<DT, kU> t;
    int i = 0;
    int r = j0 + wave * kTile;
    if constexpr (kAhead) {
        // Tiles 0 and 1 of the wave (rows ra and rb), each from its own page; a tile that
        // reaches j1 takes the checked loads and scores, as the walk's last tile does.
        Tile<DT, kU> t1;
        const int ra = r, rb = r + kW * kTile;
        const int pa = __shfl(pid, 0), pb = __shfl(pid, 1);
        const bool va = ra < j1 && pa >= 0 && pa < pv.num_pages;
        const bool vb = rb < j1 && pb >= 0 && pb < pv.num_pages;
        const int a0 = ra / P * P, b0 = rb / P * P;
        auto ld = [&](Tile<DT, kU>& tt, int page, int rr, int p0) {
            const Slot sp = page_slot<DT>(pv, page, h, slice);
            if (rr + kTile <= j1) load_tile<DT, kU, false>(tt, sp, rr - p0, j1 - p0, slot_row);
            else load_tile<DT, kU, true>(tt, sp, rr - p0, j1 - p0, slot_row);
        };
        if (va) ld(t, pa, ra, a0);
        if (vb) ld(t1, pb, rb, b0);
        auto take = [&](Tile<DT, kU>& tt, int page, int rr, int p0) {
            if (kFresh && cur >= rr && cur < min(rr + kTile, j1)) {
                const size_t rk = ((size_t)page * 2 * pv.NH + h) * P + (cur - p0);
                const FreshDst fd{kv_out, kv_scale_out, rk, rk + (size_t)pv.NH * P, slice};
                patch_tile<DT, kU>(tt, fr, fd, rr - p0, slot_row, cur - p0);
            }
            if (rr + kTile <= j1) consume_tile<DT, kU, false, kHw>(tt, rr - p0, j1 - p0, slot_row, q, m, l, acc);
            else consume_tile<DT, kU, true, kHw>(tt, rr - p0, j1 - p0, slot_row, q, m, l, acc);
        };
        if (va) take(t, pa, ra, a0);
        if (vb) take(t1, pb, rb, b0);
        r = rb + kW * kTile;
        i = 2;
    }
    for (; r < j1; r += kW * kTile, ++i) {
        const int page = __shfl(pid, i);
        if (page < 0 || page >= pv.num_pages) continue;
        const int pr0 = r / P * P;
        const Slot sp = page_slot<DT>(pv, page, h, slice);
        auto fresh = [&]() {
            if (kFresh && cur >= r && cur < min(r + kTile, j1)) {
                const size_t rk = ((size_t)page * 2 * pv.NH + h) * P + (cur - pr0);
                const FreshDst fd{kv_out, kv_scale_out, rk, rk + (size_t)pv.NH * P, slice};
                patch_tile<DT, kU>(t, fr, fd, r - pr0, slot_row, cur - pr0);
            }
        };
        // Full tiles take the unchecked loads and scores (no per-row conditions around the
        // loads), as the contiguous walk does; only a segment's last tile is checked.
        if (r + kTile <= j1) {
            load_tile<DT, kU, false>(t, sp, r - pr0, j1 - pr0, slot_row);
            fresh();
            consume_tile<DT, kU, false, kHw>(t, r - pr0, j1 - pr0, slot_row, q, m, l, acc);
        } else {
            load_tile<DT, kU, true>(t, sp, r - pr0, j1 - pr0, slot_row);
            fresh();
            consume_tile<DT, kU, true, kHw>(t, r - pr0, j1 - pr0, slot_row, q, m, l, acc);
        }
    }
}

// ------------------------------------------------------------------------------------
// fused_single: one workgroup per (b,h), grid B*NH.  Pass 1 writes every score to LDS
// and finds the exact maximum; pass 2 weights V with exp2(score - max).
// ------------------------------------------------------------------------------------
template <int DT, int U, bool kChecked, bool kFresh, bool kHw = false>
__device__ __forceinline__ void score_tile(const Slot& sl, int r, int total, int slot_row, int slice,
                                           const float (&q)[Row<DT>::kElems], float* scores, float& mloc,
                                           const FreshRaw<DT>& fr, const FreshDst& fd) {
    using R = Row<DT>;
    constexpr int kRPL = kRowsPerLoad<DT>;
    uint4 kd[U];
    float ks[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int row = r + u * kRPL + slot_row;
        if (!kChecked || row < total) {
            kd[u] = load16(sl.k + (uint32_t)row * R::kBytes);
            if constexpr (R::k8bit) ks[u] = sl.ks[row];
        } else {
            kd[u] = make_uint4(0u, 0u, 0u, 0u);
            if constexpr (R::k8bit) ks[u] = 0.0f;
        }
    }
    // The fresh row (position total - 1) replaces the cache row and is written out here.
    const int cur = total - 1;
    if (kFresh && cur >= r && cur < r + U * kRPL) {
        const Fresh<DT> f = finish_fresh<DT>(fr);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (r + u * kRPL + slot_row == cur) {
                kd[u] = f.k;
                if constexpr (R::k8bit) ks[u] = f.ks;
                store_fresh<DT>(fd, f);
            }
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        float s = row_sum<R::kLanes>(dot_chunk<DT, kHw>(q, kd[u]));
        if constexpr (R::k8bit) s *= ks[u];
        const int row = r + u * kRPL + slot_row;
        if (!kChecked || row < total) {
            mloc = fmaxf(mloc, s);
            if (slice == 0) scores[row] = s;
        }
    }
}

template <int DT, int U, bool kChecked, bool kFresh>
__device__ __forceinline__ void weight_tile(const Slot& sl, int r, int total, int slot_row, float M,
                                            const float* scores, float& l, float (&acc)[Row<DT>::kElems],
                                            const FreshRaw<DT>& fr) {
    using R = Row<DT>;
    constexpr int kRPL = kRowsPerLoad<DT>;
    uint4 vd[U];
    float vs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int row = r + u * kRPL + slot_row;
        if (!kChecked || row < total) {
            vd[u] = load16(sl.v + (uint32_t)row * R::kBytes);
            if constexpr (R::k8bit) vs[u] = sl.vs[row];
        } else {
            vd[u] = make_uint4(0u, 0u, 0u, 0u);
            if constexpr (R::k8bit) vs[u] = 0.0f;
        }
    }
    const int cur = total - 1;
    if (kFresh && cur >= r && cur < r + U * kRPL) {
        const Fresh<DT> f = finish_fresh<DT>(fr);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (r + u * kRPL + slot_row == cur) {
                vd[u] = f.v;
                if constexpr (R::k8bit) vs[u] = f.vs;
            }
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int row = r + u * kRPL + slot_row;
        if (!kChecked || row < total) {
            const float p = exp2_fast(scores[row] - M);
            l += p;
            const float pv = R::k8bit ? p * vs[u] : p;
            float x[R::kElems];
            decode<DT>(vd[u], x);
#pragma unroll
            for (int e = 0; e < R::kElems; ++e) acc[e] = fmaf(pv, x[e], acc[e]);
        }
    }
}

// kFresh: append and attend in one launch; kv_out / kv_scale_out receive the current
// token's row (they alias kv / kv_scale, whose row cur_len is then never used).
template <int DT, int kThreads, int kU, bool kFresh>
// Parameters in the order the first loads need them: the leading 14 dwords are preloaded
// into SGPRs at wave launch (the library is built with kernel-argument preloading).
__global__ __launch_bounds__(kThreads) void fused_single_kernel(
    const void* __restrict__ qkv, const uint8_t* kv, const int* __restrict__ cur_len, int lens_per_seq, int B,
    int NH, int maxT, int spec_rows, float qscale, const float* kv_scale, void* __restrict__ out, uint8_t* kv_out,
    float* kv_scale_out) {
    using R = Row<DT>;
    constexpr int kW = kThreads / kWave;
    constexpr int kRPL = kRowsPerLoad<DT>;
    constexpr int kTile = kRPL * kU;
    extern __shared__ float s_scores[];
    __shared__ float s_max[kW];
    __shared__ float s_l[kW];
    __shared__ float s_acc[kW][kHeadDim];

    const int bh = blockIdx.x;
    const int b = B == 1 ? 0 : bh / NH, h = bh - b * NH;   // the grid is B * NH: bh < NH when B == 1
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int slot_row = lane / R::kLanes, slice = lane % R::kLanes;
    const Slot sl = make_slot<DT>(kv, kv_scale, B, NH, maxT, bh, slice);
    // When the host's length hint fits the one-tile-per-wave shape, the tile and q are
    // requested before the device length is read (rows at or beyond it are masked later).
    const int spec_lim = min(spec_rows, maxT);
    const bool spec = spec_lim > 0 && spec_lim <= kW * kTile;
    Tile<DT, kU> t;
    QRaw<DT> qr;
    if (spec) {
        load_tile<DT, kU, true>(t, sl, wave * kTile, spec_lim, slot_row);
        qr = load_q<DT>(qkv, b, h, NH, slice);
    }
    FreshRaw<DT> fr{};
    if constexpr (kFresh) fr = load_fresh<DT>(qkv, b, h, NH, slice);
    const int total = seq_total(cur_len, lens_per_seq, b, maxT);
    const int cur = total - 1;
    FreshDst fd{};
    if constexpr (kFresh) fd = fresh_dst(kv_out, kv_scale_out, B, NH, maxT, bh, slice, cur);
    float q[R::kElems];

    float l = 0.0f, acc[R::kElems];
#pragma unroll
    for (int e = 0; e < R::kElems; ++e) acc[e] = 0.0f;

    if (total <= kW * kTile) {
        // Every wave owns at most one tile: its K and V rows are requested together, the
        // scores stay in registers and only the workgroup maximum passes through LDS.
        const int r = wave * kTile;
        if (!spec || total > spec_lim) {
            load_tile<DT, kU, true>(t, sl, r, total, slot_row);
            qr = load_q<DT>(qkv, b, h, NH, slice);
        }
        convert_q<DT, true>(qr, qscale, q);
        if (kFresh && cur >= r && cur < r + kTile) patch_tile<DT, kU>(t, fr, fd, r, slot_row, cur);
        // A tile requested for a longer hinted length holds rows at or beyond `total`.
        mask_tile_v<DT, kU>(t, r, total, slot_row);
        float s[kU];
        float mloc = kStartMax;
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            s[u] = row_sum<R::kLanes>(dot_chunk<DT, true>(q, t.k[u]));
            if constexpr (R::k8bit) s[u] *= t.ks[u];
            if (r + u * kRPL + slot_row < total) mloc = fmaxf(mloc, s[u]);
            else s[u] = -INFINITY;
        }
        mloc = slot_reduce<R::kLanes, true>(mloc);   // a row's lanes hold the same scores
        if (lane == 0) s_max[wave] = mloc;
        __syncthreads();
        float M = s_max[0];
#pragma unroll
        for (int w = 1; w < kW; ++w) M = fmaxf(M, s_max[w]);
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const float p = exp2_fast(s[u] - M);
            l += p;
            const float pv = R::k8bit ? p * t.vs[u] : p;
            float x[R::kElems];
            decode<DT>(t.v[u], x);
#pragma unroll
            for (int e = 0; e < R::kElems; ++e) acc[e] = fmaf(pv, x[e], acc[e]);
        }
    } else {
        // Scores staged in LDS.  Pass 1: tiles of kTile rows go round-robin to the waves,
        // every score is written to LDS and the exact maximum is found.
        convert_q<DT, true>(load_q<DT>(qkv, b, h, NH, slice), qscale, q);
        float mloc = kStartMax;
        const int full = total / kTile * kTile;
        for (int r = wave * kTile; r < full; r += kW * kTile)
            score_tile<DT, kU, false, kFresh, true>(sl, r, total, slot_row, slice, q, s_scores, mloc, fr, fd);
        for (int r = full + wave * kTile; r < total; r += kW * kTile)
            score_tile<DT, kU, true, kFresh, true>(sl, r, total, slot_row, slice, q, s_scores, mloc, fr, fd);
        mloc = slot_reduce<R::kLanes, true>(mloc);   // a row's lanes hold the same scores
        if (lane == 0) s_max[wave] = mloc;
        __syncthreads();
        float M = s_max[0];
#pragma unroll
        for (int w = 1; w < kW; ++w) M = fmaxf(M, s_max[w]);
        // Pass 2: V rows weighted by exp2(score - M).
        for (int r = wave * kTile; r < full; r += kW * kTile)
            weight_tile<DT, kU, false, kFresh>(sl, r, total, slot_row, M, s_scores, l, acc, fr);
        for (int r = full + wave * kTile; r < total; r += kW * kTile)
            weight_tile<DT, kU, true, kFresh>(sl, r, total, slot_row, M, s_scores, l, acc, fr);
    }

    l = slot_reduce<R::kLanes, false>(l);
    if (lane == 0) s_l[wave] = l;
    s_acc[wave][slice * R::kElems + slot_row] = slot_reduce_scatter<R::kLanes, R::kElems>(acc);
    __syncthreads();
    if (threadIdx.x < kHeadDim) {
        const int c = threadIdx.x;
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < kW; ++w) { L += s_l[w]; A += s_acc[w][c]; }
        store_out<DT>(out, (size_t)bh * kHeadDim + c, A / L);
    }
}

// ------------------------------------------------------------------------------------
// Split kernels.
// ------------------------------------------------------------------------------------
// kDesignatedDev: the designated merger over segments planned on the device (seg_rows ==
// kDevicePlanDes), a separate instance so that its speculative first tile leaves the
// host-planned instance's code as it is.  kPartialsStrided: kPartialsOnly for ragged lengths
// on half the grid, each workgroup taking two (or more) packed segments (a separate instance:
// sharing one kernel with the one-segment form costs the streaming kernel a third of its
// occupancy).
enum SplitMode {
    kPartialsOnly = 0, kLastBlockMerge = 1, kCoopMerge = 2, kDesignated = 3, kDesignatedDev = 4, kPartialsStrided = 5
};

struct SplitArgs {
    void* out;
    float* part_out;
    float* part_lse;
    float* part_max;
    unsigned* counters;
    // Designated merger: the tagged partials (64-bit words: the value in the low half, 1 in
    // the high half once written in the current call, 0 otherwise):
    // tag_ml[2 * slot] = {max (natural log units), exp-sum}, tag_out[slot * 64 + c].
    unsigned long long* tag_ml;
    unsigned long long* tag_out;
    const void* qkv;
    const uint8_t* kv;
    const float* kv_scale;
    uint8_t* kv_out;        // append-and-attend launches: where the current row goes
    float* kv_scale_out;
    // Paged cache (table != nullptr): kv / kv_scale are page pools [page][2][NH][page_rows]
    // rows, table[b * max_pages + j / page_rows] is the page holding position j of sequence b.
    const int* table;
    int max_pages, page_rows, num_pages;
    const int* cur_len;
    int lens_per_seq;
    int B, NH, maxT;
    int S;          // segment slots per (b,h): the grid stride and the partial stride
    int seg_rows;   // > 0: fixed rows per segment; 0: reference partition ceil(total/S);
                    // kDevicePlan: planned_rows(total) of the device length
    int spec_rows;  // the host's view of the attended length (0: unknown); see split_kernel
    float qscale;   // scale * log2(e)
    // Designated merger and cooperative barrier: workspace status words (see kWsStatus*), the
    // cooperative launch's barrier word {generation, count}, and the bound on their waits.
    unsigned* status;
    unsigned long long* barrier;
    int merge_polls;
};

// Kernel parameter arrays of split_kernel and merge_kernel (their leading scalars, then the
// struct), for launches through hipLaunchKernel, cooperative launches and graph nodes.
// split_spec(x) is the packed length hint pk_spec of split_kernel, split_pks(x, ...) its
// packed slot word pk_S, split_pnh(x, ...) its pk_NH and x.B * x.NH its pk_BNH; SPLIT_PARAMS
// needs int lvalues `spec`, `pks`, `pnh` and `bnh` holding them.
// pk_S: bits 0-16 the segment slots S (at most kMaxSegments); bit 30 the designated grid's
// XCD-local layout.  The designated instances take the dispatch id and the queue pointer in
// user SGPRs (the call's tag), which leaves 10 dwords of preloaded arguments: pk_spec falls
// out of them, so for those instances pk_S also carries what the first requests need of the
// length hint: bits 17-23 the segments the hint covers (at most 64), bit 24 per-sequence
// lengths.
constexpr int kXcdLocalBit = 1 << 30;
constexpr int kSlotMask = (1 << 17) - 1;
constexpr int kHintSegShift = 17;
constexpr int kLensBit = 1 << 24;
constexpr int kXcdRotShift = 25;   // bits 25-27: the test rotation of xcd_slot_rotated
inline int split_spec(const SplitArgs& a) { return a.lens_per_seq ? -1 : (a.spec_rows > 0 ? a.spec_rows : 0); }
#define SPLIT_PARAMS(x) {&(x).kv, &(x).qkv, &(x).cur_len, &pnh, &(x).maxT, &pks, &(x).seg_rows, &bnh, \
                         &spec, &(x).B, &(x)}
#define MERGE_PARAMS(x) {&(x).part_max, &(x).part_lse, &(x).part_out, &(x).cur_len, &(x).B, &(x).NH, &(x).maxT, \
                         &(x).S, &(x).seg_rows, &(x).lens_per_seq, &(x)}

struct Item {
    int b, h, s, total, n_seg, rows;
};

__host__ __device__ __forceinline__ int ceil_div_i(int a, int b) { return (a + b - 1) / b; }

constexpr int kDevicePlan = -1;     // rows from planned_rows() of the device length
constexpr int kDevicePlanDes = -2;  // rows from designated_rows() of the device length
constexpr int kDesignatedMaxGrid = 256;  // AUTO: designated merger while heads x segments <= this

// Rows per segment for an attended length of `total`: the whole length in one segment up
// to kFusedMaxRows positions, otherwise about four segments of a power-of-two length
// between kMinSegRows and kMaxSegRows.  The host plans with it from its length hint; with
// seg_rows == kDevicePlan every workgroup plans with it from the device length, so one
// launch (or one captured graph) serves every length up to maxT.
// Smallest power of two >= x (x >= 1), without a loop or branch, so that kernels can keep
// loads issued before a plan is computed in flight across it.
__host__ __device__ __forceinline__ int ceil_pow2(int x) {
#if defined(__HIP_DEVICE_COMPILE__)
    const int lz = __clz(x - 1);
#else
    const int lz = x > 1 ? __builtin_clz((unsigned)(x - 1)) : 32;
#endif
    return x > 1 ? 1 << (32 - lz) : 1;
}

__host__ __device__ __forceinline__ int planned_rows(int total) {
    const int want = ceil_div_i(total, 4);
    int r = min(max(kMinSegRows, ceil_pow2(max(want, 1))), kMaxSegRows);
    // Past kMaxMergeSegments segments of kMaxSegRows rows the rows grow instead, up to what a
    // paged wave walks.
    r = max(r, min(ceil_pow2(max(ceil_div_i(total, kMaxMergeSegments), 1)), kMaxPagedSegRows));
    return total <= kFusedMaxRows ? (total > 0 ? total : 1) : r;
}

// Rows per segment for the designated merger over `heads` = B*NH slots: the whole length
// in one segment up to kFusedMaxRows positions; otherwise 128-row segments for up to 16
// heads and 256 rows beyond (shorter segments cut each workgroup's streaming time, longer
// ones keep the grid within what the GPU runs at once), doubled only where a (b,h) would
// get more than 64 segments.
__host__ __device__ __forceinline__ int designated_base_rows(int heads) { return heads <= 16 ? 128 : 256; }
__host__ __device__ __forceinline__ int designated_rows(int total, int heads) {
    const int r = max(designated_base_rows(heads), ceil_pow2(max(ceil_div_i(total, kMaxDesignatedSegments), 1)));
    return total <= kFusedMaxRows ? (total > 0 ? total : 1) : r;
}

// Segments of a (b,h) whose length is `total` under fixed or device-planned rows
// (seg_rows != 0); `rows` receives the segment length.
__device__ __forceinline__ int seg_count(int seg_rows, int total, int heads, int& rows) {
    rows = seg_rows > 0 ? seg_rows
                        : (seg_rows == kDevicePlanDes ? designated_rows(total, heads) : planned_rows(total));
    return ceil_div_i(total, rows);
}

// Map a workgroup index to (b, h, segment).  Uniform lengths (or the reference
// partition) use the dense grid B*NH*S; ragged lengths with fixed-size segments pack
// the real segments of all sequences at the front of the grid using a prefix sum over
// the per-sequence segment counts, computed redundantly by every wave.  `dense`: the dense
// grid whatever the lengths (designated grids, whose slot order places every segment of a
// head on one XCD; slots beyond a head's segment count exit).
__device__ __forceinline__ bool locate(const SplitArgs& a, int BNH, int x, Item& it, bool dense) {
    if (dense || !a.lens_per_seq || a.seg_rows == 0) {
        if (!dense_slot(x, a.S, BNH, a.NH, it.b, it.h, it.s)) return false;
        it.total = seq_total_uniform(a.cur_len, a.lens_per_seq, it.b, a.maxT);
        it.rows = 0;
        it.n_seg = a.seg_rows != 0 ? seg_count(a.seg_rows, it.total, BNH, it.rows) : a.S;
        return it.s < it.n_seg;
    }
    const int lane = threadIdx.x & (kWave - 1);
    int base = 0;
    for (int b0 = 0; b0 < a.B; b0 += kWave) {
        const int b = b0 + lane;
        int tot = 0, cnt = 0;
        if (b < a.B) {
            int rows;
            tot = seq_total(a.cur_len, 1, b, a.maxT);
            cnt = a.NH * seg_count(a.seg_rows, tot, a.B * a.NH, rows);
        }
        int incl = cnt;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            const int v = __shfl_up(incl, d);
            if (lane >= d) incl += v;
        }
        const int pass_total = __shfl(incl, kWave - 1);
        if (x < base + pass_total) {
            const unsigned long long hit = __ballot(base + incl > x);
            const int L = __ffsll((long long)hit) - 1;
            const int excl = __shfl(incl - cnt, L);
            it.b = b0 + L;
            it.total = __shfl(tot, L);
            it.n_seg = seg_count(a.seg_rows, it.total, a.B * a.NH, it.rows);
            const int local = x - base - excl;
            it.h = local / it.n_seg;
            it.s = local - it.h * it.n_seg;
            return true;
        }
        base += pass_total;
    }
    return false;
}

// Partials of the in-kernel merge travel between workgroups that may sit on different
// XCDs (each with its own L2).  They are written and read as agent-scope relaxed atomics,
// which the gfx950 code generator emits as write-through / coherent stores and loads
// (sc1), so no L2 write-back or invalidate is needed: a writer waits until its stores are
// acknowledged (vmcnt 0) before it bumps the (b,h) counter, and the workgroup that takes
// the counter to n_seg reads the partials afterwards.
template <bool kCoherent>
__device__ __forceinline__ void put(float* p, float v) {
    if constexpr (kCoherent) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}
template <bool kCoherent>
__device__ __forceinline__ float get(const float* p) {
    if constexpr (kCoherent) return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *p;
}

// Tagged partial words of the designated merger: the value in the low half, the call's tag
// in the high half.  The tag is the launch's dispatch id (one per kernel dispatch,
// increasing along the queue; every replay of a captured graph dispatches anew) with the top
// bit set, so a word counts only for the dispatch that wrote it: words left by an earlier
// call (a plan with other slots on the same workspace, producers that finished after their
// merger stopped waiting) are never taken for this call's, the slots need no clearing, and
// a zeroed workspace holds no valid word.
//
// Where the words travel.  The host lays a designated grid out so that every segment of a
// head runs on one XCD (xcd_slot below).  Producers publish with plain stores, which land in
// their XCD's L2 and stay there (write-back); the merger polls with agent-scope loads (sc1),
// which miss the CU's L1 and hit a line of the XCD's L2 that holds written data.  Measured
// on MI355X (two workgroups handing a flag back and forth, 200 rounds): 460 ns per round
// trip on one XCD, against 925 ns with write-through (sc1) stores, which an agent-scope load
// then has to fetch from memory; across XCDs a plain store is never seen, which the merger's
// bounded wait and fallback cover (split_kernel).  Each slot's words sit in lines of their
// own (tag_ml: kMlStride words per slot), so a line the merger polls is written by one
// producer only.
constexpr int kDefaultMergePolls = 1 << 16;  // the designated merger's polls before it computes missing segments
constexpr int kMlStride = 16;                // u64 words per slot in tag_ml: {max, exp-sum}, one 128-byte line

// XCD placement of a designated grid (xcd_slot, lanes.hpp): segment s of head 8k + r is
// workgroup 8 (S k + s) + r, so every segment of a head runs on one XCD.  The grid is
// 8 * ceil(B*NH / 8) * S workgroups; those of heads beyond B*NH exit at once.
// The layout is used from kXcdLocalHeads heads on: with fewer, whole XCDs would sit idle
// while the ones holding a head stream all of its bytes; those grids keep the dense slot
// order, and their producers publish with write-through (sc1) stores, which an agent-scope
// load sees from any XCD.
constexpr int kXcdLocalHeads = 8;
__host__ __device__ __forceinline__ bool xcd_local_layout(int B, int NH) { return B * NH >= kXcdLocalHeads; }
__host__ __device__ __forceinline__ long long designated_grid(int B, int NH, int S) {
    return xcd_local_layout(B, NH) ? 8ll * ((B * NH + 7) / 8) * S : (long long)B * NH * S;
}

// Rotation of the designated grid's producers against their merger's XCD
// (kvattn_set_xcd_layout_offset, a test setting; 0 in use).
std::atomic<int> g_xcd_rot{0};

// pk_S of a split launch: the slot count and, for the designated instances, the XCD-local
// layout bit (and its test rotation) and the length hint in the form their first requests use
// (the segments the hint puts in use, per-sequence lengths).
inline int split_pks(const SplitArgs& a, bool des) {
    int pks = a.S;
    if (des) {
        if (xcd_local_layout(a.B, a.NH))
            pks |= kXcdLocalBit | (g_xcd_rot.load(std::memory_order_relaxed) & 7) << kXcdRotShift;
        if (a.lens_per_seq) pks |= kLensBit;
        else if (a.seg_rows > 0 && a.spec_rows > 0)
            pks |= std::min(ceil_div_i(a.spec_rows, a.seg_rows), kMaxDesignatedSegments) << kHintSegShift;
    }
    return pks;
}

// pk_NH of a split launch: NH, and for the designated instances NH | B * NH << 16 (both below
// 2^16: a designated grid has at least B * NH workgroups and must fit on the GPU at once).
inline int split_pnh(const SplitArgs& a, bool des) {
    return des ? (int)((unsigned)a.NH | (unsigned)(a.B * a.NH) << 16) : a.NH;
}

// Merge the n_seg partials of (b,h) = bh into out; executed by one full wave, lane c
// producing channel c.  Lane s holds the max and exp-sum of segment s (64 segments per
// round), and the weighted V partials are requested 16 segments at a time together with
// them, so up to 16 segments merge in a single memory round trip.
template <int DT, bool kCoherent>
__device__ __forceinline__ void merge_partials(void* out, const float* part_out, const float* part_lse,
                                               const float* part_max, int S, int n_seg, int bh, int c) {
    constexpr int kBatch = 16;
    const size_t p0 = (size_t)bh * S;
    float M = kEmptyMax, L = 0.0f, O = 0.0f;
    for (int s0 = 0; s0 < n_seg; s0 += kWave) {
        const int n = min(kWave, n_seg - s0);
        const float pm = c < n ? get<kCoherent>(part_max + p0 + s0 + c) : kEmptyMax;
        const float pl = c < n ? get<kCoherent>(part_lse + p0 + s0 + c) : 0.0f;
        float e = 0.0f;
        for (int k = 0; k < n; k += kBatch) {
            float v[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                v[u] = (k + u < n) ? get<kCoherent>(part_out + (p0 + s0 + k + u) * kHeadDim + c) : 0.0f;
            if (k == 0) {
                // Rescale what earlier rounds accumulated to the new running maximum.
                const float Mn = fmaxf(M, wave_max(pm));
                const float f = exp2_fast((M - Mn) * kLog2e);
                O *= f;
                L = L * f + wave_sum(exp2_fast((pm - Mn) * kLog2e) * pl);
                e = exp2_fast((pm - Mn) * kLog2e);
                M = Mn;
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                O = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), k + u)), v[u], O);
        }
    }
    store_out<DT>(out, (size_t)bh * kHeadDim + c, O / L);
}

// Workgroups of the streaming shape a CU should hold at once (bounds the register budget).
#ifndef KVATTN_STREAM_MIN_BLOCKS
#define KVATTN_STREAM_MIN_BLOCKS 1
#endif

// kFresh: append and attend in one launch (the workgroup whose segment holds position
// cur_len takes that row from qkv and writes it to the cache).  kPaged: the cache is a page
// pool addressed through a block table (segments then start at multiples of the tile).
template <int DT, int kMode, int kW, int kU, bool kFresh, bool kPaged>
__global__ __launch_bounds__(kW * kWave, kW == kWaves ? KVATTN_STREAM_MIN_BLOCKS : 1) void split_kernel(const uint8_t* pk_kv, const void* pk_qkv, const int* pk_len, int pk_NH, int pk_maxT,
                                         int pk_S, int pk_seg_rows, int pk_BNH, int pk_spec, int pk_B, SplitArgs a) {
    // The fields that the first loads depend on also come as leading scalar parameters: the
    // library is built with kernel-argument preloading, so the hardware hands them over in
    // SGPRs at wave launch and the first K/V, q and length requests do not wait for a scalar
    // load of the argument block.  The designated instances also take the dispatch id and the
    // queue pointer (their tag) in user SGPRs, which leaves 10 of the 16 for arguments: the
    // first 10 dwords here are all their first requests need (NH and B * NH packed into pk_NH,
    // both below 2^16 in any grid the GPU holds at once; the length hint packed into pk_S);
    // pk_BNH, pk_spec (the length hint of the other instances; -1: per-sequence lengths, the
    // hint not used) and B come after them (preloaded for the other instances, read later
    // from the argument block by the designated ones).  The struct keeps the rest; the q
    // scale is the constant of hs = 64.
    constexpr bool kDesMode = kMode == kDesignated || kMode == kDesignatedDev;
    a.kv = pk_kv;
    a.qkv = pk_qkv;
    a.cur_len = pk_len;
    a.NH = kDesMode ? (int)((unsigned)pk_NH & 0xFFFFu) : pk_NH;
    a.maxT = pk_maxT;
    a.S = pk_S & kSlotMask;
    a.seg_rows = pk_seg_rows;
    a.B = pk_B;
    const int BNH = kDesMode ? (int)((unsigned)pk_NH >> 16) : pk_BNH;
    int hint_segs = 0;   // designated: segments the host's length hint puts in use
    if constexpr (kDesMode) {
        a.lens_per_seq = (pk_S & kLensBit) != 0 ? 1 : 0;
        hint_segs = (pk_S >> kHintSegShift) & 127;
    } else {
        a.lens_per_seq = pk_spec < 0 ? 1 : 0;
        a.spec_rows = pk_spec < 0 ? 0 : pk_spec;
    }
    a.qscale = kQScale;
    using R = Row<DT>;
    // The latency shape (tiles of KVATTN_SPLIT_LAT_ROWS rows) takes the hardware bf16 dot.
    constexpr bool kHwDot = kU == kUnrollSplitLat<DT>;
    // Paged 8-bit caches in the latency shape request each wave's second tile with its first
    // (measured on 12-layer graphs, 64- and 256-row pages: INT8 and FP8 3-17 % faster at
    // 64-4096 positions; BF16 3-6 % slower, so it keeps the plain walk).
    constexpr bool kPagedAhead = kPaged && kHwDot && R::k8bit;
    __shared__ float s_m[kW];
    __shared__ float s_l[kW];
    __shared__ float s_acc[kW][kHeadDim];

    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int slot_row = lane / R::kLanes, slice = lane % R::kLanes;
    // Designated grids of the XCD-local layout: the slot this workgroup works on (every segment
    // of a head on one XCD).
    const bool xl = kDesMode && (pk_S & kXcdLocalBit) != 0;
    const int vbx = xl ? xcd_slot_rotated(blockIdx.x, a.S, (pk_S >> kXcdRotShift) & 7) : (int)blockIdx.x;

    // Uniform lengths with fixed-size segments: (b, h, s) and the segment's nominal rows
    // [j0, min(j0 + seg_rows, maxT)) follow from blockIdx alone, and the nominal range
    // always contains the true one [j0, min(j0 + seg_rows, total)).  When the host's length
    // hint says the segment is in use, each wave requests its first tile of the nominal
    // range, and its q slice, before reading the device length, so the three memory
    // round trips overlap; rows beyond the true length are masked afterwards.  Otherwise
    // the same first tile is requested once the length is known.
    // Designated segments planned on the device (kDesignatedDev) are designated_base_rows()
    // long at every length from kFusedMaxRows + 1 up to 64 segments' worth, so every
    // workgroup guesses that length (there is no hint to go by).  Segment 0 is also the
    // whole length up to kFusedMaxRows: wave w requests tile w of the segment's first kW tiles
    // early, and tile w of the next kW once the length shows they hold rows.  A segment the
    // length plans otherwise (doubled rows) drops the guess and requests its true first tile.
    constexpr bool kDev = kMode == kDesignatedDev;
    // The guess: first tile, q slice and fresh row; whether it was made and holds this
    // wave's tile; this wave's rows of the nominal range; the nominal range [g_j0, g_end).
    Tile<DT, kU> g_tile;
    QRaw<DT> g_q;
    FreshRaw<DT> g_fresh{};
    bool g_on = false, g_has_tile = true;
    int g_w0 = 0, g_w1 = 0, g_j0 = 0, g_end = 0;
    if (!kPaged && kMode != kPartialsStrided && !a.lens_per_seq && (kDev || a.seg_rows > 0)) {
        const int nom = kDev ? designated_base_rows(BNH) : a.seg_rows;
        const int bh0 = div_uniform(vbx, a.S);   // beyond B * NH only in a designated grid padded to whole XCD rounds
        const int s0 = vbx - bh0 * a.S;
        const int j0 = s0 * nom;
        const bool first = kDev && j0 == 0 && nom < kFusedMaxRows;
        // Segment 0 of the device plan may hold up to kFusedMaxRows rows: wave w takes tile w of
        // the first kW tiles now, and tile w of the next kW once the length shows it has rows
        // (segment lambda below); every other guess splits the nominal rows over the waves.
        constexpr int kTileRows = kRowsPerLoad<DT> * kU;
        int nend, w0, w1;
        guess_rows(s0, nom, first ? kFusedMaxRows : nom, a.maxT, first, kW, kTileRows, wave, nend, w0, w1);
        // Every cache type guesses in every segment (measured against 8-bit caches guessing in
        // segment 0 alone: INT8 and FP8 device-planned calls 5 % faster from 384 positions on,
        // none slower).
        // In use by the host's hint: s0 * nom < hint, i.e. s0 below the hinted segment count.
        const bool hinted = kDesMode ? s0 < hint_segs : j0 < a.spec_rows;
        if (guess_slot_live(bh0, BNH) && (kDev || hinted) && j0 < nend) {
            g_w0 = w0;
            g_w1 = w1;
            g_j0 = j0;
            g_end = nend;
            g_has_tile = !first || g_w1 <= j0 + nom;
            const Slot sl0 = make_slot<DT>(a.kv, a.kv_scale, 1, BNH, a.maxT, bh0, slice);
            if (g_has_tile) load_tile<DT, kU, true>(g_tile, sl0, g_w0, g_w1, slot_row);
            // The sequence index (a division by NH) is needed only for q's address: keep it
            // behind the tile's requests.
            __builtin_amdgcn_sched_barrier(0);
            const int b0 = BNH == a.NH ? 0 : bh0 / a.NH;
            g_q = load_q<DT>(a.qkv, b0, bh0 - b0 * a.NH, a.NH, slice);
            if constexpr (kFresh) g_fresh = load_fresh<DT>(a.qkv, b0, bh0 - b0 * a.NH, a.NH, slice);
            g_on = true;
        }
    }

    // Designated grids: the call's tag, and in the XCD-local layout this wave's XCD.  Every
    // segment of a head is laid out on the merger's XCD (xcd_slot), where the producers' plain
    // stores stay in the L2 the merger polls.  That rests on how the hardware hands workgroups
    // to XCDs; a producer whose stores the merger would not see holds it for its whole poll
    // bound.  So each merger (segment 0 of a real head) publishes the XCD it runs on,
    // write-through, once it knows the length (below, after locate); each producer reads that
    // word once its own tiles are consumed and publishes with plain stores only when it names
    // its own XCD, write-through otherwise (counted in the workspace's status words).
    uint32_t des_tag = 0, my_xcc = 0;
    if constexpr (kDesMode) {
        des_tag = call_tag();
        if (xl) my_xcc = xcc_id();
    }

    // The work of one segment `it` (active: the workgroup has one; the cooperative launch
    // also runs it without, for the grid barrier).  The guess comes in through the
    // parameters (spec: made; spec_tile: holds this wave's tile; [spec_j0, spec_end): its
    // nominal range), so that the strided loop below passes an empty one and carries no
    // tile from one segment to the next.
    // pid_in / have_pid (paged caches): this wave's page ids for the segment, requested
    // earlier by the caller (paged_tile_ids), or not.
    auto segment = [&](const Item& it, const bool active, Tile<DT, kU>& t0, QRaw<DT>& q0, FreshRaw<DT>& fr,
                       const bool spec, const bool spec_tile, int w0, int w1, const int spec_j0,
                       const int spec_end, const int pid_in = -1, const bool have_pid = false) {
        const int bh = it.b * a.NH + it.h;
        const size_t pidx = (size_t)bh * a.S + it.s;
        constexpr bool kCoh = kMode == kLastBlockMerge || kMode == kCoopMerge;
        constexpr bool kDes = kMode == kDesignated || kDev;

        // Rows [sj0, sj1) of segment s of this (b,h).
        auto seg_range = [&](int s, int& sj0, int& sj1) {
            if (a.seg_rows != 0) {
                sj0 = s * it.rows;
                sj1 = min(sj0 + it.rows, it.total);
            } else {
                const int chunk = ceil_div_i(it.total, a.S);
                sj0 = s * chunk;
                sj1 = min(sj0 + chunk, it.total);
            }
        };
        int j0 = 0, j1 = 0;
        if (active) seg_range(it.s, j0, j1);


        if (active) {
            if (j1 <= j0) {
                // Empty segment (reference partition with total < S): neutral partial (the
                // designated merger skips empty segments instead).
                if (!kDes && wave == 0) {
                    put<kCoh>(a.part_out + pidx * kHeadDim + lane, 0.0f);
                    if (lane == 0) { put<kCoh>(a.part_max + pidx, kEmptyMax); put<kCoh>(a.part_lse + pidx, 0.0f); }
                }
            } else {
                const int cur = it.total - 1;
                float m = kStartMax, l = 0.0f, acc[R::kElems];
#pragma unroll
                for (int e = 0; e < R::kElems; ++e) acc[e] = 0.0f;
                Slot sl{};
                FreshDst fd{};
                PagedView pv{};
                unsigned long long mword = 0;   // designated producer: the merger's XCD word
                if constexpr (kPaged) {
                    q0 = load_q<DT>(a.qkv, it.b, it.h, a.NH, slice);
                    if constexpr (kFresh) fr = load_fresh<DT>(a.qkv, it.b, it.h, a.NH, slice);
                    pv = PagedView{a.kv, a.kv_scale, a.table, a.max_pages, a.page_rows, a.num_pages, a.NH};
                    online_tiles_paged<DT, kU, kW, kFresh, kHwDot, kPagedAhead>(
                        pv, it.b, it.h, j0, j1, wave, slot_row, slice, q0, a.qscale, fr, a.kv_out, a.kv_scale_out,
                        cur, m, l, acc, pid_in, have_pid);
                } else {
                    sl = make_slot<DT>(a.kv, a.kv_scale, 1, BNH, a.maxT, bh, slice);   // B * NH: preloaded
                    // Device-planned segment 0 beyond its first kW tiles (128 < length <= 256): this
                    // wave's second tile, kW tiles further on, requested before the first is consumed.
                    constexpr int kTileRows = kRowsPerLoad<DT> * kU;
                    int x0 = 0, x1 = 0;
                    Tile<DT, kU> tx;
                    if (spec && (!kDev || (j0 == spec_j0 && j1 <= spec_end))) {
                        if (kDev && j0 == 0 && designated_base_rows(BNH) < kFusedMaxRows) {
                            x0 = w0 + kW * kTileRows;
                            x1 = min(x0 + kTileRows, j1);
                        }
                        w1 = min(w1, j1);
                        if (kDev && !spec_tile && w0 < w1) load_tile<DT, kU, true>(t0, sl, w0, w1, slot_row);
                        if (kDev && x0 < x1) load_tile<DT, kU, true>(tx, sl, x0, x1, slot_row);
                    } else {
                        const int per_wave = ceil_div_i(j1 - j0, kW);
                        w0 = min(j0 + wave * per_wave, j1);
                        w1 = min(w0 + per_wave, j1);
                        load_tile<DT, kU, true>(t0, sl, w0, w1, slot_row);
                        q0 = load_q<DT>(a.qkv, it.b, it.h, a.NH, slice);
                        if constexpr (kFresh) fr = load_fresh<DT>(a.qkv, it.b, it.h, a.NH, slice);
                    }
                    if constexpr (kFresh)
                        fd = fresh_dst(a.kv_out, a.kv_scale_out, 1, BNH, a.maxT, bh, slice, cur);
                    online_rows_from<DT, kU, kFresh, kHwDot>(t0, q0, sl, w0, w1, slot_row, a.qscale, fr, fd, cur, m, l,
                                                             acc);
                    if (kDev && x0 < x1)
                        online_rows_from<DT, kU, kFresh, kHwDot>(tx, q0, sl, x0, x1, slot_row, a.qscale, fr, fd, cur, m,
                                                                 l, acc);
                }
                // A producer's look at its merger's XCD word: requested once its tiles are consumed,
                // needed only when it publishes.  (Requested before the tiles are consumed, it
                // found the word not yet written for a fifth of the producers, which then published
                // write-through: +0.2 us per call.)
                if constexpr (kDes) {
                    if (xl && it.s != 0 && wave == 0) mword = get_word(a.tag_ml + (size_t)kMlStride * bh * a.S);
                }

                // Combine the row slots of this wave, then the 4 waves.
                const float mw = slot_reduce<R::kLanes, true>(m);
                const float f = exp2_fast(m - mw);
                l = slot_reduce<R::kLanes, false>(l * f);
#pragma unroll
                for (int e = 0; e < R::kElems; ++e) acc[e] *= f;
                if (lane == 0) { s_m[wave] = mw; s_l[wave] = l; }
                s_acc[wave][slice * R::kElems + slot_row] = slot_reduce_scatter<R::kLanes, R::kElems>(acc);
                __syncthreads();
                if (wave == 0) {
                    float Mb = s_m[0];
#pragma unroll
                    for (int w = 1; w < kW; ++w) Mb = fmaxf(Mb, s_m[w]);
                    float L = 0.0f, A = 0.0f;
#pragma unroll
                    for (int w = 0; w < kW; ++w) {
                        const float g = exp2_fast(s_m[w] - Mb);
                        L = fmaf(g, s_l[w], L);
                        A = fmaf(g, s_acc[w][lane], A);
                    }
                    if ((kMode == kLastBlockMerge || kMode == kCoopMerge || kDes) && it.n_seg == 1) {
                        // The only segment of its (b,h): the result needs no merge.
                        store_out<DT>(a.out, (size_t)bh * kHeadDim + lane, A / L);
                    } else if constexpr (kDes) {
                        const uint32_t tag = des_tag;
                        if (it.s != 0) {
                            // Producer: publish the tagged partial and finish; nothing waits.  Plain
                            // stores only when the merger's word names this XCD.
                            const bool seen = xl && word_is(mword, tag);
                            const bool local = seen && (uint32_t)mword == my_xcc;
                            publish_word(a.tag_out + pidx * kHeadDim + lane, tagged_word(A, tag), local);
                            if (lane == 0) {
                                publish_word(a.tag_ml + kMlStride * pidx, tagged_word(Mb * kLn2, tag), local);
                                publish_word(a.tag_ml + kMlStride * pidx + 1, tagged_word(L, tag), local);
                                if (xl && !local)
                                    __hip_atomic_fetch_add(a.status + (seen ? kWsStatusXcdRemote : kWsStatusXcdUnseen),
                                                           1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            }
                        } else {
                            // Designated merger (segment 0): lane u follows segment u.  A head's
                            // segments have consecutive slots with segment 0 first, all on this
                            // XCD, and workgroups are dispatched in id order, so the producers
                            // waited for are resident or next in line behind workgroups that do
                            // not wait, and their words land in this XCD's L2.  The wait is bounded
                            // all the same (a.merge_polls rounds): a merger that reaches the bound
                            // computes every producer segment itself on this wave (same tile
                            // code), so the result never depends on where or when the producers
                            // run, and counts itself in the workspace's status words.
                            const int n = it.n_seg;
                            const size_t p0 = (size_t)bh * a.S;
                            bool lost = n > kMaxDesignatedSegments;
                            int uj0 = 0, uj1 = 0;
                            if (lane < n) seg_range(lane, uj0, uj1);
                            const bool need = lane >= 1 && lane < n && uj1 > uj0 && !lost;
                            const unsigned long long prod = __ballot(need);   // segments a producer publishes
                            // Channel words of up to 16 segments per batch (8 when there are at most
                            // 8 segments); the first batch is requested together with the maxima and
                            // exp-sums, so up to 17 segments merge after one memory round trip.  A
                            // poll round has no branch: every word is requested (slots past the last
                            // one clamped to it) and the check masks what nothing is published for
                            // (lane 0's own slot, empty segments, slots past n).
                            const int last = n - 1;   // n >= 2 here
                            float O = 0.0f, LL = 1.0f;
                            auto merge_batches = [&](auto batch) {
                                constexpr int kB = decltype(batch)::value;
                                const size_t ml = (size_t)kMlStride * (p0 + min(lane, last));
                                unsigned long long wm, wl, w[kB];
                                for (int r = 0;; ++r) {
                                    if (r >= a.merge_polls) { lost = true; return; }
                                    wm = get_word(a.tag_ml + ml);
                                    wl = get_word(a.tag_ml + ml + 1);
#pragma unroll
                                    for (int u = 0; u < kB; ++u)
                                        w[u] = get_word(a.tag_out + (p0 + min(1 + u, last)) * kHeadDim + lane);
                                    uint32_t bad = need ? (((uint32_t)(wm >> 32) ^ tag) | ((uint32_t)(wl >> 32) ^ tag))
                                                        : 0u;
#pragma unroll
                                    for (int u = 0; u < kB; ++u)
                                        bad |= ((prod >> (1 + u)) & 1ull) ? ((uint32_t)(w[u] >> 32) ^ tag) : 0u;
                                    if (__all(bad == 0u)) break;
                                }
                                // Merge this wave's partial (segment 0) and the producers' partials,
                                // in segment order, with merge_partials' arithmetic.  Lanes from n on
                                // hold -FLT_MAX and 0, so with up to 8 (16) segments the reductions stop
                                // after the first 8 (16) lanes: the same steps, the same result, a
                                // shorter chain of dependent instructions.
                                const float pm = lane == 0 ? Mb * kLn2 : (need ? word_value(wm) : kEmptyMax);
                                const float pl = lane == 0 ? L : (need ? word_value(wl) : 0.0f);
                                float Mx, Ls;
                                if (n <= 8) {
                                    Mx = row_max<8>(pm);
                                    Ls = row_sum<8>(exp2_fast((pm - Mx) * kLog2e) * pl);
                                } else if (n <= 16) {
                                    Mx = row_max<16>(pm);
                                    Ls = row_sum<16>(exp2_fast((pm - Mx) * kLog2e) * pl);
                                } else {
                                    Mx = wave_max(pm);
                                    Ls = wave_sum(exp2_fast((pm - Mx) * kLog2e) * pl);
                                }
                                LL = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(Ls), 0));
                                // Words of slots nothing is published for (empty segments, slots past
                                // n, whose clamped words may be stale) enter as 0, so the fold of the
                                // first batch needs no branch and no stale value reaches it; their
                                // weights are finite, so they drop out exactly.
                                const float e = exp2_fast((pm - Mx) * kLog2e);
                                O = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), 0)) * A;
#pragma unroll
                                for (int u = 0; u < kB; ++u)
                                    O = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), 1 + u)),
                                             ((prod >> (1 + u)) & 1ull) ? word_value(w[u]) : 0.0f, O);
                                // Later batches (more than 17 segments), each polled for in turn.
                                if constexpr (kB == 16) {
                                    for (int k = 1 + kB; k < n; k += kB) {
                                        for (int r = 0;; ++r) {
                                            if (r >= a.merge_polls) { lost = true; return; }
#pragma unroll
                                            for (int u = 0; u < kB; ++u)
                                                w[u] = get_word(a.tag_out + (p0 + min(k + u, last)) * kHeadDim + lane);
                                            uint32_t bad2 = 0u;
#pragma unroll
                                            for (int u = 0; u < kB; ++u)
                                                bad2 |= (k + u < n && ((prod >> (k + u)) & 1ull))
                                                            ? ((uint32_t)(w[u] >> 32) ^ tag) : 0u;
                                            if (__all(bad2 == 0u)) break;
                                        }
#pragma unroll
                                        for (int u = 0; u < kB; ++u)
                                            if (k + u < n)
                                                O = fmaf(__int_as_float(
                                                             __builtin_amdgcn_readlane(__float_as_int(e), k + u)),
                                                         ((prod >> (k + u)) & 1ull) ? word_value(w[u]) : 0.0f, O);
                                    }
                                }
                            };
                            if (!lost) {
                                if (n <= 8) merge_batches(std::integral_constant<int, 8>{});
                                else merge_batches(std::integral_constant<int, 16>{});
                            }
                            float res = O / LL;
                            if (lost) {
                                // Fallback: this wave computes segments 1 .. n-1 itself (rows of
                                // each over all its row slots, the fresh row patched in as the
                                // producer would) and folds them, in segment order, into this
                                // segment's partial.
                                float Mo = Mb * kLn2, Lo = L, Oo = A;
                                for (int u = 1; u < n; ++u) {
                                    int sj0 = 0, sj1 = 0;
                                    seg_range(u, sj0, sj1);
                                    float mm = kStartMax, ll = 0.0f, ac[R::kElems];
#pragma unroll
                                    for (int e2 = 0; e2 < R::kElems; ++e2) ac[e2] = 0.0f;
                                    if (sj1 > sj0) {
                                        if constexpr (kPaged) {
                                            for (int w2 = 0; w2 < kW; ++w2)
                                                online_tiles_paged<DT, kU, kW, kFresh, kHwDot>(
                                                    pv, it.b, it.h, sj0, sj1, w2, slot_row, slice, q0, a.qscale, fr,
                                                    a.kv_out, a.kv_scale_out, cur, mm, ll, ac);
                                        } else {
                                            Tile<DT, kU> tf;
                                            load_tile<DT, kU, true>(tf, sl, sj0, sj1, slot_row);
                                            online_rows_from<DT, kU, kFresh, kHwDot>(tf, q0, sl, sj0, sj1, slot_row,
                                                                                     a.qscale, fr, fd, cur, mm, ll, ac);
                                        }
                                    }
                                    const float mw2 = slot_reduce<R::kLanes, true>(mm);
                                    const float f2 = exp2_fast(mm - mw2);
                                    ll = slot_reduce<R::kLanes, false>(ll * f2);
                                    // Channel `lane` is element lane % kElems of slice lane / kElems.
                                    float pa = 0.0f;
#pragma unroll
                                    for (int e2 = 0; e2 < R::kElems; ++e2) {
                                        const float t2 = __shfl(slot_reduce<R::kLanes, false>(ac[e2] * f2),
                                                                lane / R::kElems);
                                        pa = lane % R::kElems == e2 ? t2 : pa;
                                    }
                                    const float pmu = mw2 * kLn2;
                                    const float Mn = fmaxf(Mo, pmu);
                                    const float fo = exp2_fast((Mo - Mn) * kLog2e), fu = exp2_fast((pmu - Mn) * kLog2e);
                                    Lo = Lo * fo + ll * fu;
                                    Oo = Oo * fo + pa * fu;
                                    Mo = Mn;
                                }
                                res = Oo / Lo;
                            }
                            store_out<DT>(a.out, (size_t)bh * kHeadDim + lane, res);
                            if (lost && lane == 0)
                                __hip_atomic_fetch_add(a.status + kWsStatusMergeTimeouts, 1u, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
                        }
                    } else {
                        put<kCoh>(a.part_out + pidx * kHeadDim + lane, A);
                        if (lane == 0) { put<kCoh>(a.part_max + pidx, Mb * kLn2); put<kCoh>(a.part_lse + pidx, L); }
                    }
                }
            }
        }

        if constexpr (kMode == kLastBlockMerge) {
            // Wave 0 wrote this segment's partial with coherent stores.  Once they are
            // acknowledged it counts the segment; the wave that brings the (b,h) counter to
            // n_seg reads every partial with coherent loads, merges them and re-arms the
            // counter for the next call.  A (b,h) of one segment has already written out.
            if (wave == 0 && it.n_seg > 1) {
                wait_vm_stores();
                unsigned prev = 0;
                if (lane == 0)
                    prev = __hip_atomic_fetch_add(a.counters + bh, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
                prev = __shfl(prev, 0);
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                if (prev == (unsigned)(it.n_seg - 1)) {
                    merge_partials<DT, true>(a.out, a.part_out, a.part_lse, a.part_max, a.S, it.n_seg, bh, lane);
                    if (lane == 0)
                        __hip_atomic_store(a.counters + bh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        } else if constexpr (kMode == kCoopMerge) {
            // Grid barrier, for the mergers only.  Wave 0 of every workgroup (with a segment or
            // not) waits until its coherent partial stores are acknowledged and arrives on the
            // barrier word {generation, count}; the last of the gridDim.x arrivals re-arms it
            // as {generation + 1, 0}.  Segment 0 of each (b,h) waits for the generation to move
            // on, then merges; every other wave has nothing left to do and finishes.  The
            // cooperative launch keeps the whole grid resident, so the wait ends (bounded by
            // a.merge_polls like the designated merger's).
            if (wave == 0) {
                wait_vm_stores();
                unsigned long long prev = 0;
                if (lane == 0) prev = __hip_atomic_fetch_add(a.barrier, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const uint32_t gen = (uint32_t)__builtin_amdgcn_readfirstlane((int)(prev >> 32));
                const uint32_t cnt = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)prev);
                const bool last = cnt == gridDim.x - 1;
                if (last && lane == 0)
                    __hip_atomic_store(a.barrier, (unsigned long long)(gen + 1u) << 32, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                if (active && it.s == 0 && it.n_seg > 1) {
                    bool lost = false;
                    for (int r = 0; !last; ++r) {
                        if (r >= a.merge_polls) { lost = true; break; }
                        if ((uint32_t)(get_word(a.barrier) >> 32) != gen) break;
                        __builtin_amdgcn_s_sleep(1);
                    }
                    if (lost) {
                        store_out<DT>(a.out, (size_t)bh * kHeadDim + lane, __builtin_nanf(""));
                        if (lane == 0)
                            __hip_atomic_fetch_add(a.status + kWsStatusMergeTimeouts, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
                    } else {
                        merge_partials<DT, true>(a.out, a.part_out, a.part_lse, a.part_max, a.S, it.n_seg, bh, lane);
                    }
                }
            }
        }
    };

    if constexpr (kMode == kPartialsStrided) {
        // Ragged lengths with fixed-size segments: the host cannot size the grid to the
        // segments (the lengths are on the device), and a grid sized for maxT leaves
        // thousands of workgroups that only read the lengths and exit (C5: 5,500 of 12,288,
        // 3.5 % of the call).  Here the grid is 1/kStridedFactor of that bound and each
        // workgroup takes segments blockIdx.x, blockIdx.x + gridDim.x, ... of the packed
        // list: the empties halve, and the workgroups holding two segments are the first
        // dispatched, so the hardware's dynamic dispatch still balances the tail.  Each
        // workgroup counts the segments of every sequence once, into LDS, and finds
        // (b, h, s) there for each of its segments.
        __shared__ int s_seg_end[kStridedMaxSeqs];   // inclusive prefix of segment counts
        __shared__ int s_total[kStridedMaxSeqs];     // attended length of each sequence
        if (wave == 0) {
            int base = 0;
            for (int b0 = 0; b0 < a.B; b0 += kWave) {
                const int b = b0 + lane;
                int tot = 0, cnt = 0;
                if (b < a.B) {
                    int rows;
                    tot = seq_total(a.cur_len, 1, b, a.maxT);
                    cnt = a.NH * seg_count(a.seg_rows, tot, a.B * a.NH, rows);
                }
                int incl = cnt;
#pragma unroll
                for (int d = 1; d < kWave; d <<= 1) {
                    const int v = __shfl_up(incl, d);
                    if (lane >= d) incl += v;
                }
                if (b < a.B) { s_seg_end[b] = base + incl; s_total[b] = tot; }
                base += __shfl(incl, kWave - 1);
            }
        }
        __syncthreads();
        const int count = s_seg_end[a.B - 1];
        auto item_at = [&](int x) {
            Item it;
            int b = -1;
            for (int b0 = 0; b < 0; b0 += kWave) {
                const int bb = b0 + lane;
                const unsigned long long hit = __ballot(bb < a.B && s_seg_end[bb] > x);
                if (hit) b = b0 + __ffsll((long long)hit) - 1;
            }
            it.b = b;
            it.total = s_total[b];
            it.n_seg = seg_count(a.seg_rows, it.total, a.B * a.NH, it.rows);
            const int local = x - (b > 0 ? s_seg_end[b - 1] : 0);
            it.h = local / it.n_seg;
            it.s = local - it.h * it.n_seg;
            return it;
        };
        // Paged caches: the page ids of the workgroup's next segment are requested before the
        // current one is worked on, so that its first tiles wait for one round trip, not two.
        int pid_next = -1;
        bool have_next = false;
        for (int x = blockIdx.x; x < count; x += gridDim.x) {
            const Item it = item_at(x);
            const int pid_now = pid_next;
            const bool have_now = have_next;
            have_next = false;
            if constexpr (kPaged) {
                if (x + (int)gridDim.x < count) {
                    const Item nx = item_at(x + (int)gridDim.x);
                    const int nj0 = nx.s * nx.rows;
                    const PagedView npv{a.kv, a.kv_scale, a.table, a.max_pages, a.page_rows, a.num_pages, a.NH};
                    pid_next = paged_tile_ids<DT, kU, kW>(npv, nx.b, nj0, min(nj0 + nx.rows, nx.total), wave);
                    have_next = true;
                }
            }
            Tile<DT, kU> t;
            QRaw<DT> q;
            FreshRaw<DT> f{};
            segment(it, true, t, q, f, false, true, 0, 0, 0, 0, pid_now, have_now);
            __syncthreads();   // the next segment reuses s_m, s_l, s_acc
        }
    } else {
        Item it;
        const bool active = locate(a, BNH, vbx, it, kDesMode);
        if constexpr (kMode != kCoopMerge) {
            if (!active) return;
        }
        // The merger's XCD word (segment 0 of a real head, whose slot is vbx), which a head of
        // one segment, with no producer to read it, does without.
        if constexpr (kDesMode) {
            if (xl && it.s == 0 && it.n_seg > 1 && threadIdx.x == 0)
                __hip_atomic_store(a.tag_ml + (size_t)kMlStride * vbx, ((unsigned long long)des_tag << 32) | my_xcc,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        segment(it, active, g_tile, g_q, g_fresh, g_on, g_has_tile, g_w0, g_w1, g_j0, g_end);
    }
}

// Stand-alone merge: one wave per (b,h).
template <int DT>
// The partial pointers, the length and the shape also come as leading scalars (preloaded
// into SGPRs, as for split_kernel), so the partial loads issue without a scalar wait.
__global__ __launch_bounds__(kWave) void merge_kernel(const float* pk_max, const float* pk_lse, const float* pk_out,
                                                      const int* pk_len, int pk_B, int pk_NH, int pk_maxT, int pk_S,
                                                      int pk_seg_rows, int pk_lens, SplitArgs a) {
    a.part_max = const_cast<float*>(pk_max);
    a.part_lse = const_cast<float*>(pk_lse);
    a.part_out = const_cast<float*>(pk_out);
    a.cur_len = pk_len;
    a.B = pk_B;
    a.NH = pk_NH;
    a.maxT = pk_maxT;
    a.S = pk_S;
    a.seg_rows = pk_seg_rows;
    a.lens_per_seq = pk_lens;
    const int bh = blockIdx.x;
    const int b = bh / a.NH;
    const int c = threadIdx.x;
    constexpr int kBatch = 16;
    int n_seg = a.S, rows;
    if (a.seg_rows != 0 && a.S <= kBatch) {
        // The segment count follows from the device length.  Every slot's partial is
        // requested together with that length (one memory round trip instead of two), and
        // the slots beyond the count, whose words are stale, are dropped by selects.  The
        // arithmetic is merge_partials' for one batch.
        // Slot indices are clamped to S - 1 rather than branched on, so that no load sits
        // behind a branch and all of them issue ahead of the length's wait.
        const size_t p0 = (size_t)bh * a.S;
        const int last = a.S - 1;
        const float pm_all = a.part_max[p0 + min(c, last)];
        const float pl_all = a.part_lse[p0 + min(c, last)];
        float v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) v[u] = a.part_out[(p0 + min(u, last)) * kHeadDim + c];
        n_seg = seg_count(a.seg_rows, seq_total(a.cur_len, a.lens_per_seq, b, a.maxT), a.B * a.NH, rows);
        const float pm = c < n_seg ? pm_all : kEmptyMax;
        const float pl = c < n_seg ? pl_all : 0.0f;
        const float M = fmaxf(kEmptyMax, wave_max(pm));
        const float L = 0.0f * exp2_fast((kEmptyMax - M) * kLog2e) + wave_sum(exp2_fast((pm - M) * kLog2e) * pl);
        const float e = exp2_fast((pm - M) * kLog2e);
        float O = 0.0f;
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            O = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), u)), u < n_seg ? v[u] : 0.0f, O);
        store_out<DT>(a.out, (size_t)bh * kHeadDim + c, O / L);
        return;
    }
    if (a.seg_rows != 0) n_seg = seg_count(a.seg_rows, seq_total(a.cur_len, a.lens_per_seq, b, a.maxT), a.B * a.NH, rows);
    merge_partials<DT, false>(a.out, a.part_out, a.part_lse, a.part_max, a.S, n_seg, bh, c);
}

// ------------------------------------------------------------------------------------
// KV append.
// ------------------------------------------------------------------------------------
// Where column cl of (b, h) lives: the contiguous cache [2][B][NH][maxT] rows, or, with a
// block table, row cl % page_rows of head h in page table[b][cl / page_rows] of a pool
// [page][2][NH][page_rows].  Returns false for a page id outside [0, num_pages).
struct CacheMap {
    const int* table;      // nullptr: contiguous
    int max_pages, page_rows, num_pages;
};

__device__ __forceinline__ bool cache_rows(const CacheMap& cm, int B, int NH, int maxT, int b, int h, int cl,
                                           size_t& rk, size_t& rv) {
    if (!cm.table) {
        rk = ((size_t)b * NH + h) * maxT + cl;
        rv = (size_t)B * NH * maxT + rk;
        return true;
    }
    const int page = cm.table[(size_t)b * cm.max_pages + cl / cm.page_rows];
    if (page < 0 || page >= cm.num_pages) return false;
    rk = ((size_t)page * 2 * NH + h) * cm.page_rows + cl % cm.page_rows;
    rv = rk + (size_t)NH * cm.page_rows;
    return true;
}

// F32 / BF16: one thread per 16-byte chunk of the 2*B*NH rows (K rows, then V rows).
template <int DT>
__global__ __launch_bounds__(kBlock) void cache_write_kernel(uint8_t* __restrict__ kv, const uint8_t* __restrict__ qkv,
                                                             const int* __restrict__ cur_len, int lens_per_seq,
                                                             int B, int NH, int maxT, CacheMap cm) {
    constexpr int kChunks = Row<DT>::kBytes / 16;
    const int t = blockIdx.x * kBlock + threadIdx.x;
    const int rows = 2 * B * NH;
    if (t >= rows * kChunks) return;
    const int row = t / kChunks, c = t - row * kChunks;
    const int is_v = row >= B * NH;
    const int kh = row - is_v * B * NH;
    const int b = kh / NH, h = kh - b * NH;
    const int cl = seq_total(cur_len, lens_per_seq, b, maxT) - 1;
    size_t rk, rv;
    if (!cache_rows(cm, B, NH, maxT, b, h, cl, rk, rv)) return;
    const size_t src = (((size_t)b * 3 + 1 + is_v) * NH + h) * Row<DT>::kBytes + c * 16;
    const size_t dst = (is_v ? rv : rk) * Row<DT>::kBytes + c * 16;
    *reinterpret_cast<uint4*>(kv + dst) = *reinterpret_cast<const uint4*>(qkv + src);
}

// INT8 / FP8: one wave per row, lane c = channel c.  amax over the row, scale =
// amax / limit (127 or 448, IEEE division), codes of x / scale, zero codes for a zero row.
template <int DT>
__global__ __launch_bounds__(kBlock) void cache_write_w8_kernel(uint8_t* __restrict__ kv, float* __restrict__ kv_scale,
                                                                const uint16_t* __restrict__ qkv,
                                                                const int* __restrict__ cur_len, int lens_per_seq,
                                                                int B, int NH, int maxT, CacheMap cm) {
    const int row = blockIdx.x * kWaves + threadIdx.x / kWave;
    const int c = threadIdx.x & (kWave - 1);
    if (row >= 2 * B * NH) return;
    const int is_v = row >= B * NH;
    const int kh = row - is_v * B * NH;
    const int b = kh / NH, h = kh - b * NH;
    const int cl = seq_total(cur_len, lens_per_seq, b, maxT) - 1;
    const float x = bf16_to_f32(qkv[(((size_t)b * 3 + 1 + is_v) * NH + h) * kHeadDim + c]);
    const float amax = wave_max(fabsf(x));
    const float scale = amax / kW8Limit<DT>;
    const uint8_t code = w8_code<DT>(x, scale);
    size_t rk, rv;
    if (!cache_rows(cm, B, NH, maxT, b, h, cl, rk, rv)) return;   // uniform over the wave
    const size_t r = is_v ? rv : rk;
    kv[r * kHeadDim + c] = code;
    if (c == 0) kv_scale[r] = scale;
}

__device__ int g_cur_len = 0;

// Zero n 32-bit words (grid-stride).
__global__ __launch_bounds__(kBlock) void zero_words_kernel(uint32_t* __restrict__ p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (size_t)gridDim.x * kBlock) p[i] = 0u;
}

// The identity a tagged word carries for this dispatch: {dispatch id, queue pointer, tag}.
__global__ __launch_bounds__(kWave) void call_identity_kernel(unsigned long long* __restrict__ out) {
    if (threadIdx.x == 0) {
        out[0] = kvattn_dispatch_id();
        out[1] = (unsigned long long)(uintptr_t)__builtin_amdgcn_queue_ptr();
        out[2] = call_tag();
    }
}

// Stream-ordered write of the device length (one lane, one vector store).
__global__ __launch_bounds__(kWave) void set_len_kernel(int* __restrict__ p, int v) {
    if (threadIdx.x == 0) *p = v;
}

// ------------------------------------------------------------------------------------
// Host side.
// ------------------------------------------------------------------------------------
thread_local int t_last_hip_error = 0;

// Bound on the designated merger's polls for launches from now on (kvattn_set_merge_poll_limit).
std::atomic<int> g_merge_polls{kDefaultMergePolls};

#define KV_HIP(expr)                                            \
    do {                                                        \
        hipError_t e_ = (expr);                                 \
        if (e_ != hipSuccess) {                                 \
            t_last_hip_error = (int)e_;                         \
            return KVATTN_ERR_HIP;                              \
        }                                                       \
    } while (0)

#define KV_TRY(expr)                      \
    do {                                  \
        int st_ = (expr);                 \
        if (st_ != KVATTN_OK) return st_; \
    } while (0)

bool is_8bit(int dt) { return dt == KVATTN_KV_INT8 || dt == KVATTN_KV_FP8_E4M3; }
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int resolve_len(const int*& p) {
    if (p) return KVATTN_OK;
    int dev = 0;
    KV_HIP(hipGetDevice(&dev));
    static std::mutex mu;
    static std::map<int, int*> cache;
    std::lock_guard<std::mutex> lock(mu);
    auto itc = cache.find(dev);
    if (itc == cache.end()) {
        int* ptr = nullptr;
        KV_HIP(hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(g_cur_len)));
        itc = cache.emplace(dev, ptr).first;
    }
    p = itc->second;
    return KVATTN_OK;
}

int check_common(const void* qkv, const void* kv, const float* kv_scale, int B, int NH, int hs,
                 int maxT, int kv_dtype) {
    if (hs != kHeadDim) return KVATTN_ERR_HEAD_DIM;
    if (B < 1 || NH < 1 || maxT < 1 || maxT > kMaxT) return KVATTN_ERR_SHAPE;
    if ((long long)B * NH > (1ll << 24)) return KVATTN_ERR_SHAPE;
    if (kv_dtype < KVATTN_KV_F32 || kv_dtype > KVATTN_KV_FP8_E4M3) return KVATTN_ERR_DTYPE;
    if (!qkv || !kv) return KVATTN_ERR_NULL_POINTER;
    if (is_8bit(kv_dtype) && !kv_scale) return KVATTN_ERR_DTYPE;
    if (!aligned16(qkv) || !aligned16(kv)) return KVATTN_ERR_MISALIGNED;
    if (is_8bit(kv_dtype) && ((uintptr_t)kv_scale & 3u)) return KVATTN_ERR_MISALIGNED;
    return KVATTN_OK;
}

float qscale_for(int hs) { return (1.0f / sqrtf((float)hs)) * kLog2e; }

template <typename F>
int dispatch_dtype(int dt, F&& f) {
    switch (dt) {
        case KVATTN_KV_F32: return f(std::integral_constant<int, KVATTN_KV_F32>{});
        case KVATTN_KV_BF16: return f(std::integral_constant<int, KVATTN_KV_BF16>{});
        case KVATTN_KV_INT8: return f(std::integral_constant<int, KVATTN_KV_INT8>{});
        case KVATTN_KV_FP8_E4M3: return f(std::integral_constant<int, KVATTN_KV_FP8_E4M3>{});
        default: return KVATTN_ERR_DTYPE;
    }
}

// kv_out == nullptr: attention only.  Otherwise the kernel also appends the current
// token's row into kv_out / kv_scale_out (the same cache as kv / kv_scale).
// spec_rows: the hinted length the kernel may request tiles for before it reads the device
// length (one length for the batch), else 0.  hint_rows: the host's hinted (longest) length,
// or maxT when any length may come, which picks the tile shape only; 0: the general shape.
int launch_fused_single(void* out, const void* qkv, const void* kv, const float* kv_scale, void* kv_out,
                        float* kv_scale_out, int B, int NH, int maxT, const int* cur_len, int lens_per_seq,
                        int spec_rows, int hint_rows, int kv_dtype, hipStream_t stream) {
    const size_t lds = (size_t)maxT * sizeof(float);
    if (lds > kFusedMaxLds) return KVATTN_ERR_LDS;
    const float qs = qscale_for(kHeadDim);
    const bool short_tiles = hint_rows > 0 && hint_rows <= kFusedShortWaves * kFusedShortRows;
    const bool wide_f32 = kv_dtype == KVATTN_KV_F32 && (long long)B * NH > kFusedF32WideHeads;
    return dispatch_dtype(kv_dtype, [&](auto dtc) -> int {
        constexpr int DT = decltype(dtc)::value;
        auto launch = [&](auto threads_c, auto unroll_c) {
            constexpr int kThreads = decltype(threads_c)::value;
            constexpr int kU = decltype(unroll_c)::value;
            if (kv_out)
                hipLaunchKernelGGL((fused_single_kernel<DT, kThreads, kU, true>), dim3(B * NH), dim3(kThreads), lds,
                                   stream, qkv, (const uint8_t*)kv, cur_len, lens_per_seq, B, NH, maxT, spec_rows, qs,
                                   kv_scale, out, (uint8_t*)kv_out, kv_scale_out);
            else
                hipLaunchKernelGGL((fused_single_kernel<DT, kThreads, kU, false>), dim3(B * NH), dim3(kThreads), lds,
                                   stream, qkv, (const uint8_t*)kv, cur_len, lens_per_seq, B, NH, maxT, spec_rows, qs,
                                   kv_scale, out, (uint8_t*)nullptr, (float*)nullptr);
        };
        if (short_tiles)
            launch(std::integral_constant<int, kFusedShortWaves * kWave>{},
                   std::integral_constant<int, unroll_for<DT>(kFusedShortRows)>{});
        else if (DT == KVATTN_KV_F32 && wide_f32)
            launch(std::integral_constant<int, kWavesLat * kWave>{},
                   std::integral_constant<int, unroll_for<DT>(kFusedF32WideRows)>{});
        else
            launch(std::integral_constant<int, kFusedWaves<DT> * kWave>{},
                   std::integral_constant<int, unroll_for<DT>(kFusedRows<DT>)>{});
        KV_HIP(hipGetLastError());
        return KVATTN_OK;
    });
}

// Split kernel instance for a mode, a shape (`lat`: the latency shape, else the streaming
// shape) and whether the launch also appends the current row.
// (Paged caches have no cooperative instance, which the host never plans for them, and no
// kDesignatedDev instance: their first tile is never requested before the length.)
template <int DT, int W, int U, bool kFresh, bool kPaged>
const void* split_ptr_mode(int mode) {
    if (mode == kPartialsOnly) return (const void*)&split_kernel<DT, kPartialsOnly, W, U, kFresh, kPaged>;
    if (mode == kPartialsStrided) {
        if constexpr (W == kWaves) return (const void*)&split_kernel<DT, kPartialsStrided, W, U, kFresh, kPaged>;
        else return nullptr;
    }
    if (mode == kLastBlockMerge) return (const void*)&split_kernel<DT, kLastBlockMerge, W, U, kFresh, kPaged>;
    if (mode == kDesignated) return (const void*)&split_kernel<DT, kDesignated, W, U, kFresh, kPaged>;
    if constexpr (kPaged) return nullptr;
    else if (mode == kDesignatedDev) return (const void*)&split_kernel<DT, kDesignatedDev, W, U, kFresh, false>;
    else return (const void*)&split_kernel<DT, kCoopMerge, W, U, kFresh, false>;
}

template <int DT, int W, int U>
const void* split_ptr_shape(int mode, bool fresh, bool paged) {
    if (paged) return fresh ? split_ptr_mode<DT, W, U, true, true>(mode) : split_ptr_mode<DT, W, U, false, true>(mode);
    return fresh ? split_ptr_mode<DT, W, U, true, false>(mode) : split_ptr_mode<DT, W, U, false, false>(mode);
}

template <int DT>
const void* split_ptr(int mode, bool lat, bool fresh, bool paged) {
    if (lat) return split_ptr_shape<DT, kWavesLat, kUnrollSplitLat<DT>>(mode, fresh, paged);
    return split_ptr_shape<DT, kWaves, kUnroll<DT>>(mode, fresh, paged);
}

int split_threads(bool lat) { return (lat ? kWavesLat : kWaves) * kWave; }

// The split kernel for these arguments: appending when kv_out is set, paged when table is.
const void* split_ptr_for(const SplitArgs& a, int kv_dtype, int mode, bool lat) {
    const void* fn = nullptr;
    dispatch_dtype(kv_dtype, [&](auto dtc) -> int {
        fn = split_ptr<decltype(dtc)::value>(mode, lat, a.kv_out != nullptr, a.table != nullptr);
        return KVATTN_OK;
    });
    return fn;
}

int launch_split(const SplitArgs& a, int kv_dtype, int mode, bool lat, hipStream_t stream) {
    const void* fn = split_ptr_for(a, kv_dtype, mode, lat);
    if (!fn) return KVATTN_ERR_DTYPE;
    SplitArgs args = a;
    const int threads = split_threads(lat);
    long long grid = (long long)a.B * a.NH * a.S;
    // Ragged lengths with fixed-size segments on the streaming shape: half the grid, two
    // packed segments per workgroup (kPartialsStrided).
    // (Below 2^30 slots, so that x + gridDim.x in the kernel's walk stays within int.)
    if (mode == kPartialsOnly && !lat && a.lens_per_seq && a.seg_rows != 0 && a.B <= kStridedMaxSeqs &&
        grid < (1ll << 30)) {
        fn = split_ptr_for(a, kv_dtype, kPartialsStrided, lat);
        if (!fn) return KVATTN_ERR_DTYPE;
        grid = (grid + kStridedFactor - 1) / kStridedFactor;
    }
    const bool des = mode == kDesignated || mode == kDesignatedDev;
    if (des) grid = designated_grid(a.B, a.NH, a.S);
    if (des && (long long)a.B * a.NH >= (1 << 16)) return KVATTN_ERR_GRID_TOO_LARGE;
    int spec = split_spec(args);
    int pks = split_pks(args, des);
    int pnh = split_pnh(args, des);
    int bnh = a.B * a.NH;
    void* params[] = SPLIT_PARAMS(args);
    KV_HIP(hipLaunchKernel(fn, dim3((unsigned)grid), dim3(threads), params, 0, stream));
    return KVATTN_OK;
}

int launch_merge(const SplitArgs& a, int kv_dtype, hipStream_t stream) {
    return dispatch_dtype(kv_dtype, [&](auto dtc) -> int {
        constexpr int DT = decltype(dtc)::value;
        hipLaunchKernelGGL((merge_kernel<DT>), dim3(a.B * a.NH), dim3(kWave), 0, stream, a.part_max, a.part_lse,
                           a.part_out, a.cur_len, a.B, a.NH, a.maxT, a.S, a.seg_rows, a.lens_per_seq, a);
        KV_HIP(hipGetLastError());
        return KVATTN_OK;
    });
}

int stream_capturing(hipStream_t stream, bool& capturing) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    KV_HIP(hipStreamIsCapturing(stream, &st));
    capturing = st != hipStreamCaptureStatusNone;
    return KVATTN_OK;
}

// Workgroups of kernel `fn` (with `threads` threads) that the current device holds at once
// (occupancy per CU x CUs), and whether the device launches cooperatively; queried once per
// (device, kernel) and cached: the occupancy and attribute queries cost host time that an
// eager call should not pay every time.
int resident_capacity(const void* fn, int threads, long long& cap, bool* coop_out = nullptr) {
    int dev = 0;
    KV_HIP(hipGetDevice(&dev));
    static std::mutex mu;
    static std::map<std::tuple<int, const void*, int>, std::pair<long long, bool>> cache;
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_tuple(dev, fn, threads);
    auto itc = cache.find(key);
    if (itc == cache.end()) {
        int cus = 0, coop = 0, per_cu = 0;
        KV_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        KV_HIP(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev));
        KV_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, 0));
        itc = cache.emplace(key, std::make_pair((long long)per_cu * cus, coop != 0)).first;
    }
    cap = itc->second.first;
    if (coop_out) *coop_out = itc->second.second;
    return KVATTN_OK;
}

int launch_coop(const SplitArgs& a, int kv_dtype, bool lat, hipStream_t stream) {
    bool capturing = false;
    KV_TRY(stream_capturing(stream, capturing));
    if (capturing) return KVATTN_ERR_CAPTURE;
    const long long blocks = (long long)a.B * a.NH * a.S;
    // Every workgroup must be resident at once: take the latency shape if the grid fits
    // with it, else the 4-wave shape, else refuse.
    for (int attempt = 0; attempt < 2; ++attempt) {
        const bool use_lat = lat && attempt == 0;
        if (attempt == 1 && !lat) break;
        const void* fn = split_ptr_for(a, kv_dtype, kCoopMerge, use_lat);
        if (!fn) return KVATTN_ERR_DTYPE;
        const int threads = split_threads(use_lat);
        long long cap = 0;
        bool coop = false;
        KV_TRY(resident_capacity(fn, threads, cap, &coop));
        if (!coop) return KVATTN_ERR_COOP_TOO_LARGE;
        if (blocks > cap) continue;
        SplitArgs args = a;
        int spec = split_spec(args);
        int pks = split_pks(args, false);
        int pnh = split_pnh(args, false);
        int bnh = a.B * a.NH;
        void* params[] = SPLIT_PARAMS(args);
        KV_HIP(hipLaunchCooperativeKernel(fn, dim3((unsigned)blocks), dim3(threads), params, 0, stream));
        return KVATTN_OK;
    }
    return KVATTN_ERR_COOP_TOO_LARGE;
}

// hipGraph holding the split and merge kernel nodes, built once per argument set.
// Every kernel argument of the two nodes is part of the key (the length hint spec_rows
// decides which rows the split kernel requests before it reads the device length).
struct GraphKey {
    int dev, dt, lat;
    const void *out, *qkv, *kv, *ks, *kv_out, *ks_out, *table, *len, *po, *pl, *pm;
    int lens_per_seq, B, NH, maxT, S, seg_rows, spec_rows, max_pages, page_rows, num_pages;
    bool operator<(const GraphKey& o) const {
        return std::tie(dev, dt, lat, out, qkv, kv, ks, kv_out, ks_out, table, len, po, pl, pm, lens_per_seq, B,
                        NH, maxT, S, seg_rows, spec_rows, max_pages, page_rows, num_pages) <
               std::tie(o.dev, o.dt, o.lat, o.out, o.qkv, o.kv, o.ks, o.kv_out, o.ks_out, o.table, o.len, o.po,
                        o.pl, o.pm, o.lens_per_seq, o.B, o.NH, o.maxT, o.S, o.seg_rows, o.spec_rows,
                        o.max_pages, o.page_rows, o.num_pages);
    }
};

int launch_graph_pair(const SplitArgs& a, int kv_dtype, bool lat, hipStream_t stream) {
    bool capturing = false;
    KV_TRY(stream_capturing(stream, capturing));
    if (capturing) {
        // Inside a caller's capture the two kernels become nodes of the caller's graph.
        KV_TRY(launch_split(a, kv_dtype, kPartialsOnly, lat, stream));
        return launch_merge(a, kv_dtype, stream);
    }
    int dev = 0;
    KV_HIP(hipGetDevice(&dev));
    GraphKey key{dev,        kv_dtype,   lat ? 1 : 0, a.out,      a.qkv,          a.kv,       a.kv_scale,
                 a.kv_out,   a.kv_scale_out, a.table, a.cur_len,  a.part_out,     a.part_lse, a.part_max,
                 a.lens_per_seq, a.B,    a.NH,        a.maxT,     a.S,            a.seg_rows, a.spec_rows,
                 a.max_pages, a.page_rows, a.num_pages};
    static std::mutex mu;
    static std::map<GraphKey, hipGraphExec_t> cache;
    std::lock_guard<std::mutex> lock(mu);
    auto itc = cache.find(key);
    if (itc == cache.end()) {
        if (cache.size() >= 256) {
            for (auto& kvp : cache) (void)hipGraphExecDestroy(kvp.second);
            cache.clear();
        }
        void* fsplit = const_cast<void*>(split_ptr_for(a, kv_dtype, kPartialsOnly, lat));
        void* fmerge = nullptr;
        dispatch_dtype(kv_dtype, [&](auto dtc) -> int {
            fmerge = (void*)&merge_kernel<decltype(dtc)::value>;
            return KVATTN_OK;
        });
        SplitArgs args = a;
        int spec = split_spec(args);
        int pks = split_pks(args, false);
        int pnh = split_pnh(args, false);
        int bnh = a.B * a.NH;
        void* params[] = SPLIT_PARAMS(args);
        void* mparams[] = MERGE_PARAMS(args);
        hipGraph_t g = nullptr;
        KV_HIP(hipGraphCreate(&g, 0));
        hipKernelNodeParams ps{};
        ps.func = fsplit;
        ps.gridDim = dim3((unsigned)a.B * a.NH * a.S);
        ps.blockDim = dim3(split_threads(lat));
        ps.sharedMemBytes = 0;
        ps.kernelParams = params;
        ps.extra = nullptr;
        hipGraphNode_t nsplit = nullptr, nmerge = nullptr;
        hipError_t e = hipGraphAddKernelNode(&nsplit, g, nullptr, 0, &ps);
        if (e == hipSuccess) {
            hipKernelNodeParams pm = ps;
            pm.func = fmerge;
            pm.kernelParams = mparams;
            pm.gridDim = dim3((unsigned)a.B * a.NH);
            pm.blockDim = dim3(kWave);
            e = hipGraphAddKernelNode(&nmerge, g, &nsplit, 1, &pm);
        }
        hipGraphExec_t exec = nullptr;
        if (e == hipSuccess) e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (e != hipSuccess) {
            t_last_hip_error = (int)e;
            return KVATTN_ERR_HIP;
        }
        itc = cache.emplace(key, exec).first;
    }
    KV_HIP(hipGraphLaunch(itc->second, stream));
    return KVATTN_OK;
}

// Workspace (a caller's buffer or the static scratch), every region 256-byte aligned:
//   status [64] u32                           sticky status words (kWsStatus*)
//   counters u32                              last-block merge, one per (b,h)
//   part_max, part_lse [B*NH*S] f32, part_out [B*NH*S*64] f32   reference-format partials
//   tag_ml [B*NH*S*16] u64, tag_out [B*NH*S*64] u64   designated merger
// kvattn_workspace_init zeroes it once; the last-block kernels leave the counters at 0, and
// the designated merger's words carry the dispatch that wrote them, so they need no clearing.
// A caller's buffer is laid out by kvattn_layout::ws_layout (layout.hpp), so that calls of
// different plans on one buffer never find their counters or tags where another left
// partials.
struct Workspace {
    unsigned* status;
    unsigned* counters;
    float* part_max;
    float* part_lse;
    float* part_out;
    unsigned long long* tag_ml;
    unsigned long long* tag_out;
    size_t bytes;
};
static_assert(kvattn_layout::kWsStatusBytes == kWsStatusBytes && kvattn_layout::kWsMlWords == kMlStride &&
                  kvattn_layout::kWsChannels == kHeadDim, "workspace layout constants");

Workspace at(uint8_t* p, const kvattn_layout::WsLayout& l) {
    Workspace w;
    w.status = (unsigned*)p;
    w.counters = (unsigned*)(p + l.counters);
    w.part_max = (float*)(p + l.part_max);
    w.part_lse = (float*)(p + l.part_lse);
    w.part_out = (float*)(p + l.part_out);
    w.tag_ml = (unsigned long long*)(p + l.tag_ml);
    w.tag_out = (unsigned long long*)(p + l.tag_out);
    w.bytes = l.bytes;
    return w;
}

// avail: the caller's buffer size (0: the size query).  w.bytes is what the plan needs of a
// buffer of that size: it fits iff w.bytes <= avail.
Workspace carve(void* base, int B, int NH, int S, size_t avail = 0) {
    return at((uint8_t*)base, kvattn_layout::ws_layout((long long)B * NH, S, avail));
}

// S > 0: reference partition, S slots.  S < 0: -S rows per segment.  S == 0: sized for
// the smallest automatic segment length.
int segment_slots(int maxT, int S, int& slots, int& seg_rows) {
    if (S > 0) {
        if (S > kMaxSegments) return KVATTN_ERR_SPLIT;
        slots = S;
        seg_rows = 0;
        return KVATTN_OK;
    }
    seg_rows = S < 0 ? -S : kMinSegRows;
    if (seg_rows < 1) return KVATTN_ERR_SPLIT;
    slots = ceil_div_i(maxT, seg_rows);
    if (slots > kMaxSegments) return KVATTN_ERR_SPLIT;
    return KVATTN_OK;
}

// Automatic rows per segment: about four segments for the host's length hint, between
// kMinSegRows and 512 rows.  Small problems (a GPT-2 layer at B=1: 12 heads x 1024
// positions) then launch ~48 workgroups whose single in-kernel merge round is short;
// large ones stream 512-row segments, long enough to amortise a partial and short
// enough to balance ragged lengths across 256 CUs.
int auto_seg_rows(int total_hint) {
    const int want = (total_hint + 3) / 4;
    int r = kMinSegRows;
    while (r < want && r < kMaxSegRows) r <<= 1;
    return r;
}

// Segment slots that cover planned_rows() at every length up to maxT: one segment up to
// kFusedMaxRows positions, at most four while planned_rows(total) >= total / 4,
// ceil(total / kMaxSegRows) beyond, at most kMaxMergeSegments from there until the rows
// reach kMaxPagedSegRows, and ceil(total / kMaxPagedSegRows) past that.
// Segment slots covering designated_rows() at every length up to maxT.
int designated_slots(int maxT, int heads) {
    if (maxT <= kFusedMaxRows) return 1;
    return std::min(kMaxDesignatedSegments, ceil_div_i(maxT, designated_base_rows(heads)));
}

int planned_slots(int maxT) {
    if (maxT <= kFusedMaxRows) return 1;
    const int s = maxT <= kMaxSegRows * kMaxMergeSegments
                      ? ceil_div_i(maxT, kMaxSegRows)
                      : std::max(kMaxMergeSegments, ceil_div_i(maxT, kMaxPagedSegRows));
    return s > 4 ? s : 4;
}

constexpr long long kStreamRows = 1 << 19; // AUTO: split + merge kernel from this many rows
// ... and with per-sequence lengths of up to kRaggedLatMaxRows positions from this many (the
// longest length counted for every sequence): between the two, the last-block merge on the
// latency shape measured 1-18 % faster than split + merge (BF16, INT8, FP8, B = 6-64,
// 589,824-786,432 rows, contiguous and paged), while longer contexts (8-bit 17-25 % slower at
// 16384-32768 positions) and one length for the batch (FP8 and FP32 up to 26 % slower) keep
// the lower bound.
constexpr long long kStreamRowsRagged = 1 << 20;
constexpr int kRaggedLatMaxRows = 8192;
// ... and from this many with per-sequence lengths of up to kRaggedShortRows positions (96-320
// sequences of up to 1024 positions: the last-block merge up to 11 % faster than split + merge,
// one shape of twelve 2 % slower; at 2048-8192 positions a bound of 2^21 was already mixed,
// BF16 +2 to +3 %, 8-bit -1 to -5 %).
constexpr long long kStreamRowsRaggedShort = 1 << 22;
constexpr int kRaggedShortRows = 1024;
// ... and for contiguous 8-bit caches from this many up to kRagged8MidRows positions (INT8
// and FP8, 24-64 sequences of 2048-4096 positions: 1-8 % faster than from 2^20; BF16 2-3 %
// slower there, a paged INT8 cache +5 % to -3 %).
constexpr long long kStreamRowsRagged8Mid = 1 << 21;
constexpr int kRagged8MidRows = 4096;

// Resolve AUTO and the segmentation.  S > 0: reference partition with S slots; S < 0:
// -S rows per segment; S == 0: automatic rows per segment, from the length hint, or
// planned on the device from the device length when there is no hint (len_hint == -1).
struct Plan {
    int strategy, slots, seg_rows;
    bool lat;   // the latency shape: tiles of KVATTN_SPLIT_LAT_ROWS rows (else the streaming shape's)
};

// A call is latency bound while it streams fewer rows than kStreamRows (with per-sequence
// lengths: kStreamRowsRaggedShort up to kRaggedShortRows positions, for contiguous 8-bit
// caches (k8) kStreamRowsRagged8Mid up to kRagged8MidRows, kStreamRowsRagged up to
// kRaggedLatMaxRows).
bool latency_bound(int B, int NH, int total_rows, bool ragged = false, bool k8 = false) {
    long long bound = kStreamRows;
    if (ragged && total_rows <= kRaggedShortRows) bound = kStreamRowsRaggedShort;
    else if (ragged && k8 && total_rows <= kRagged8MidRows) bound = kStreamRowsRagged8Mid;
    else if (ragged && total_rows <= kRaggedLatMaxRows) bound = kStreamRowsRagged;
    return (long long)B * NH * total_rows < bound;
}

// AUTO's tuned plan for an attended length of total_hint (the host's hint, or maxT for a call
// that must serve every length), beyond fused_single: the plan measured fastest across
// B = 1..64, contexts 512..8192 and the four cache types (12-layer graphs on MI355X, 13 plans
// per shape).  make_plan decides where it applies (paged caches and calls without a hint take
// only its first two cases).
// - One segment per (b,h) (last-block instance, which then stores without a merge) when the
//   heads alone give 192 or more workgroups and no head is longer than 512 rows; 8-bit caches
//   take the streaming shape's 64-row tiles there.
// - The designated merger while its grid stays within kAutoDesignatedMaxGrid workgroups and
//   the call streams at most kAutoDesignatedMaxBytes: segments of max(128, maxT / 16) rows
//   (a power of two, so at most 16 per head; up to 64 per head when fewer than 12 heads
//   share the GPU), doubled up to 512 rows while the grid is too large; not when the
//   doubling left 8 or more segments per head of a call above kAutoDoubledMaxBytes (96 heads
//   x 8 segments of 256 or 512 rows: measured slower than the split + merge kernel).  Up to
//   64 heads whose segments are long (256 rows or more, 512 for 8-bit caches) the grid may
//   reach 1024 workgroups (49-64 heads x 16 segments; measured, A/B over NH = 12-64: BF16 at
//   4096 positions -7 % to +1 %, INT8 and FP8 at 8192 -1 % to -16 %, with or without a
//   hint; with 128-row segments the wider grid lost 4-17 %).  8-bit
//   caches take the streaming shape for segments of 256 rows or more on grids of up to 384
//   workgroups (one 64-row tile per wave).
// - Beyond that the call is bandwidth bound: with one length for every sequence, BF16 streams
//   256-row segments with the latency shape's tiles and INT8 256-row segments with the
//   streaming shape's (512 rows and the latency shape from contexts of 8192), through the
//   split + merge kernels, at most 64 segments per head (longer rows, in the streaming shape,
//   from contexts of 16384 (BF16) or 32768 (INT8) on: measured 1-12 % faster at 32768-131072
//   positions than 128-512 segments per head); FP32 and FP8, and per-sequence lengths (whose streaming kernel
//   packs two segments per workgroup on the general plan: 64 sequences of up to 8192
//   positions ran 9 % slower on 256-row segments), keep the general plan (false).
// Returns false to leave the plan to the general rules below.
constexpr long long kAutoDesignatedMaxGrid = 768;
constexpr long long kAutoDesignatedMaxBytes = 64ll << 20;
constexpr long long kAutoDoubledMaxBytes = 40ll << 20;
bool tuned_auto(int B, int NH, int maxT, int total_hint, int kv_dtype, bool ragged, Plan& p) {
    const long long heads = (long long)B * NH;
    const bool k8 = is_8bit(kv_dtype);
    const long long row_bytes = kv_dtype == KVATTN_KV_F32 ? 512 : (kv_dtype == KVATTN_KV_BF16 ? 256 : 136);
    const long long bytes = heads * total_hint * row_bytes;
    if (maxT <= 512 && heads >= 192) {
        p.strategy = KVATTN_SPLIT_LASTBLOCK;
        p.seg_rows = 512;
        p.slots = 1;
        p.lat = !k8;
        return true;
    }
    // At most 16 segments per head once the heads give 192 workgroups with them; fewer heads
    // take up to 64 (the merger's limit).
    const int target = (int)std::min<long long>(kMaxDesignatedSegments, std::max<long long>(16, 192 / heads));
    const int r0 = std::max(128, ceil_pow2(ceil_div_i(maxT, target)));
    int r = r0;
    const long long max_grid = heads <= 64 && r0 >= (k8 ? 512 : 256) ? 1024 : kAutoDesignatedMaxGrid;
    while (heads * ceil_div_i(maxT, r) > max_grid && r < 512) r <<= 1;
    const int segs = ceil_div_i(maxT, r);
    const long long grid = heads * segs;
    if (grid <= max_grid && bytes <= kAutoDesignatedMaxBytes &&
        !(r > r0 && segs >= 8 && bytes > kAutoDoubledMaxBytes)) {
        p.strategy = KVATTN_SPLIT_DESIGNATED;
        p.seg_rows = r;
        p.slots = segs;
        p.lat = !(k8 && r >= 256 && grid <= 384);
        return true;
    }
    if (!ragged && (kv_dtype == KVATTN_KV_BF16 || kv_dtype == KVATTN_KV_INT8)) {
        const bool long_int8 = kv_dtype == KVATTN_KV_INT8 && maxT >= 8192;
        p.strategy = KVATTN_SPLIT_MERGE;
        p.seg_rows = long_int8 ? 512 : 256;
        p.lat = kv_dtype == KVATTN_KV_BF16 || long_int8;
        // At most kMaxMergeSegments segments per head: longer rows, in the streaming shape,
        // once the context passes that many segments.
        const int capped = ceil_pow2(ceil_div_i(total_hint, kMaxMergeSegments));
        if (capped > p.seg_rows) {
            p.seg_rows = capped;
            p.lat = false;
        }
        p.slots = ceil_div_i(maxT, p.seg_rows);
        return true;
    }
    return false;
}

// paged: a paged cache, which has no fused_single or cooperative instance and whose
// segments start at multiples of 64 rows (the tile), so rows per segment are planned on
// the device unless S < 0 gives a multiple of 64.
// ragged: per-sequence lengths.  tuned: AUTO may take tuned_auto's plan (off: the general
// rules alone).
int make_plan(int B, int NH, int maxT, int len_hint, int S, int strategy, int kv_dtype, Plan& p,
              bool paged = false, bool ragged = false, bool tuned = true) {
    if (strategy < KVATTN_AUTO || strategy > KVATTN_SPLIT_DESIGNATED) return KVATTN_ERR_STRATEGY;
    if (len_hint >= maxT || len_hint < -1) return KVATTN_ERR_LENGTH;
    if (paged) {
        if (strategy == KVATTN_FUSED_SINGLE || strategy == KVATTN_SINGLE_LAUNCH_COOP) return KVATTN_ERR_STRATEGY;
        if (S > 0 || (S < 0 && ((-S) % kMinSegRows != 0 || -S > kMaxPagedSegRows))) return KVATTN_ERR_SPLIT;
    }
    const int total_hint = (len_hint < 0 ? maxT - 1 : len_hint) + 1;
    const bool auto_strategy = strategy == KVATTN_AUTO;
    if (strategy == KVATTN_AUTO) {
        // Short contexts: one workgroup per (b,h).  Otherwise split; a single launch with
        // the in-kernel merge while the whole call is latency bound, and split + merge
        // kernel once the call streams enough rows to be bandwidth bound.
        const bool fits = (size_t)maxT * sizeof(float) <= kFusedMaxLds;
        const bool fused = !paged && fits && total_hint <= kFusedMaxRows;
        const bool hinted = len_hint >= 0;
        if (tuned && !fused && S == 0 && !(paged && hinted && total_hint <= kFusedMaxRows)) {
            int slots_bound = 0, rows_bound = 0;   // the workspace bound of S == 0, checked as below
            KV_TRY(segment_slots(maxT, S, slots_bound, rows_bound));
            const long long heads = (long long)B * NH;
            // Without a hint: beyond the device-planned designated grid of a few heads, the
            // designated window (or one segment per head) of the hinted plan at maxT, with fixed
            // rows, whose grid serves every length up to maxT.  Without a hint and on a paged
            // cache, the split + merge plans stay planned on the device (a paged cache's short
            // hinted lengths too, and segments longer than a paged wave walks).
            if (hinted || heads > 16 || heads * designated_slots(maxT, B * NH) > kDesignatedMaxGrid) {
                Plan q{};
                if (tuned_auto(B, NH, maxT, hinted ? total_hint : maxT, kv_dtype, ragged, q) &&
                    (q.strategy != KVATTN_SPLIT_MERGE || (hinted && !paged)) &&
                    !(paged && q.seg_rows > kMaxPagedSegRows)) {
                    p = q;
                    return heads * p.slots >= (1ll << 31) ? KVATTN_ERR_SHAPE : KVATTN_OK;
                }
            }
        }
        if (fused) strategy = KVATTN_FUSED_SINGLE;
        else if (!latency_bound(B, NH, total_hint, ragged, is_8bit(kv_dtype) && !paged)) strategy = KVATTN_SPLIT_MERGE;
        else if ((long long)B * NH * ceil_div_i(total_hint, designated_rows(total_hint, B * NH)) <= kDesignatedMaxGrid)
            strategy = KVATTN_SPLIT_DESIGNATED;
        else strategy = KVATTN_SPLIT_LASTBLOCK;
    }
    p.strategy = strategy;
    p.lat = latency_bound(B, NH, total_hint, ragged && auto_strategy, is_8bit(kv_dtype) && !paged);
    if (strategy == KVATTN_FUSED_SINGLE) {
        p.slots = 1;
        p.seg_rows = 0;
        return KVATTN_OK;
    }
    KV_TRY(segment_slots(maxT, S, p.slots, p.seg_rows));
    const bool des = strategy == KVATTN_SPLIT_DESIGNATED;
    if (S == 0 && (len_hint < 0 || paged)) {
        p.seg_rows = des ? kDevicePlanDes : kDevicePlan;
        p.slots = des ? designated_slots(maxT, B * NH) : planned_slots(maxT);
    } else if (S == 0) {
        // Rows fixed from the hint; the grid covers every device length up to maxT, so the
        // designated merger also needs rows >= maxT / 64.
        p.seg_rows = des ? std::max(designated_rows(total_hint, B * NH), designated_rows(maxT, B * NH))
                         : auto_seg_rows(total_hint);
        // AUTO with one length for the batch: past kMaxMergeSegments segments of 512 rows
        // (32768 positions) the rows grow instead.  Measured with 1024-row segments against
        // 128 of 512 at 40000-65536 positions: FP8 5-7 %, FP32 1-4 % faster; per-sequence
        // lengths (-3 % to +7 %) and explicit strategies keep 512.
        if (!des && auto_strategy && !ragged)
            p.seg_rows = std::max(p.seg_rows, ceil_pow2(ceil_div_i(total_hint, kMaxMergeSegments)));
        p.slots = ceil_div_i(maxT, p.seg_rows);
    }
    if ((long long)B * NH * p.slots >= (1ll << 31)) return KVATTN_ERR_SHAPE;
    const bool des_fits = p.slots <= kMaxDesignatedSegments &&
                          !(paged && p.seg_rows == kDevicePlanDes && designated_rows(maxT, B * NH) > kMaxPagedSegRows);
    if (des && !des_fits) {
        // More segments per (b,h) than the merger follows (or longer paged segments than a
        // wave walks): AUTO takes the last-block merge with its own segmentation.
        if (!auto_strategy) return KVATTN_ERR_SPLIT;
        return make_plan(B, NH, maxT, len_hint, S, KVATTN_SPLIT_LASTBLOCK, kv_dtype, p, paged, ragged);
    }
    return KVATTN_OK;
}

// append == true: the launch also writes the current token's K/V row (kvattn_append_decode).
// pm != nullptr: kv / kv_scale are page pools addressed through pm's block table.
// use_scratch: the workspace is the library's static device array (kvattn_decode_static).
int scratch_base(hipStream_t stream, uint8_t*& base);
bool carve_scratch(uint8_t* base, int B, int NH, int S, Workspace& w);

int decode_impl(void* out, const void* qkv, const void* kv, const float* kv_scale, int B, int NH, int hs,
                int maxT, const int* d_cur_len, int lens_per_seq, int len_hint, void* workspace,
                size_t workspace_bytes, int S, int strategy, int kv_dtype, void* stream_v, bool append,
                const CacheMap* pm = nullptr, bool use_scratch = false) {
    KV_TRY(check_common(qkv, kv, kv_scale, B, NH, hs, maxT, kv_dtype));
    if (!out) return KVATTN_ERR_NULL_POINTER;
    if (!aligned16(out)) return KVATTN_ERR_MISALIGNED;
    Plan plan{};
    KV_TRY(make_plan(B, NH, maxT, len_hint, S, strategy, kv_dtype, plan, pm != nullptr, lens_per_seq != 0));
    hipStream_t stream = (hipStream_t)stream_v;

    if (plan.strategy == KVATTN_FUSED_SINGLE) {
        KV_TRY(resolve_len(d_cur_len));
        return launch_fused_single(out, qkv, kv, kv_scale, append ? const_cast<void*>(kv) : nullptr,
                                   append ? const_cast<float*>(kv_scale) : nullptr, B, NH, maxT, d_cur_len,
                                   lens_per_seq, (lens_per_seq || len_hint < 0) ? 0 : len_hint + 1,
                                   len_hint < 0 ? maxT : len_hint + 1, kv_dtype, stream);
    }

    Workspace w{};
    if (use_scratch) {
        // The cooperative launch and the library's own graph pair are not offered here: the
        // runtime may allocate device memory for them.
        if (plan.strategy == KVATTN_SINGLE_LAUNCH_COOP || plan.strategy == KVATTN_SINGLE_LAUNCH_GRAPH)
            return KVATTN_ERR_STRATEGY;
        uint8_t* base = nullptr;
        KV_TRY(scratch_base(stream, base));
        if (!carve_scratch(base, B, NH, plan.slots, w)) {
            // A tuned AUTO plan may hold more segments than the array has room for where the
            // general plan's fit: AUTO then takes the general plan.
            if (strategy != KVATTN_AUTO) return KVATTN_ERR_WORKSPACE;
            KV_TRY(make_plan(B, NH, maxT, len_hint, S, strategy, kv_dtype, plan, pm != nullptr, lens_per_seq != 0,
                             false));
            if (!carve_scratch(base, B, NH, plan.slots, w)) return KVATTN_ERR_WORKSPACE;
        }
    } else {
        if (!workspace) return KVATTN_ERR_WORKSPACE;
        if (!aligned16(workspace)) return KVATTN_ERR_MISALIGNED;
        w = carve(workspace, B, NH, plan.slots, workspace_bytes);
        if (w.bytes > workspace_bytes) return KVATTN_ERR_WORKSPACE;
    }
    KV_TRY(resolve_len(d_cur_len));

    SplitArgs a{};
    a.out = out;
    a.part_out = w.part_out;
    a.part_lse = w.part_lse;
    a.part_max = w.part_max;
    a.counters = w.counters;
    a.tag_ml = w.tag_ml;
    a.tag_out = w.tag_out;
    a.status = w.status;
    a.barrier = reinterpret_cast<unsigned long long*>(w.status + kWsStatusBarrier);
    a.merge_polls = g_merge_polls.load(std::memory_order_relaxed);
    a.qkv = qkv;
    a.kv = (const uint8_t*)kv;
    a.kv_scale = kv_scale;
    a.kv_out = append ? (uint8_t*)const_cast<void*>(kv) : nullptr;
    a.kv_scale_out = append ? const_cast<float*>(kv_scale) : nullptr;
    if (pm) {
        a.table = pm->table;
        a.max_pages = pm->max_pages;
        a.page_rows = pm->page_rows;
        a.num_pages = pm->num_pages;
    }
    a.cur_len = d_cur_len;
    a.lens_per_seq = lens_per_seq ? 1 : 0;
    a.B = B;
    a.NH = NH;
    a.maxT = maxT;
    a.S = plan.slots;
    a.seg_rows = plan.seg_rows;
    a.spec_rows = len_hint >= 0 ? len_hint + 1 : 0;
    a.qscale = qscale_for(hs);

    switch (plan.strategy) {
        case KVATTN_SPLIT_MERGE:
            KV_TRY(launch_split(a, kv_dtype, kPartialsOnly, plan.lat, stream));
            return launch_merge(a, kv_dtype, stream);
        case KVATTN_SPLIT_LASTBLOCK: return launch_split(a, kv_dtype, kLastBlockMerge, plan.lat, stream);
        case KVATTN_SPLIT_DESIGNATED: {
            const int mode = plan.seg_rows == kDevicePlanDes && !pm ? kDesignatedDev : kDesignated;
            // The mergers wait for their producers, so the whole grid must fit on the GPU at once
            // (AUTO plans at most kAutoDesignatedMaxGrid segments; the workgroups an XCD-local
            // grid adds exit at once and do not count).  An AUTO plan whose grid this GPU does
            // not hold takes the last-block merge instead.
            const long long grid = (long long)B * NH * plan.slots;
            if (grid > kDesignatedMaxGrid) {
                const void* fn = split_ptr_for(a, kv_dtype, mode, plan.lat);
                if (!fn) return KVATTN_ERR_DTYPE;
                long long cap = 0;
                KV_TRY(resident_capacity(fn, split_threads(plan.lat), cap));
                if (grid > cap) {
                    if (strategy != KVATTN_AUTO) return KVATTN_ERR_GRID_TOO_LARGE;
                    return launch_split(a, kv_dtype, kLastBlockMerge, plan.lat, stream);
                }
            }
            return launch_split(a, kv_dtype, mode, plan.lat, stream);
        }
        case KVATTN_SINGLE_LAUNCH_COOP: return launch_coop(a, kv_dtype, plan.lat, stream);
        case KVATTN_SINGLE_LAUNCH_GRAPH: return launch_graph_pair(a, kv_dtype, plan.lat, stream);
        default: return KVATTN_ERR_STRATEGY;
    }
}

// ------------------------------------------------------------------------------------
// kvattn_decode_static: the workspace in a static device array.
// ------------------------------------------------------------------------------------
// Layout: the status words, a fixed region of merge counters for up to kScratchMaxHeads
// (b,h) (so that calls of different B*NH never find another plan's partials where their
// counters sit; the last-block kernels leave the counters at zero after every call), then
// the partials and tagged words of the current plan (carved as in a caller's workspace).
constexpr size_t kScratchBytes = 8u << 20;
constexpr int kScratchMaxHeads = 16384;
constexpr size_t kScratchCounterBytes = kScratchMaxHeads * sizeof(unsigned);
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// Device address of this device's `scratch`, found once per device with hipGetSymbolAddress
// (the host-side name of the array is a stand-in, not a device address); on that first call
// its status words and counters are cleared with a fill kernel on `stream`.
int scratch_base(hipStream_t stream, uint8_t*& base) {
    int dev = 0;
    KV_HIP(hipGetDevice(&dev));
    static std::mutex mu;
    static std::map<int, uint8_t*> bases;
    std::lock_guard<std::mutex> lock(mu);
    auto itb = bases.find(dev);
    if (itb == bases.end()) {
        uint8_t* ptr = nullptr;
        KV_HIP(hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch)));
        if (!ptr) return KVATTN_ERR_HIP;
        const size_t words = (kWsStatusBytes + kScratchCounterBytes) / sizeof(uint32_t);
        hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((words + kBlock - 1) / kBlock)), dim3(kBlock), 0,
                           stream, (uint32_t*)ptr, words);
        KV_HIP(hipGetLastError());
        itb = bases.emplace(dev, ptr).first;
    }
    base = itb->second;
    return KVATTN_OK;
}

// The plan's workspace regions inside the scratch array; false when they do not fit.
bool carve_scratch(uint8_t* base, int B, int NH, int S, Workspace& w) {
    if ((long long)B * NH > kScratchMaxHeads) return false;
    const kvattn_layout::WsLayout l = kvattn_layout::ws_layout((long long)B * NH, S, kScratchBytes, kScratchCounterBytes);
    if (l.bytes > kScratchBytes) return false;
    w = at(base, l);
    return true;
}

SplitArgs caller_partials(void* out, const void* qkv, const void* kv, const float* kv_scale, int B, int NH,
                          int maxT, const int* cur_len, int lens_per_seq, float* part_out, float* part_lse,
                          float* part_max, int S) {
    SplitArgs a{};
    a.out = out;
    a.part_out = part_out;
    a.part_lse = part_lse;
    a.part_max = part_max;
    a.counters = nullptr;
    a.qkv = qkv;
    a.kv = (const uint8_t*)kv;
    a.kv_scale = kv_scale;
    a.cur_len = cur_len;
    a.lens_per_seq = lens_per_seq ? 1 : 0;
    a.B = B;
    a.NH = NH;
    a.maxT = maxT;
    a.S = S;
    a.seg_rows = 0;
    a.qscale = qscale_for(kHeadDim);
    return a;
}

int launch_cache_write(void* kv, float* kv_scale, const void* qkv, int B, int NH, int maxT, const int* d_cur_len,
                       int lens_per_seq, int kv_dtype, const CacheMap& cm, hipStream_t stream) {
    const int lps = lens_per_seq ? 1 : 0;
    return dispatch_dtype(kv_dtype, [&](auto dtc) -> int {
        constexpr int DT = decltype(dtc)::value;
        if constexpr (Row<DT>::k8bit) {
            const int rows = 2 * B * NH;
            hipLaunchKernelGGL((cache_write_w8_kernel<DT>), dim3((rows + kWaves - 1) / kWaves), dim3(kBlock), 0,
                               stream, (uint8_t*)kv, kv_scale, (const uint16_t*)qkv, d_cur_len, lps, B, NH, maxT,
                               cm);
        } else {
            const int chunks = 2 * B * NH * (Row<DT>::kBytes / 16);
            hipLaunchKernelGGL((cache_write_kernel<DT>), dim3((chunks + kBlock - 1) / kBlock), dim3(kBlock), 0,
                               stream, (uint8_t*)kv, (const uint8_t*)qkv, d_cur_len, lps, B, NH, maxT, cm);
        }
        KV_HIP(hipGetLastError());
        return KVATTN_OK;
    });
}

// Paged-cache arguments; maxT receives the positions a sequence can hold.
int check_paged(const int* table, int max_pages, int page_rows, int num_pages, int NH, int& maxT) {
    if (!table) return KVATTN_ERR_NULL_POINTER;
    if ((uintptr_t)table & 3u) return KVATTN_ERR_MISALIGNED;
    if (max_pages < 1 || num_pages < 1 || page_rows < kMinSegRows || page_rows % kMinSegRows != 0)
        return KVATTN_ERR_SHAPE;
    if ((long long)max_pages * page_rows > kMaxT) return KVATTN_ERR_SHAPE;
    if ((long long)num_pages * 2 * NH * page_rows >= (1ll << 40)) return KVATTN_ERR_SHAPE;
    maxT = max_pages * page_rows;
    return KVATTN_OK;
}

int check_partials(const float* po, const float* pl, const float* pm, int S) {
    if (!po || !pl || !pm) return KVATTN_ERR_NULL_POINTER;
    if (!aligned16(po) || ((uintptr_t)pl & 3u) || ((uintptr_t)pm & 3u)) return KVATTN_ERR_MISALIGNED;
    if (S < 1 || S > kMaxSegments) return KVATTN_ERR_SPLIT;
    return KVATTN_OK;
}


// The sticky status words at st (a workspace's first 256 bytes, or the static scratch's):
// waits for `stream`, reads the merge-timeout count, clears the words on request.
int read_status(unsigned* st, int clear, hipStream_t stream, int* merge_timeouts) {
    unsigned n = 0;
    KV_HIP(hipMemcpyAsync(&n, st + kWsStatusMergeTimeouts, sizeof(n), hipMemcpyDeviceToHost, stream));
    KV_HIP(hipStreamSynchronize(stream));
    if (clear && n != 0) {
        hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(kBlock), 0, stream, (uint32_t*)st,
                           kWsStatusBytes / sizeof(uint32_t));
        KV_HIP(hipGetLastError());
        KV_HIP(hipStreamSynchronize(stream));
    }
    if (merge_timeouts) *merge_timeouts = (int)n;
    return n ? KVATTN_ERR_MERGE_TIMEOUT : KVATTN_OK;
}
}  // namespace

// Shared with the other translation units of the library (not exported).
namespace kvattn_internal {
__attribute__((visibility("hidden"))) void set_last_hip_error(int e) { t_last_hip_error = e; }
__attribute__((visibility("hidden"))) int merge_poll_limit() { return g_merge_polls.load(std::memory_order_relaxed); }
}  // namespace kvattn_internal

// ======================================================================================
// C ABI
// ======================================================================================
extern "C" {

const char* kvattn_strerror(int status) {
    switch (status) {
        case KVATTN_OK: return "ok";
        case KVATTN_ERR_NULL_POINTER: return "a required pointer is NULL";
        case KVATTN_ERR_MISALIGNED: return "a buffer is not 16-byte aligned";
        case KVATTN_ERR_HEAD_DIM: return "head size must be 64";
        case KVATTN_ERR_SHAPE: return "B, NH or maxT out of range";
        case KVATTN_ERR_DTYPE: return "unknown kv dtype or missing kv_scale for an 8-bit cache";
        case KVATTN_ERR_STRATEGY: return "unknown strategy";
        case KVATTN_ERR_WORKSPACE: return "workspace missing or too small";
        case KVATTN_ERR_SPLIT: return "segment count or segment length out of range";
        case KVATTN_ERR_COOP_TOO_LARGE: return "cooperative grid exceeds co-resident capacity";
        case KVATTN_ERR_LDS: return "fused_single scores for maxT exceed the LDS budget";
        case KVATTN_ERR_CAPTURE: return "cooperative launch is not allowed inside stream capture";
        case KVATTN_ERR_LENGTH: return "length hint outside [-1, maxT-1]";
        case KVATTN_ERR_HIP: return "HIP runtime error";
        case KVATTN_ERR_GRID_TOO_LARGE: return "designated-merger grid exceeds what the GPU holds at once";
        case KVATTN_ERR_MERGE_TIMEOUT: return "a merge stopped waiting (designated: computed its producers' segments itself; cooperative: output NaN)";
        default: return "unknown status";
    }
}

int kvattn_last_hip_error(void) { return t_last_hip_error; }

int kvattn_cur_len_symbol(int** d_cur_len) {
    if (!d_cur_len) return KVATTN_ERR_NULL_POINTER;
    const int* p = nullptr;
    KV_TRY(resolve_len(p));
    *d_cur_len = const_cast<int*>(p);
    return KVATTN_OK;
}

int kvattn_set_cur_len(int cur_len) {
    KV_HIP(hipMemcpyToSymbol(HIP_SYMBOL(g_cur_len), &cur_len, sizeof(int), 0, hipMemcpyHostToDevice));
    return KVATTN_OK;
}

int kvattn_set_cur_len_async(int* d_cur_len, int cur_len, void* stream) {
    if (cur_len < 0 || cur_len >= kMaxT) return KVATTN_ERR_LENGTH;
    const int* p = d_cur_len;
    KV_TRY(resolve_len(p));
    hipLaunchKernelGGL(set_len_kernel, dim3(1), dim3(kWave), 0, (hipStream_t)stream, const_cast<int*>(p), cur_len);
    KV_HIP(hipGetLastError());
    return KVATTN_OK;
}

int kvattn_cache_write(void* kv_cache, float* kv_scale, const void* qkv, int B, int NH, int hs, int maxT,
                       const int* d_cur_len, int lens_per_seq, int kv_dtype, void* stream_v) {
    KV_TRY(check_common(qkv, kv_cache, kv_scale, B, NH, hs, maxT, kv_dtype));
    KV_TRY(resolve_len(d_cur_len));
    return launch_cache_write(kv_cache, kv_scale, qkv, B, NH, maxT, d_cur_len, lens_per_seq, kv_dtype, CacheMap{},
                              (hipStream_t)stream_v);
}

int kvattn_append(void* kv_cache, float* kv_scale, const void* qkv, int B, int NH, int hs, int maxT,
                  const int* d_cur_len, int kv_dtype, void* stream) {
    return kvattn_cache_write(kv_cache, kv_scale, qkv, B, NH, hs, maxT, d_cur_len, 0, kv_dtype, stream);
}

int kvattn_paged_cache_write(void* pages, float* page_scales, const int* block_table, int max_pages,
                             int page_rows, int num_pages, const void* qkv, int B, int NH, int hs,
                             const int* d_cur_len, int lens_per_seq, int kv_dtype, void* stream) {
    int maxT = 0;
    KV_TRY(check_paged(block_table, max_pages, page_rows, num_pages, NH, maxT));
    KV_TRY(check_common(qkv, pages, page_scales, B, NH, hs, maxT, kv_dtype));
    KV_TRY(resolve_len(d_cur_len));
    return launch_cache_write(pages, page_scales, qkv, B, NH, maxT, d_cur_len, lens_per_seq, kv_dtype,
                              CacheMap{block_table, max_pages, page_rows, num_pages}, (hipStream_t)stream);
}

int kvattn_paged_decode(void* out, const void* qkv, void* pages, float* page_scales, const int* block_table,
                        int max_pages, int page_rows, int num_pages, int B, int NH, int hs, const int* d_cur_len,
                        int lens_per_seq, int len_hint, void* workspace, size_t workspace_bytes, int S,
                        int strategy, int kv_dtype, int append, void* stream) {
    int maxT = 0;
    KV_TRY(check_paged(block_table, max_pages, page_rows, num_pages, NH, maxT));
    const CacheMap cm{block_table, max_pages, page_rows, num_pages};
    return decode_impl(out, qkv, pages, page_scales, B, NH, hs, maxT, d_cur_len, lens_per_seq, len_hint, workspace,
                       workspace_bytes, S, strategy, kv_dtype, stream, append != 0, &cm);
}

int kvattn_forward_small(void* out, const void* qkv, const void* kv_cache, const float* kv_scale, int B, int NH,
                         int hs, int maxT, const int* d_cur_len, int lens_per_seq, int kv_dtype, void* stream) {
    KV_TRY(check_common(qkv, kv_cache, kv_scale, B, NH, hs, maxT, kv_dtype));
    if (!out) return KVATTN_ERR_NULL_POINTER;
    if (!aligned16(out)) return KVATTN_ERR_MISALIGNED;
    KV_TRY(resolve_len(d_cur_len));
    return launch_fused_single(out, qkv, kv_cache, kv_scale, nullptr, nullptr, B, NH, maxT, d_cur_len,
                               lens_per_seq, 0, 0, kv_dtype, (hipStream_t)stream);
}

int kvattn_forward_large(void* out, const void* qkv, const void* kv_cache, const float* kv_scale, int B, int NH,
                         int hs, int maxT, const int* d_cur_len, int lens_per_seq, float* part_out,
                         float* part_lse, float* part_max, int S, int kv_dtype, void* stream_v) {
    KV_TRY(check_common(qkv, kv_cache, kv_scale, B, NH, hs, maxT, kv_dtype));
    if (!out) return KVATTN_ERR_NULL_POINTER;
    if (!aligned16(out)) return KVATTN_ERR_MISALIGNED;
    KV_TRY(check_partials(part_out, part_lse, part_max, S));
    KV_TRY(resolve_len(d_cur_len));
    hipStream_t stream = (hipStream_t)stream_v;
    SplitArgs a = caller_partials(out, qkv, kv_cache, kv_scale, B, NH, maxT, d_cur_len, lens_per_seq, part_out,
                                  part_lse, part_max, S);
    const bool lat = latency_bound(B, NH, maxT);
    bool capturing = false;
    KV_TRY(stream_capturing(stream, capturing));
    if (B == 1 && !capturing && S <= kMaxDesignatedSegments) {
        // The reference saves the merge launch for B == 1 with a cooperative launch.  On this
        // stack a cooperative dispatch costs ~20 us of GPU time even for an empty kernel
        // (2.4 us for an ordinary one), so the single launch here is the designated merger,
        // over the reference partition.  Its tagged partials live in the library's static
        // scratch array (as kvattn_decode_static's do), so the call only enqueues: no
        // allocation, no synchronisation.  A grid the GPU cannot hold at once, or tags that do
        // not fit in the array, take the split + merge pair over the caller's partials.
        const void* fn = split_ptr_for(a, kv_dtype, kDesignated, lat);
        long long cap = 0;
        if (!fn) return KVATTN_ERR_DTYPE;
        KV_TRY(resident_capacity(fn, split_threads(lat), cap));
        Workspace w{};
        uint8_t* base = nullptr;
        if ((long long)B * NH * S <= cap) {
            KV_TRY(scratch_base(stream, base));
            if (carve_scratch(base, B, NH, S, w)) {
                a.tag_ml = w.tag_ml;
                a.tag_out = w.tag_out;
                a.status = w.status;
                a.barrier = reinterpret_cast<unsigned long long*>(w.status + kWsStatusBarrier);
                a.merge_polls = g_merge_polls.load(std::memory_order_relaxed);
                return launch_split(a, kv_dtype, kDesignated, lat, stream);
            }
        }
    }
    KV_TRY(launch_split(a, kv_dtype, kPartialsOnly, lat, stream));
    return launch_merge(a, kv_dtype, stream);
}

int kvattn_split(float* part_out, float* part_lse, float* part_max, const void* qkv, const void* kv_cache,
                 const float* kv_scale, int B, int NH, int hs, int maxT, const int* d_cur_len, int lens_per_seq,
                 int S, int kv_dtype, void* stream) {
    KV_TRY(check_common(qkv, kv_cache, kv_scale, B, NH, hs, maxT, kv_dtype));
    KV_TRY(check_partials(part_out, part_lse, part_max, S));
    KV_TRY(resolve_len(d_cur_len));
    const SplitArgs a = caller_partials(nullptr, qkv, kv_cache, kv_scale, B, NH, maxT, d_cur_len, lens_per_seq,
                                        part_out, part_lse, part_max, S);
    return launch_split(a, kv_dtype, kPartialsOnly, latency_bound(B, NH, maxT), (hipStream_t)stream);
}

int kvattn_merge(void* out, const float* part_out, const float* part_lse, const float* part_max, int B, int NH,
                 int hs, int S, int kv_dtype, void* stream) {
    if (hs != kHeadDim) return KVATTN_ERR_HEAD_DIM;
    if (B < 1 || NH < 1 || (long long)B * NH > (1ll << 24)) return KVATTN_ERR_SHAPE;
    if (kv_dtype < KVATTN_KV_F32 || kv_dtype > KVATTN_KV_FP8_E4M3) return KVATTN_ERR_DTYPE;
    if (!out) return KVATTN_ERR_NULL_POINTER;
    if (!aligned16(out)) return KVATTN_ERR_MISALIGNED;
    KV_TRY(check_partials(part_out, part_lse, part_max, S));
    SplitArgs a = caller_partials(out, nullptr, nullptr, nullptr, B, NH, 1, nullptr, 0,
                                  const_cast<float*>(part_out), const_cast<float*>(part_lse),
                                  const_cast<float*>(part_max), S);
    return launch_merge(a, kv_dtype, (hipStream_t)stream);
}

size_t kvattn_workspace_bytes(int B, int NH, int hs, int maxT, int S) {
    if (hs != kHeadDim || B < 1 || NH < 1 || maxT < 1 || maxT > kMaxT) return 0;
    int slots = 0, seg_rows = 0;
    if (segment_slots(maxT, S, slots, seg_rows) != KVATTN_OK) return 0;
    return carve(nullptr, B, NH, slots).bytes;
}

int kvattn_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
    if (!workspace) return KVATTN_ERR_NULL_POINTER;
    if (!aligned16(workspace)) return KVATTN_ERR_MISALIGNED;
    // A fill kernel rather than hipMemsetAsync, so that the call may also sit in a graph.
    const size_t words = workspace_bytes / 4;
    if (words == 0) return KVATTN_OK;
    const size_t blocks = std::min<size_t>((words + kBlock - 1) / kBlock, 4096);
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)blocks), dim3(kBlock), 0, (hipStream_t)stream,
                       (uint32_t*)workspace, words);
    KV_HIP(hipGetLastError());
    return KVATTN_OK;
}

int kvattn_workspace_status(void* workspace, size_t workspace_bytes, int clear, void* stream_v,
                            int* merge_timeouts) {
    if (!workspace) return KVATTN_ERR_NULL_POINTER;
    if (!aligned16(workspace)) return KVATTN_ERR_MISALIGNED;
    if (workspace_bytes < kWsStatusBytes) return KVATTN_ERR_WORKSPACE;
    return read_status((unsigned*)workspace, clear, (hipStream_t)stream_v, merge_timeouts);
}

int kvattn_call_identity(unsigned long long* out, void* stream) {
    if (!out) return KVATTN_ERR_NULL_POINTER;
    if ((uintptr_t)out & 7u) return KVATTN_ERR_MISALIGNED;
    hipLaunchKernelGGL(call_identity_kernel, dim3(1), dim3(kWave), 0, (hipStream_t)stream, out);
    KV_HIP(hipGetLastError());
    return KVATTN_OK;
}

int kvattn_scratch_status(int clear, void* stream_v, int* merge_timeouts) {
    hipStream_t stream = (hipStream_t)stream_v;
    uint8_t* base = nullptr;
    KV_TRY(scratch_base(stream, base));
    return read_status((unsigned*)base, clear, stream, merge_timeouts);
}

int kvattn_set_xcd_layout_offset(int rot) { return g_xcd_rot.exchange(rot & 7); }

int kvattn_set_merge_poll_limit(int polls) {
    return g_merge_polls.exchange(polls < 0 ? kDefaultMergePolls : polls);
}

int kvattn_plan(int B, int NH, int hs, int maxT, int len_hint, int S, int strategy, int kv_dtype,
                int* strategy_out, int* segments_out, int* seg_rows_out) {
    if (hs != kHeadDim) return KVATTN_ERR_HEAD_DIM;
    if (B < 1 || NH < 1 || maxT < 1 || maxT > kMaxT || (long long)B * NH > (1ll << 24)) return KVATTN_ERR_SHAPE;
    if (kv_dtype < KVATTN_KV_F32 || kv_dtype > KVATTN_KV_FP8_E4M3) return KVATTN_ERR_DTYPE;
    if (!strategy_out || !segments_out || !seg_rows_out) return KVATTN_ERR_NULL_POINTER;
    Plan p{};
    KV_TRY(make_plan(B, NH, maxT, len_hint, S, strategy, kv_dtype, p));
    *strategy_out = p.strategy;
    *segments_out = p.slots;
    *seg_rows_out = p.seg_rows < 0 ? -1 : p.seg_rows;
    return KVATTN_OK;
}

int kvattn_decode(void* out, const void* qkv, const void* kv_cache, const float* kv_scale, int B, int NH, int hs,
                  int maxT, const int* d_cur_len, int lens_per_seq, int len_hint, void* workspace,
                  size_t workspace_bytes, int S, int strategy, int kv_dtype, void* stream) {
    return decode_impl(out, qkv, kv_cache, kv_scale, B, NH, hs, maxT, d_cur_len, lens_per_seq, len_hint,
                       workspace, workspace_bytes, S, strategy, kv_dtype, stream, false);
}

int kvattn_decode_static(void* out, const void* qkv, const void* kv_cache, const float* kv_scale, int B, int NH,
                         int hs, int maxT, const int* d_cur_len, int lens_per_seq, int len_hint, int S, int strategy,
                         int kv_dtype, void* stream) {
    return decode_impl(out, qkv, kv_cache, kv_scale, B, NH, hs, maxT, d_cur_len, lens_per_seq, len_hint, nullptr, 0,
                       S, strategy, kv_dtype, stream, false, nullptr, true);
}

int kvattn_append_decode(void* out, const void* qkv, void* kv_cache, float* kv_scale, int B, int NH, int hs,
                         int maxT, const int* d_cur_len, int lens_per_seq, int len_hint, void* workspace,
                         size_t workspace_bytes, int S, int strategy, int kv_dtype, void* stream) {
    return decode_impl(out, qkv, kv_cache, kv_scale, B, NH, hs, maxT, d_cur_len, lens_per_seq, len_hint,
                       workspace, workspace_bytes, S, strategy, kv_dtype, stream, true);
}

}  // extern "C"
