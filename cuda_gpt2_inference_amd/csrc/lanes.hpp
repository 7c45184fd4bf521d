// lanes.hpp -- wave64 building blocks shared by the gfx950 kernels of this library:
// bfloat16 and 8-bit code conversion, the append's 8-bit row quantiser, 16-byte lane loads
// and DPP / permlane reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kvattn.h"
#include "layout.hpp"

// The 64-bit dispatch id of the running kernel dispatch (LLVM's llvm.amdgcn.dispatch.id; it
// has no clang builtin).  Kernels that call it receive it in two user SGPRs at wave launch.
extern "C" __device__ unsigned long long kvattn_dispatch_id() __asm("llvm.amdgcn.dispatch.id");

namespace {

constexpr int kWave = 64;

// ------------------------------------------------------------------------------------
// Element helpers.
// ------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// float -> bfloat16 bits, round to nearest even; NaN stays a quiet NaN.  Written as a select
// rather than an early return, so that it compiles without a branch.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    const uint32_t quiet = (u >> 16) | 0x40u;
    return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? quiet : rounded);
}

// Sixteen 8-bit codes of one 16-byte chunk as floats: FP8 through the hardware OCP E4M3
// conversion (v_cvt_pk_f32_fp8), INT8 by sign extension.
template <bool kFp8>
__device__ __forceinline__ void decode_codes(const uint4& d, float (&x)[16]) {
    const uint32_t w[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (kFp8) {
            const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], false);
            const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], true);
            x[4 * i] = lo[0]; x[4 * i + 1] = lo[1]; x[4 * i + 2] = hi[0]; x[4 * i + 3] = hi[1];
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) x[4 * i + k] = (float)(int8_t)(w[i] >> (8 * k));
        }
    }
}

// 16-byte row-chunk load; KVATTN_NT_LOADS=1 marks K/V loads non-temporal (streamed once).
#ifndef KVATTN_NT_LOADS
#define KVATTN_NT_LOADS 1
#endif
__device__ __forceinline__ uint4 load16(const uint8_t* p) {
#if KVATTN_NT_LOADS
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
#else
    return *reinterpret_cast<const uint4*>(p);
#endif
}

// ------------------------------------------------------------------------------------
// Cross-lane reductions.  DPP control words (GFX9 encoding).
// ------------------------------------------------------------------------------------
constexpr int kDppQuadXor1 = 0xB1;    // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;    // quad_perm [2,3,0,1]
constexpr int kDppRowRor4 = 0x124;    // rotate 16-lane row by 4
constexpr int kDppRowRor8 = 0x128;    // rotate 16-lane row by 8
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i inside each 8-lane half row
constexpr int kDppRowMirror = 0x140;  // lane i <-> 15-i inside each 16-lane row
constexpr int kDppQuadRev = 0x1B;     // quad_perm [3,2,1,0]

template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xF, 0xF, true));
}

// Sum over the kLanes lanes holding one row (aligned groups of 4, 8 or 16 lanes).
template <int kLanes>
__device__ __forceinline__ float row_sum(float x) {
    x += dpp<kDppQuadXor1>(x);
    x += dpp<kDppQuadXor2>(x);
    if constexpr (kLanes >= 8) x += dpp<kDppHalfMirror>(x);
    if constexpr (kLanes >= 16) x += dpp<kDppRowMirror>(x);
    return x;
}

// op(x, x of lane ^ 16) and op(x, x of lane ^ 32) with the gfx950 row-swap permutes:
// permlane16_swap / permlane32_swap of x with itself return x with 16-lane rows (resp.
// 32-lane halves) exchanged in one of the two results, so op over both outputs is op
// over the lane pair.
template <bool kMax>
__device__ __forceinline__ float op_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
    return kMax ? fmaxf(a, b) : a + b;
}
template <bool kMax>
__device__ __forceinline__ float op_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
    return kMax ? fmaxf(a, b) : a + b;
}

// Reduce over the lanes that hold the same channel slice of different rows
// (lane = row_slot * kLanes + slice): every lane receives the result for its slice.
template <int kLanes, bool kMax>
__device__ __forceinline__ float slot_reduce(float x) {
    auto op = [](float a, float b) { return kMax ? fmaxf(a, b) : a + b; };
    if constexpr (kLanes == 4) { x = op(x, dpp<kDppRowRor4>(x)); x = op(x, dpp<kDppRowRor8>(x)); }
    if constexpr (kLanes == 8) { x = op(x, dpp<kDppRowRor8>(x)); }
    x = op_xor16<kMax>(x);
    x = op_xor32<kMax>(x);
    return x;
}

// Maximum over aligned groups of kLanes (4, 8 or 16) lanes: the first steps of wave_max, so
// that a group whose other lanes hold -FLT_MAX gets wave_max's result bit for bit.
template <int kLanes>
__device__ __forceinline__ float row_max(float x) {
    x = fmaxf(x, dpp<kDppQuadXor1>(x));
    x = fmaxf(x, dpp<kDppQuadXor2>(x));
    if constexpr (kLanes >= 8) x = fmaxf(x, dpp<kDppHalfMirror>(x));
    if constexpr (kLanes >= 16) x = fmaxf(x, dpp<kDppRowMirror>(x));
    return x;
}

// Reduce-scatter over the row slots of a wave.  Lane = slot * kLanes + slice holds, for its
// row slot, kElems values: elements 0 .. kElems-1 of its slice.  There are as many row slots
// as elements (64 / kLanes = kElems), so afterwards each lane returns one sum over all row
// slots: element `slot` of its slice, channel slice * kElems + slot.  Each step pairs lanes that
// differ in one slot bit; the lane with the bit clear keeps the lower half of its values, its
// partner the upper half, and each adds the half that its partner sends.  permlane32_swap and
// permlane16_swap of (lower, upper) hand both operands of those sums over in one instruction
// (the lane with the bit clear receives its partner's lower half, and the partner the upper);
// inside a 16-lane row, row_ror:8 pairs lanes 8 apart, and a quad reversal followed by a
// half-row mirror pairs lanes 4 apart.
template <int kLanes, int kElems>
__device__ __forceinline__ float slot_reduce_scatter(float (&a)[kElems]) {
    static_assert(kLanes * kElems == kWave && kElems >= 4 && kElems <= 16, "one channel per lane");
    const int lane = threadIdx.x & (kWave - 1);
    constexpr int h32 = kElems / 2, h16 = kElems / 4, h8 = kElems / 8, h4 = kElems / 16;
#pragma unroll
    for (int i = 0; i < h32; ++i) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[i]), __float_as_uint(a[h32 + i]), false,
                                                        false);
        a[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int i = 0; i < h16; ++i) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a[i]), __float_as_uint(a[h16 + i]), false,
                                                        false);
        a[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    if constexpr (h8 > 0) {
        const bool hi = (lane & 8) != 0;
#pragma unroll
        for (int i = 0; i < h8; ++i) {
            const float send = hi ? a[i] : a[h8 + i];
            a[i] = (hi ? a[h8 + i] : a[i]) + dpp<kDppRowRor8>(send);
        }
    }
    if constexpr (h4 > 0) {
        const bool hi = (lane & 4) != 0;
        const float send = hi ? a[0] : a[1];
        a[0] = (hi ? a[1] : a[0]) + dpp<kDppHalfMirror>(dpp<kDppQuadRev>(send));
    }
    return a[0];
}

__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp<kDppQuadXor1>(x));
    x = fmaxf(x, dpp<kDppQuadXor2>(x));
    x = fmaxf(x, dpp<kDppHalfMirror>(x));
    x = fmaxf(x, dpp<kDppRowMirror>(x));
    x = op_xor16<true>(x);
    x = op_xor32<true>(x);
    return x;
}

__device__ __forceinline__ float wave_sum(float x) {
    x += dpp<kDppQuadXor1>(x);
    x += dpp<kDppQuadXor2>(x);
    x += dpp<kDppHalfMirror>(x);
    x += dpp<kDppRowMirror>(x);
    x = op_xor16<false>(x);
    x = op_xor32<false>(x);
    return x;
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }


// OCP E4M3 ("FN": max 448, no infinities) encode of y, round to nearest even, finite
// overflow saturates to +-448 (the reference's __NV_SATFINITE request).
__device__ __forceinline__ uint8_t f32_to_e4m3_sat(float y) {
    if (y != y) return 0x7F;
    const uint32_t sign = (__float_as_uint(y) >> 24) & 0x80u;
    const float a = fabsf(y);
    if (a >= 448.0f) return (uint8_t)(sign | 0x7Eu);
    if (a < 0.015625f) {                       // subnormal grid m * 2^-9; 8 -> 2^-6
        return (uint8_t)(sign | (uint32_t)rintf(a * 512.0f));
    }
    const uint32_t u = __float_as_uint(a);
    uint32_t keep = u >> 20;                   // exponent | top 3 mantissa bits
    const uint32_t rem = u & 0xFFFFFu;
    keep += (rem > 0x80000u || (rem == 0x80000u && (keep & 1u))) ? 1u : 0u;
    uint32_t code = keep - (120u << 3);        // rebias 127 -> 7
    code = code > 0x7Eu ? 0x7Eu : code;
    return (uint8_t)(sign | code);
}

// 8-bit row quantisation of the append: scale = amax / limit (IEEE division), code of
// x / scale (INT8: round half to even, clamp to +-127; FP8: saturating E4M3), and zero
// codes when the scale is not positive (an all-zero row).
template <int DT> constexpr float kW8Limit = DT == KVATTN_KV_FP8_E4M3 ? 448.0f : 127.0f;

template <int DT>
__device__ __forceinline__ uint8_t w8_code(float x, float scale) {
    if (!(scale > 0.0f)) return 0;
    const float y = x / scale;
    if constexpr (DT == KVATTN_KV_FP8_E4M3) {
        return f32_to_e4m3_sat(y);
    } else {
        int qv = (int)rintf(y);
        qv = qv < -127 ? -127 : (qv > 127 ? 127 : qv);
        return (uint8_t)(int8_t)qv;
    }
}

// ------------------------------------------------------------------------------------
// Tagged words handed between workgroups: a float in the low half, the call's tag in the
// high half.  A word counts only for the dispatch that wrote it, so slots need no clearing.
// Published with plain stores when writer and reader run on one XCD (the word lands in that
// XCD's L2, where the reader's agent-scope loads hit it), else with write-through (sc1)
// stores, which agent-scope loads see from any XCD.
//
// The tag is the dispatch id plus a per-queue offset, with the top bit set (so that a zeroed
// buffer holds no valid word).  Dispatch ids count packets per HSA queue: every queue starts
// at 0, and HIP spreads its streams over several queues (4 here), so two streams' calls carry
// equal ids all the time.  The offset, a multiplicative hash of the queue's address (the
// queue pointer the dispatch arrives with), keeps those apart: on one queue the tags of 2^31
// consecutive dispatches are distinct; a word from another queue matches only when the two
// queues' dispatch counts differ by exactly the difference of their offsets (mod 2^31), a
// pseudo-random value fixed per pair of queues.
// ------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t queue_salt() {
    const uint64_t q = (uint64_t)(uintptr_t)__builtin_amdgcn_queue_ptr();
    return (uint32_t)(((q >> 6) * 0x9E3779B97F4A7C15ull) >> 32);
}
__device__ __forceinline__ uint32_t call_tag() {
    return ((uint32_t)kvattn_dispatch_id() + queue_salt()) | 0x80000000u;
}

// The XCD (accelerator complex die) this wave runs on: HW_REG_XCC_ID bits 3:0.
__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & 0xFu;
}
__device__ __forceinline__ void publish_word(unsigned long long* p, unsigned long long w, bool xcd_local) {
    if (xcd_local) *p = w;
    else __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long get_word(const unsigned long long* p) {
    return __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long tagged_word(float v, uint32_t tag) {
    return ((unsigned long long)tag << 32) | __float_as_uint(v);
}
__device__ __forceinline__ bool word_is(unsigned long long w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }
__device__ __forceinline__ float word_value(unsigned long long w) { return __uint_as_float((uint32_t)w); }

using kvattn_layout::dense_slot;
using kvattn_layout::div_uniform;
using kvattn_layout::guess_rows;
using kvattn_layout::guess_slot_live;
using kvattn_layout::xcd_slot;
using kvattn_layout::xcd_slot_rotated;

// s_waitcnt vmcnt(0) (GFX9 encoding: expcnt and lgkmcnt fields left at their maximum),
// fenced against compiler reordering on both sides.
__device__ __forceinline__ void wait_vm_stores() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

}  // namespace
