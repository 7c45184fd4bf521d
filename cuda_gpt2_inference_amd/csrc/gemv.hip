// gemv.hip -- the decode step's fully connected layer on MI355X (gfx950, wave64):
// out[b][m] = act(scale_m * sum_k W[m][k] x[b][k] + bias[m]), act = identity or GPT-2's
// tanh GELU, for FP32, BF16 and 8-bit (INT8 / FP8-E4M3 codes with one FP32 scale per row)
// weights.  The attention output projection consumes the attention output this way.
//
// One wave per kR output rows (kR = 1 for the per-layer shapes; for tall matrices such as
// the vocabulary projection 4 with 8-bit weights, 2 otherwise).  A row of K weights is K*wbytes/16 chunks of 16
// bytes; lane l holds chunks l, l+64, ... of a block of 64*kC chunks of each of its rows in
// registers (all requested at once), multiplies them with the matching x chunks of every
// input vector, and a wave reduction (DPP + permlane) finishes each dot product.  Rows longer
// than one block loop over blocks.  At GPT-2's per-layer sizes (0.6 to 4.7 MB of weights) a
// call is bound by launch and memory latency, and one row per wave gives the most waves; a
// tall matrix (50304 x 768) streams, and 2-4 rows per wave keep 3-6 KB per wave in flight.
// MFMA is not used (B is a handful of decode tokens, 1-2 flops per byte).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "kvattn.h"
#include "lanes.hpp"

namespace {

constexpr int kGemvWaves = 4;          // waves per workgroup
constexpr int kGemvMaxChunks = 16;     // 16-byte weight chunks per lane and row in one block
constexpr int kGemvMaxRowChunks = 16;  // kR * kC: weight registers of a wave (64 VGPRs)

template <int WT> struct WFmt;
template <> struct WFmt<KVATTN_KV_F32> {   // x, bias, out: float
    static constexpr int kWBytes = 4, kElems = 4, kXBytes = 16;
    static constexpr bool kActF32 = true, k8bit = false;
};
template <> struct WFmt<KVATTN_KV_BF16> {  // x, bias, out: bf16
    static constexpr int kWBytes = 2, kElems = 8, kXBytes = 16;
    static constexpr bool kActF32 = false, k8bit = false;
};
template <> struct WFmt<KVATTN_KV_INT8> {  // x, bias, out: bf16
    static constexpr int kWBytes = 1, kElems = 16, kXBytes = 32;
    static constexpr bool kActF32 = false, k8bit = true;
};
template <> struct WFmt<KVATTN_KV_FP8_E4M3> {
    static constexpr int kWBytes = 1, kElems = 16, kXBytes = 32;
    static constexpr bool kActF32 = false, k8bit = true;
};

struct GemvArgs {
    void* out;
    void* pre_gelu;
    const uint8_t* W;
    const float* w_scale;
    const uint8_t* x;
    const void* bias;
    int B, M, K, gelu;
    // QKV projection with the KV append in its epilogue (kv != nullptr): out is qkv
    // [B][3][NH][64], and its K and V rows also go to column cur_len of the cache
    // [2][B][NH][maxT][64], in the activation type or (kv_dtype 8-bit) as codes with a row
    // scale in kv_scale [2][B][NH][maxT].  8-bit rows pass through `words` (tagged u64
    // [B][2][NH][64]), their wait bounded by `polls`.
    uint8_t* kv;
    const int* cur_len;
    int lens_per_seq, NH, maxT;
    int kv_dtype;
    float* kv_scale;
    unsigned long long* words;
    int polls;
};

// The x values one 16-byte weight chunk multiplies: 16 bytes (4 floats or 8 bf16), or 32
// bytes (16 bf16) for 8-bit weights.
template <int WT>
struct XRaw {
    uint4 v[WFmt<WT>::kXBytes / 16];
};

template <int WT>
__device__ __forceinline__ XRaw<WT> load_x(const uint8_t* xp) {
    XRaw<WT> r;
#pragma unroll
    for (int h = 0; h < WFmt<WT>::kXBytes / 16; ++h) r.v[h] = reinterpret_cast<const uint4*>(xp)[h];
    return r;
}

// Dot product of one 16-byte weight chunk with the x values it multiplies.
template <int WT>
__device__ __forceinline__ float chunk_dot(const uint4& w, const XRaw<WT>& xr) {
    using F = WFmt<WT>;
    float wf[F::kElems], xf[F::kElems];
    if constexpr (WT == KVATTN_KV_F32) {
        const uint4 xv = xr.v[0];
        wf[0] = __uint_as_float(w.x); wf[1] = __uint_as_float(w.y);
        wf[2] = __uint_as_float(w.z); wf[3] = __uint_as_float(w.w);
        xf[0] = __uint_as_float(xv.x); xf[1] = __uint_as_float(xv.y);
        xf[2] = __uint_as_float(xv.z); xf[3] = __uint_as_float(xv.w);
    } else if constexpr (WT == KVATTN_KV_BF16) {
        const uint4 xv = xr.v[0];
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w}, xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            wf[2 * i] = bf16_lo(ww[i]); wf[2 * i + 1] = bf16_hi(ww[i]);
            xf[2 * i] = bf16_lo(xw[i]); xf[2 * i + 1] = bf16_hi(xw[i]);
        }
    } else {
        decode_codes<WT == KVATTN_KV_FP8_E4M3>(w, wf);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint4 xv = xr.v[h];
            const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xf[8 * h + 2 * i] = bf16_lo(xw[i]);
                xf[8 * h + 2 * i + 1] = bf16_hi(xw[i]);
            }
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < F::kElems; ++e) s = fmaf(wf[e], xf[e], s);
    return s;
}

template <int WT>
__device__ __forceinline__ float load_act(const void* p, size_t i) {
    if constexpr (WFmt<WT>::kActF32) return reinterpret_cast<const float*>(p)[i];
    else return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

template <int WT>
__device__ __forceinline__ void store_act(void* p, size_t i, float v) {
    if constexpr (WFmt<WT>::kActF32) reinterpret_cast<float*>(p)[i] = v;
    else reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
}

// out / pre_gelu element: float or bf16 (the output type may differ from the activations,
// as in the reference's float logits over bf16 activations).
template <bool kOutF32>
__device__ __forceinline__ void store_res(void* p, size_t i, float v) {
    if constexpr (kOutF32) reinterpret_cast<float*>(p)[i] = v;
    else reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
}

// GPT-2's GELU, tanh form: 0.5 v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3))).
__device__ __forceinline__ float gelu_tanh(float v) {
    const float cube = 0.044715f * v * v * v;
    return 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + cube)));
}

constexpr int kHd = 64;   // head size of the QKV epilogue
constexpr int kHeadRowGroups = kHd / kGemvWaves;   // workgroups of one head row (64 channels, one row per wave)
// The epilogue of a launch (a template parameter, so that the plain GEMV carries none of it).
enum GemvEpilogue { kEpiNone = 0, kEpiAppend = 1, kEpiAppend8 = 2 };
// Bits of the preloaded M argument above the row count (M < 2^29): GELU, and the XCD-local
// layout of kEpiAppend8.
constexpr int kGeluFlag = 1 << 29, kXcdLocalFlag = 1 << 30, kRowMask = (1 << 29) - 1;

// Cache row (in units of kHd elements) of part 1 (K) or 2 (V), head h, sequence b at the
// position being appended: column cur_len, clamped to [0, maxT - 1] as the append does.
// len0: cur_len[0], loaded ahead with the weights.
__device__ __forceinline__ size_t cache_row(const GemvArgs& a, int b, int part, int h, int len0) {
    int cl = a.lens_per_seq && b > 0 ? a.cur_len[b] : len0;
    cl = cl < 0 ? 0 : (cl > a.maxT - 1 ? a.maxT - 1 : cl);
    size_t row = ((size_t)b * a.NH + h) * a.maxT + cl;
    if (part == 2) row += (size_t)a.B * a.NH * a.maxT;
    return row;
}

// The weights, x, scales, bias, shape and output also come as leading scalar parameters
// (13 dwords, preloaded into SGPRs at wave launch: the library is built with kernel-argument
// preloading), so the weight and x loads issue without a scalar load of the argument block.
// kC: 16-byte chunks per lane and row in one block of the row; kR: rows per wave; kOutF32:
// out and pre_gelu as float (else bf16); kEpi: the QKV epilogue (GemvEpilogue).  Rows of more
// than 64*kC chunks take several blocks (the weights are then read again for each input
// vector).  pk_M: the rows M with the GELU and XCD-local flags in bits 29 and 30.  The 8-bit
// epilogue takes the dispatch id and the queue pointer (its tag) in user SGPRs, which leaves 10
// dwords of preloaded arguments: W, x, the scales, the bias, M and K, all its first loads
// need; B and out follow.
template <int WT, int kC, int kR, bool kOutF32, int kEpi>
__global__ __launch_bounds__(kGemvWaves * kWave) void gemv_kernel(const uint8_t* pk_W, const uint8_t* pk_x,
                                                                  const float* pk_w_scale, const void* pk_bias,
                                                                  int pk_M, int pk_K, int pk_B, void* pk_out,
                                                                  GemvArgs a) {
    static_assert(kR * kC <= kGemvMaxRowChunks && (kR == 1 || kR == 2 || kR == 4), "weight registers");
    static_assert(kEpi == kEpiNone || kR == 1, "the QKV epilogue takes one row per wave");
    a.W = pk_W;
    a.x = pk_x;
    a.w_scale = pk_w_scale;
    a.bias = pk_bias;
    a.B = pk_B;
    // B >= 1 (the host checks it): without it the code generator tests B before the first
    // weight load, which would then wait for B's scalar load whenever B is not preloaded.
    __builtin_assume(a.B >= 1);
    a.M = pk_M & kRowMask;
    a.K = pk_K;
    a.out = pk_out;
    a.gelu = (pk_M & kGeluFlag) != 0;
    using F = WFmt<WT>;
    const int lane = threadIdx.x & (kWave - 1);
    // With 4 rows per wave the row index is made wave-uniform (an SGPR), so the rows' base
    // addresses, scales and bias are scalar: 61 VGPRs and 8 waves per SIMD for 8-bit weights
    // (81 and 5 without).  At 1-2 rows per wave the vector form measured faster.
    const int wave = kR == 4 ? (int)__builtin_amdgcn_readfirstlane(threadIdx.x / kWave) : (int)(threadIdx.x / kWave);
    // kEpiAppend8 with the XCD-local layout: the 16 workgroups of a head row share an XCD.
    const bool xl = kEpi == kEpiAppend8 && (pk_M & kXcdLocalFlag) != 0;
    const int wg = xl ? xcd_slot(blockIdx.x, kHeadRowGroups) : (int)blockIdx.x;
    const int m0 = (wg * kGemvWaves + wave) * kR;
    if (m0 >= a.M) return;   // whole wave (no barrier follows)
    const int nch = a.K * F::kWBytes / 16;
    constexpr int kBlk = kWave * kC;                 // chunks of a row in one block
    const int nblk = (nch + kBlk - 1) / kBlk;
    const size_t row_bytes = (size_t)a.K * F::kWBytes;
    // Every load is unconditional, so that all of them issue before the first wait: a lane's
    // chunks beyond the row (c >= nch) read chunk nch - 1 again and their products are
    // dropped by a select, and rows beyond M (the last wave of a kR > 1 grid) read row M - 1
    // and are not stored.  (Loads behind branches make the code generator wait for each one
    // before the next: one memory round trip per chunk.)  The weights are read once per
    // call and marked non-temporal (vocabulary projection, 50304 x 768: -3 % INT8, -6 %
    // BF16, -9 % FP32 per call; the per-layer shapes within +-0.05 us).
    uint4 w[kR][kC];
    auto load_w = [&](int kb) {
#pragma unroll
        for (int r = 0; r < kR; ++r) {
            const uint8_t* wrow = a.W + (size_t)min(m0 + r, a.M - 1) * row_bytes;
#pragma unroll
            for (int i = 0; i < kC; ++i)
                w[r][i] = load16(wrow + (size_t)min(kb * kBlk + lane + i * kWave, nch - 1) * 16);
        }
    };
    load_w(0);
    constexpr int kActBytes = F::kActF32 ? 4 : 2;
    // x of the first vector and the bias are requested right behind the weights, before
    // anything waits (the weights' unpacking, which the code generator hoists out of the
    // vector loop, waits for the weights only).
    XRaw<WT> xr[kC];
    auto load_xs = [&](int b, int kb) {
        const uint8_t* xb = a.x + (size_t)b * a.K * kActBytes;
#pragma unroll
        for (int i = 0; i < kC; ++i)
            xr[i] = load_x<WT>(xb + (size_t)min(kb * kBlk + lane + i * kWave, nch - 1) * F::kXBytes);
    };
    load_xs(0, 0);
    float bias[kR], ws[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) {
        const int mr = min(m0 + r, a.M - 1);
        const float braw = load_act<WT>(a.bias ? a.bias : (const void*)a.x, a.bias ? mr : 0);
        bias[r] = a.bias ? braw : 0.0f;
        ws[r] = F::k8bit ? a.w_scale[mr] : 1.0f;
    }
    const int len0 = kEpi != kEpiNone ? a.cur_len[0] : 0;   // the QKV epilogue's column
    for (int b = 0; b < a.B; ++b) {
        float accr[kR];
#pragma unroll
        for (int r = 0; r < kR; ++r) accr[r] = 0.0f;
        for (int kb = 0; kb < nblk; ++kb) {
            if (kb > 0 || b > 0) {
                if (nblk > 1) load_w(kb);   // one block: the weights stay in registers for every vector
                load_xs(b, kb);
            }
#pragma unroll
            for (int r = 0; r < kR; ++r) {
#pragma unroll
                for (int i = 0; i < kC; ++i) {
                    const float d = accr[r] + chunk_dot<WT>(w[r][i], xr[i]);
                    accr[r] = kb * kBlk + lane + i * kWave < nch ? d : accr[r];
                }
            }
        }
#pragma unroll
        for (int r = 0; r < kR; ++r) accr[r] = wave_sum(accr[r]);
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < kR; ++r) {
                const int m = m0 + r;
                if (m >= a.M) break;
                float pre = accr[r] * ws[r] + bias[r];
                const size_t o = (size_t)b * a.M + m;
                if (a.pre_gelu) store_res<kOutF32>(a.pre_gelu, o, pre);
                if (a.gelu) pre = gelu_tanh(pre);
                store_res<kOutF32>(a.out, o, pre);
                if constexpr (kEpi == kEpiAppend) {
                    // Output m is channel c of head h of part q/k/v; K and V also land in the cache
                    // row of position cur_len, as the separate append would copy them.
                    const int part = m / (a.NH * kHd);
                    if (part > 0) {
                        const int h = (m - part * a.NH * kHd) / kHd, c = m - part * a.NH * kHd - h * kHd;
                        store_act<WT>(a.kv, cache_row(a, b, part, h, len0) * kHd + c, pre);
                    }
                }
            }
        }
        if constexpr (kEpi == kEpiAppend8) {
            // An 8-bit row's scale needs the amax of the head's 64 channels, which the 64 waves of
            // 16 workgroups compute.  Each wave publishes its channel's value (the bf16 value the
            // qkv output holds, which the append quantises) as a tagged word; the wave of channel
            // 0 (workgroup 0 of the head row, first in dispatch order) polls the row's 64 words,
            // lane c channel c, and quantises it with the append's arithmetic (the same
            // function).  With the XCD-local layout the words stay in the XCD's L2 (plain
            // stores, agent-scope loads).  The wait is bounded (a.polls rounds): channels still
            // missing then are computed by this wave itself, row by row with the producers'
            // arithmetic, so the codes never depend on where or when the producers run.
            const int m = m0;
            const int part = m / (a.NH * kHd);
            if (part > 0) {
                const int h = (m - part * a.NH * kHd) / kHd, c = m - part * a.NH * kHd - h * kHd;
                const size_t rid = ((size_t)b * 2 + (part - 1)) * a.NH + h;
                unsigned long long* row_words = a.words + rid * kHd;
                const uint32_t tag = call_tag();
                const float v = bf16_to_f32(f32_to_bf16(accr[0] * ws[0] + bias[0]));
                if (lane == 0) publish_word(row_words + c, tagged_word(v, tag), xl);
                if (c == 0) {
                    unsigned long long wv = 0;
                    bool ok = false;
                    for (int r = 0; r < a.polls; ++r) {
                        wv = get_word(row_words + lane);
                        ok = word_is(wv, tag);
                        if (__all(ok)) break;
                    }
                    float x = word_value(wv);
                    unsigned long long missing = __ballot(!ok);
                    // Fallback: the missing channels, one row at a time (the wave's chunks, the
                    // same order of sums as the wave that owns the row).
                    while (missing) {
                        const int cm = __ffsll((long long)missing) - 1;
                        missing &= missing - 1;
                        const int mr = m + cm;
                        const uint8_t* wrow = a.W + (size_t)mr * row_bytes;
                        const uint8_t* xb = a.x + (size_t)b * a.K * kActBytes;
                        float acc = 0.0f;
                        for (int kb = 0; kb < nblk; ++kb) {
                            uint4 wr[kC];
                            XRaw<WT> xq[kC];
#pragma unroll
                            for (int i = 0; i < kC; ++i) {
                                const int ci = min(kb * kBlk + lane + i * kWave, nch - 1);
                                wr[i] = load16(wrow + (size_t)ci * 16);
                                xq[i] = load_x<WT>(xb + (size_t)ci * F::kXBytes);
                            }
#pragma unroll
                            for (int i = 0; i < kC; ++i) {
                                const float d = acc + chunk_dot<WT>(wr[i], xq[i]);
                                acc = kb * kBlk + lane + i * kWave < nch ? d : acc;
                            }
                        }
                        acc = wave_sum(acc);
                        const float wsr = F::k8bit ? a.w_scale[mr] : 1.0f;
                        const float br = a.bias ? load_act<WT>(a.bias, mr) : 0.0f;
                        const float vr = bf16_to_f32(f32_to_bf16(acc * wsr + br));
                        x = lane == cm ? vr : x;
                    }
                    const float amax = wave_max(fabsf(x));
                    const size_t row = cache_row(a, b, part, h, len0);
                    if (a.kv_dtype == KVATTN_KV_FP8_E4M3) {
                        const float scale = amax / kW8Limit<KVATTN_KV_FP8_E4M3>;
                        a.kv[row * kHd + lane] = w8_code<KVATTN_KV_FP8_E4M3>(x, scale);
                        if (lane == 0) a.kv_scale[row] = scale;
                    } else {
                        const float scale = amax / kW8Limit<KVATTN_KV_INT8>;
                        a.kv[row * kHd + lane] = w8_code<KVATTN_KV_INT8>(x, scale);
                        if (lane == 0) a.kv_scale[row] = scale;
                    }
                }
            }
        }
    }
}

// Rows per wave: one for the per-layer shapes (latency bound: the most waves); from
// kGemvTallRows rows on (bandwidth bound: more bytes in flight per wave) 4 for 8-bit weights
// and 2 for the wider ones, the most that keep 8 waves per SIMD.  kC: chunks per
// lane and row in one block, the fewest that hold the row, at most kGemvMaxRowChunks / kR
// (longer rows loop over blocks).
#ifndef KVATTN_GEMV_TALL_ROWS
#define KVATTN_GEMV_TALL_ROWS 8192
#endif
constexpr int kGemvTallRows = KVATTN_GEMV_TALL_ROWS;

template <int WT, bool kOut, int kEpi>
const void* gemv_ptr(int chunks_per_lane, int rows) {
    if constexpr (kEpi == kEpiNone) {
        if constexpr (WFmt<WT>::k8bit) {
            if (rows == 4) {
                if (chunks_per_lane <= 1) return (const void*)&gemv_kernel<WT, 1, 4, kOut, kEpi>;
                if (chunks_per_lane <= 2) return (const void*)&gemv_kernel<WT, 2, 4, kOut, kEpi>;
                return (const void*)&gemv_kernel<WT, 4, 4, kOut, kEpi>;
            }
        } else if (rows == 2) {
            if (chunks_per_lane <= 1) return (const void*)&gemv_kernel<WT, 1, 2, kOut, kEpi>;
            if (chunks_per_lane <= 2) return (const void*)&gemv_kernel<WT, 2, 2, kOut, kEpi>;
            if (chunks_per_lane <= 4) return (const void*)&gemv_kernel<WT, 4, 2, kOut, kEpi>;
            return (const void*)&gemv_kernel<WT, 8, 2, kOut, kEpi>;
        }
    }
    if (chunks_per_lane <= 1) return (const void*)&gemv_kernel<WT, 1, 1, kOut, kEpi>;
    if (chunks_per_lane <= 2) return (const void*)&gemv_kernel<WT, 2, 1, kOut, kEpi>;
    if (chunks_per_lane <= 4) return (const void*)&gemv_kernel<WT, 4, 1, kOut, kEpi>;
    if (chunks_per_lane <= 8) return (const void*)&gemv_kernel<WT, 8, 1, kOut, kEpi>;
    return (const void*)&gemv_kernel<WT, kGemvMaxChunks, 1, kOut, kEpi>;
}

// The QKV epilogue writes qkv in the activation type, so only the plain GEMV takes another
// output type.
template <int WT>
const void* gemv_ptr_out(int chunks_per_lane, int rows, bool out_f32, int epi) {
    constexpr bool kAct = WFmt<WT>::kActF32;
    if (epi == kEpiAppend) return gemv_ptr<WT, kAct, kEpiAppend>(chunks_per_lane, 1);
    if (epi == kEpiAppend8) {
        if constexpr (kAct) return nullptr;   // 8-bit caches sit behind bf16 activations
        else return gemv_ptr<WT, false, kEpiAppend8>(chunks_per_lane, 1);
    }
    return out_f32 ? gemv_ptr<WT, true, kEpiNone>(chunks_per_lane, rows)
                   : gemv_ptr<WT, false, kEpiNone>(chunks_per_lane, rows);
}

}  // namespace

namespace kvattn_internal {
void set_last_hip_error(int e);   // kvattn.hip: read back by kvattn_last_hip_error
int merge_poll_limit();           // kvattn.hip: kvattn_set_merge_poll_limit's bound
}

namespace {

// Checks shared by the entry points, then the launch.  out_f32: out and pre_gelu as float,
// else bf16.
int launch_gemv(GemvArgs a, int w_dtype, bool out_f32, void* stream) {
    if (w_dtype < KVATTN_KV_F32 || w_dtype > KVATTN_KV_FP8_E4M3) return KVATTN_ERR_DTYPE;
    const bool w8 = w_dtype == KVATTN_KV_INT8 || w_dtype == KVATTN_KV_FP8_E4M3;
    const int wbytes = w_dtype == KVATTN_KV_F32 ? 4 : (w_dtype == KVATTN_KV_BF16 ? 2 : 1);
    const size_t act = w_dtype == KVATTN_KV_F32 ? 4 : 2;
    const size_t osz = out_f32 ? 4 : 2;
    const int B = a.B, M = a.M, K = a.K;
    if (B < 1 || M < 1 || M > kRowMask || K < 16 || K % 16 != 0) return KVATTN_ERR_SHAPE;
    if ((long long)B * M >= (1ll << 31) || (long long)M * K * wbytes >= (1ll << 40) || (long long)B * K >= (1ll << 31))
        return KVATTN_ERR_SHAPE;
    if (!a.out || !a.W || !a.x) return KVATTN_ERR_NULL_POINTER;
    if (w8 && !a.w_scale) return KVATTN_ERR_DTYPE;
    if (((uintptr_t)a.W & 15u) || ((uintptr_t)a.x & 15u)) return KVATTN_ERR_MISALIGNED;
    if (((uintptr_t)a.out % osz) || ((uintptr_t)a.pre_gelu % osz) || ((uintptr_t)a.bias % act) ||
        ((uintptr_t)a.w_scale & 3u) ||
        (a.kv && a.kv_dtype != KVATTN_KV_INT8 && a.kv_dtype != KVATTN_KV_FP8_E4M3 && ((uintptr_t)a.kv % act)))
        return KVATTN_ERR_MISALIGNED;
    const int nch = K * wbytes / 16;
    const int per_lane = (nch + kWave - 1) / kWave;
    // Measured at 50304 x 768 (per call, graph of calls over weights beyond the Infinity
    // Cache), INT8 / BF16 / FP32: 2 rows per wave 9.0-9.1 / 13.1-13.3 / 23.9-24.2 us; 4 rows
    // with the wave-uniform row index 8.6 / 14.0-14.2 / 25.0, without it 9.3 / 13.8 / 24.9;
    // 8 rows 9.8 / 15.5 / 24.9; one row 16.8 / 19.0 / 26.6.  Workgroups of 8 or 16 waves
    // instead of 4: +0.5 to +2.6 us.  The QKV epilogue takes one row per wave.
    const int rows = a.kv || M < kGemvTallRows ? 1 : (w8 ? 4 : 2);
    const bool kv8 = a.kv && (a.kv_dtype == KVATTN_KV_INT8 || a.kv_dtype == KVATTN_KV_FP8_E4M3);
    const int epi = !a.kv ? kEpiNone : (kv8 ? kEpiAppend8 : kEpiAppend);
    const void* fn = nullptr;
    switch (w_dtype) {
        case KVATTN_KV_F32: fn = gemv_ptr_out<KVATTN_KV_F32>(per_lane, rows, out_f32, epi); break;
        case KVATTN_KV_BF16: fn = gemv_ptr_out<KVATTN_KV_BF16>(per_lane, rows, out_f32, epi); break;
        case KVATTN_KV_INT8: fn = gemv_ptr_out<KVATTN_KV_INT8>(per_lane, rows, out_f32, epi); break;
        default: fn = gemv_ptr_out<KVATTN_KV_FP8_E4M3>(per_lane, rows, out_f32, epi); break;
    }
    if (!fn) return KVATTN_ERR_DTYPE;
    long long groups = ((M + rows - 1) / rows + kGemvWaves - 1) / kGemvWaves;
    int pk_m = a.M | (a.gelu ? kGeluFlag : 0);
    // 8-bit epilogue: the 16 workgroups of each of the 3*NH head rows on one XCD, once there are
    // enough head rows to give every XCD one (the grid is padded to whole rounds of 8).
    if (epi == kEpiAppend8 && 3 * a.NH >= 8) {
        groups = 8ll * ((3 * a.NH + 7) / 8) * kHeadRowGroups;
        pk_m |= kXcdLocalFlag;
    }
    void* params[] = {&a.W, &a.x, &a.w_scale, &a.bias, &pk_m, &a.K, &a.B, &a.out, &a};
    const hipError_t e = hipLaunchKernel(fn, dim3((unsigned)groups), dim3(kGemvWaves * kWave), params, 0,
                                         (hipStream_t)stream);
    if (e != hipSuccess) {
        kvattn_internal::set_last_hip_error((int)e);
        return KVATTN_ERR_HIP;
    }
    return KVATTN_OK;
}

}  // namespace

extern "C" int kvattn_gemv(void* out, void* pre_gelu, const void* W, const float* w_scale, const void* x,
                           const void* bias, int B, int M, int K, int w_dtype, int gelu, void* stream) {
    GemvArgs a{out, pre_gelu, (const uint8_t*)W, w_scale, (const uint8_t*)x, bias, B, M, K, gelu ? 1 : 0,
               nullptr, nullptr, 0, 0, 0, 0, nullptr, nullptr, 0};
    return launch_gemv(a, w_dtype, w_dtype == KVATTN_KV_F32, stream);
}

extern "C" int kvattn_gemv_ex(void* out, void* pre_gelu, const void* W, const float* w_scale, const void* x,
                              const void* bias, int B, int M, int K, int w_dtype, int out_dtype, int gelu,
                              void* stream) {
    if (out_dtype != KVATTN_KV_F32 && out_dtype != KVATTN_KV_BF16) return KVATTN_ERR_DTYPE;
    GemvArgs a{out, pre_gelu, (const uint8_t*)W, w_scale, (const uint8_t*)x, bias, B, M, K, gelu ? 1 : 0,
               nullptr, nullptr, 0, 0, 0, 0, nullptr, nullptr, 0};
    return launch_gemv(a, w_dtype, out_dtype == KVATTN_KV_F32, stream);
}

extern "C" size_t kvattn_gemv_qkv_append_workspace_bytes(int B, int NH) {
    if (B < 1 || NH < 1 || (long long)B * NH > (1ll << 24)) return 0;
    const size_t rows = (size_t)B * 2 * NH;   // one tagged word per channel of every appended K and V row
    return rows * kHd * sizeof(unsigned long long);
}

extern "C" int kvattn_gemv_qkv_append(void* qkv, const void* W, const float* w_scale, const void* x,
                                      const void* bias, int B, int NH, int hs, int K, void* kv_cache,
                                      float* kv_scale, int maxT, const int* d_cur_len, int lens_per_seq,
                                      int w_dtype, int kv_dtype, void* workspace, size_t workspace_bytes,
                                      void* stream) {
    if (hs != kHd) return KVATTN_ERR_HEAD_DIM;
    if (B < 1 || NH < 1 || maxT < 1 || (long long)B * NH > (1ll << 24) || maxT > (1 << 23)) return KVATTN_ERR_SHAPE;
    if (!kv_cache) return KVATTN_ERR_NULL_POINTER;
    const bool kv8 = kv_dtype == KVATTN_KV_INT8 || kv_dtype == KVATTN_KV_FP8_E4M3;
    const int act = w_dtype == KVATTN_KV_F32 ? KVATTN_KV_F32 : KVATTN_KV_BF16;
    if (!kv8 && kv_dtype != act) return KVATTN_ERR_DTYPE;          // the cache holds the activation type
    if (kv8 && (w_dtype == KVATTN_KV_F32 || !kv_scale)) return KVATTN_ERR_DTYPE;
    unsigned long long* words = nullptr;
    if (kv8) {
        const size_t need = kvattn_gemv_qkv_append_workspace_bytes(B, NH);
        if (!workspace || workspace_bytes < need) return KVATTN_ERR_WORKSPACE;
        if (((uintptr_t)workspace & 255u) || ((uintptr_t)kv_scale & 3u)) return KVATTN_ERR_MISALIGNED;
        words = (unsigned long long*)workspace;
    }
    if (!d_cur_len) {
        int* sym = nullptr;
        const int st = kvattn_cur_len_symbol(&sym);
        if (st != KVATTN_OK) return st;
        d_cur_len = sym;
    }
    GemvArgs a{qkv, nullptr, (const uint8_t*)W, w_scale, (const uint8_t*)x, bias, B, 3 * NH * hs, K, 0,
               (uint8_t*)kv_cache, d_cur_len, lens_per_seq ? 1 : 0, NH, maxT, kv_dtype, kv_scale, words,
               kvattn_internal::merge_poll_limit()};
    return launch_gemv(a, w_dtype, w_dtype == KVATTN_KV_F32, stream);
}
