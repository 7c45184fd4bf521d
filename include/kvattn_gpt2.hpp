// kvattn_gpt2.hpp -- C++ host-side mirror of the reference engine's decode-attention entry
// points, implemented over the C ABI of kvattn.h (libkvattn.so).
//
// Same names, argument order and meaning as the reference's inline host functions and
// kernel launches, so the per-layer attention block of a GPT-2 decode step ports line for
// line.  Two differences, both forced by the boundary:
//   * the KV precision is a run-time argument (the reference selects it at compile time
//     with ENABLE_FP32 / USE_KV_W8 + USE_INT8 / USE_FP8, Makefile:78-106), so pointers are
//     void* instead of floatX* / uint8_t*;
//   * the device-resident length is the library's own (kvattn_cur_len_symbol), or any
//     device int the caller passes.
// Errors behave like the reference's cudaCheck (Inference_gpt2/common.h:123-130): the
// failing call's file and line and the status text are printed and the process exits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "kvattn.h"

inline void kvattnCheck_(int status, const char* file, int line) {
    if (status != KVATTN_OK) {
        printf("[kvattn error] %s:%d: %s", file, line, kvattn_strerror(status));
        if (status == KVATTN_ERR_HIP) printf(" (hipError %d)", kvattn_last_hip_error());
        printf("\n");
        exit(EXIT_FAILURE);
    }
}
#define kvattnCheck(st) (kvattnCheck_((st), __FILE__, __LINE__))

namespace kvattn_gpt2 {

// cudaGetSymbolAddress(&d_cur_len_ptr, g_cur_len) (inference_gpt2_opt.cu:252-254).
inline int* cur_len_symbol() {
    int* p = nullptr;
    kvattnCheck(kvattn_cur_len_symbol(&p));
    return p;
}

// cudaMemcpyToSymbol(g_cur_len, &cur_len, sizeof(int)) (inference_gpt2_opt.cu:409,548).
inline void set_cur_len(int cur_len) { kvattnCheck(kvattn_set_cur_len(cur_len)); }

// The same write, enqueued on a stream (no host synchronisation; capturable).
inline void set_cur_len_async(int cur_len, hipStream_t stream, int* d_cur_len = nullptr) {
    kvattnCheck(kvattn_set_cur_len_async(d_cur_len, cur_len, stream));
}

// kv_cache_write_kernel<<<CEIL_DIV(B*NH*hs,256), 256, 0, stream>>>(kv_cache, qkv, B, NH, hs, maxT)
// (Inference_gpt2/attention_kvcache.cuh:46-64, launched at inference_gpt2_opt.cu:329).
inline void kv_cache_write(void* kv_cache, const void* qkv, int B, int NH, int hs, int maxT,
                           hipStream_t stream, int kv_dtype = KVATTN_KV_BF16, const int* d_cur_len = nullptr) {
    kvattnCheck(kvattn_cache_write(kv_cache, nullptr, qkv, B, NH, hs, maxT, d_cur_len, 0, kv_dtype, stream));
}

// kv_cache_write_kernel_w8<<<B*NH*2, 256, 0, stream>>>(kv_cache, kv_scale, qkv, B, NH, hs, maxT)
// (Inference_gpt2/attention_kvcache_w8.cuh:115-155, launched at inference_gpt2_opt.cu:302-303).
inline void kv_cache_write_w8(uint8_t* kv_cache, float* kv_scale, const void* qkv, int B, int NH, int hs,
                              int maxT, hipStream_t stream, int kv_dtype = KVATTN_KV_INT8,
                              const int* d_cur_len = nullptr) {
    kvattnCheck(kvattn_cache_write(kv_cache, kv_scale, qkv, B, NH, hs, maxT, d_cur_len, 0, kv_dtype, stream));
}

// attention_forward_kv_small (Inference_gpt2/attention_kvcache.cuh:453-459).
inline void attention_forward_kv_small(void* out, const void* qkv, void* kv_cache, int B, int NH, int hs,
                                       int maxT, hipStream_t stream, int kv_dtype = KVATTN_KV_BF16,
                                       const int* d_cur_len = nullptr) {
    kvattnCheck(kvattn_forward_small(out, qkv, kv_cache, nullptr, B, NH, hs, maxT, d_cur_len, 0, kv_dtype, stream));
}

// attention_forward_kv_small_w8 (Inference_gpt2/attention_kvcache_w8.cuh:529-536).
inline void attention_forward_kv_small_w8(void* out, const void* qkv, uint8_t* kv_cache, const float* kv_scale,
                                          int B, int NH, int hs, int maxT, hipStream_t stream,
                                          int kv_dtype = KVATTN_KV_INT8, const int* d_cur_len = nullptr) {
    kvattnCheck(kvattn_forward_small(out, qkv, kv_cache, kv_scale, B, NH, hs, maxT, d_cur_len, 0, kv_dtype, stream));
}

// attention_forward_kv_large (Inference_gpt2/attention_kvcache.cuh:464-487): B == 1 ->
// single launch (the designated merger; the reference launches cooperatively), B > 1 ->
// split + merge, caller-owned partials of S segments.
inline void attention_forward_kv_large(void* out, const void* qkv, void* kv_cache, int B, int NH, int hs,
                                       int maxT, hipStream_t stream, float* part_out, float* part_lse,
                                       float* part_max, int S, int kv_dtype = KVATTN_KV_BF16,
                                       const int* d_cur_len = nullptr) {
    kvattnCheck(kvattn_forward_large(out, qkv, kv_cache, nullptr, B, NH, hs, maxT, d_cur_len, 0, part_out,
                                     part_lse, part_max, S, kv_dtype, stream));
}

// attention_forward_kv_large_w8 (Inference_gpt2/attention_kvcache_w8.cuh:541-566).
inline void attention_forward_kv_large_w8(void* out, const void* qkv, uint8_t* kv_cache, const float* kv_scale,
                                          int B, int NH, int hs, int maxT, hipStream_t stream, float* part_out,
                                          float* part_lse, float* part_max, int S, int kv_dtype = KVATTN_KV_INT8,
                                          const int* d_cur_len = nullptr) {
    kvattnCheck(kvattn_forward_large(out, qkv, kv_cache, kv_scale, B, NH, hs, maxT, d_cur_len, 0, part_out,
                                     part_lse, part_max, S, kv_dtype, stream));
}

// attention_kv_split_kernel[_w8]<<<B*NH*S, 256, 0, stream>>>(part_out, part_lse, part_max, qkv,
// kv_cache, [kv_scale,] B, NH, hs, maxT, S, 1/sqrt(hs)) -- the capturable launch used by the
// reference's graph path (inference_gpt2_opt.cu:310-312,338-339).
inline void attention_kv_split(float* part_out, float* part_lse, float* part_max, const void* qkv,
                               const void* kv_cache, const float* kv_scale, int B, int NH, int hs, int maxT,
                               int S, hipStream_t stream, int kv_dtype = KVATTN_KV_BF16,
                               const int* d_cur_len = nullptr) {
    kvattnCheck(kvattn_split(part_out, part_lse, part_max, qkv, kv_cache, kv_scale, B, NH, hs, maxT, d_cur_len,
                             0, S, kv_dtype, stream));
}

// attention_kv_merge_kernel[_w8]<<<B*NH, 64, 0, stream>>>(out, part_out, part_lse, part_max, NH, hs, S)
// (inference_gpt2_opt.cu:313-314,340-341).  B is explicit here: the reference derives the
// grid from it at the launch site.
inline void attention_kv_merge(void* out, const float* part_out, const float* part_lse, const float* part_max,
                               int B, int NH, int hs, int S, hipStream_t stream, int kv_dtype = KVATTN_KV_BF16) {
    kvattnCheck(kvattn_merge(out, part_out, part_lse, part_max, B, NH, hs, S, kv_dtype, stream));
}

// The append launch and the attention call of one layer (inference_gpt2_opt.cu:302-316,
// 329-345) as one launch: AUTO strategy with no length hint, so the kernels plan the
// segmentation from the device length and one captured step graph serves every length.
// workspace: kvattn_workspace_bytes(B, NH, hs, maxT, 0) bytes, initialised once.
inline void kv_append_attention(void* out, const void* qkv, void* kv_cache, float* kv_scale, int B, int NH,
                                int hs, int maxT, void* workspace, size_t workspace_bytes, hipStream_t stream,
                                int kv_dtype = KVATTN_KV_BF16, const int* d_cur_len = nullptr) {
    kvattnCheck(kvattn_append_decode(out, qkv, kv_cache, kv_scale, B, NH, hs, maxT, d_cur_len, 0, -1, workspace,
                                     workspace_bytes, 0, KVATTN_AUTO, kv_dtype, stream));
}

// launch_GEMV6_fused<floatX>(out, pre_gelu, W, x, bias, M, K, do_gelu, stream)
// (Inference_gpt2/GEMV.cuh:204-208), as matmul_forward calls it for one decode token
// (inference_gpt2_opt.cu:106-116).  w_dtype: KVATTN_KV_BF16 (floatX = bf16) or KVATTN_KV_F32.
// out_dtype: the reference's OT when it differs from the activations (KVATTN_KV_F32 or
// KVATTN_KV_BF16); -1 keeps the activation type.
inline void launch_GEMV6_fused(void* out, void* pre_gelu, const void* W, const void* x, const void* bias, int M,
                               int K, bool do_gelu, hipStream_t stream, int w_dtype = KVATTN_KV_BF16,
                               int out_dtype = -1) {
    if (out_dtype < 0)
        kvattnCheck(kvattn_gemv(out, pre_gelu, W, nullptr, x, bias, 1, M, K, w_dtype, do_gelu ? 1 : 0, stream));
    else
        kvattnCheck(kvattn_gemv_ex(out, pre_gelu, W, nullptr, x, bias, 1, M, K, w_dtype, out_dtype,
                                   do_gelu ? 1 : 0, stream));
}

// launch_GEMV6_w8x2(out, pre_gelu, W, x, scale, bias, M, K, do_gelu, stream)
// (Inference_gpt2/GEMV_w8.cuh:162-184), as matmul_forward_w8 calls it (inference_gpt2_opt.cu:
// 121-132).  w_dtype: KVATTN_KV_INT8 or KVATTN_KV_FP8_E4M3 (the reference's USE_INT8 / USE_FP8).
// out_dtype KVATTN_KV_F32 is the reference's launch_GEMV6_w8x2<float, floatX>, the vocabulary
// projection into float logits (inference_gpt2_opt.cu:389-394); -1 keeps bf16.
inline void launch_GEMV6_w8x2(void* out, void* pre_gelu, const uint8_t* W, const void* x, const float* scale,
                              const void* bias, int M, int K, bool do_gelu, hipStream_t stream,
                              int w_dtype = KVATTN_KV_INT8, int out_dtype = -1) {
    if (out_dtype < 0)
        kvattnCheck(kvattn_gemv(out, pre_gelu, W, scale, x, bias, 1, M, K, w_dtype, do_gelu ? 1 : 0, stream));
    else
        kvattnCheck(kvattn_gemv_ex(out, pre_gelu, W, scale, x, bias, 1, M, K, w_dtype, out_dtype,
                                   do_gelu ? 1 : 0, stream));
}

}  // namespace kvattn_gpt2
