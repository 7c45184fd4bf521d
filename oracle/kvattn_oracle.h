/* kvattn_oracle.h -- CPU oracle for the decode-phase KV-cache attention.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: the parity tests,
 * the smoke check and the CPU-baseline leg of the benchmark call it to produce
 * expected values.  Nothing in the product path (libkvattn.so and its C++ /
 * Python hosts) links, loads or calls it.
 *
 * Every function restates a piece of the reference's algorithm and cites the
 * reference file:line it follows.  Layouts are the reference's:
 *   qkv       [B][3][NH][hs]                 (Q, K, V of the current token)
 *   kv_cache  [2][B][NH][maxT][hs]           (K block, then V block)
 *   kv_scale  [2][B][NH][maxT]  float        (8-bit caches only)
 *   out       [B][NH][hs]
 *   part_out  [B][NH][S][hs], part_max / part_lse [B][NH][S]
 * A "total" is the number of attended positions, cur_len + 1.
 */
#ifndef KVATTN_ORACLE_H
#define KVATTN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Formats of an 8-bit row code (the reference's USE_INT8 / USE_FP8 switch). */
enum { ORACLE_W8_INT8 = 0, ORACLE_W8_FP8_E4M3 = 1 };

/* ---- attention ---------------------------------------------------------- */

/* attention_kv_cpu, attention_kvcache/attention_kvcache.cu:74-102, FP32, the same
 * loop order.  All B sequences attend `total` positions.  The reference's
 * scores[1024] stack array is replaced by a heap buffer so total may exceed 1024. */
void oracle_attention_f32(float* out, const float* qkv, const float* kv_cache,
                          int B, int total, int NH, int hs, int maxT, float scale);

/* Same routine with one total per sequence (totals[b]); the ragged extension. */
void oracle_attention_f32_ragged(float* out, const float* qkv, const float* kv_cache,
                                 const int* totals, int B, int NH, int hs, int maxT,
                                 float scale);

/* Float64 twin of the ragged routine (inputs are float, every operation in double). */
void oracle_attention_f64_ragged(double* out, const float* qkv, const float* kv_cache,
                                 const int* totals, int B, int NH, int hs, int maxT,
                                 double scale);

/* ---- flash-decoding split + merge -------------------------------------- */

/* attention_kv_split_kernel, Inference_gpt2/attention_kvcache.cuh:185-288, computed
 * sequentially: partition chunk = ceil(total/S), j_start = s*chunk (:195-200), empty
 * segment -> (max=-FLT_MAX, lse=0, out=0) (:202-207), otherwise the segment max, the
 * sum of exp(score-max) and the unnormalised exp-weighted V sum. */
void oracle_split_partials(float* part_out, float* part_lse, float* part_max,
                           const float* qkv, const float* kv_cache, const int* totals,
                           int B, int NH, int hs, int maxT, int S, float scale);

/* attention_kv_merge_kernel, Inference_gpt2/attention_kvcache.cuh:298-318. */
void oracle_merge(float* out, const float* part_out, const float* part_lse,
                  const float* part_max, int B, int NH, int hs, int S);

/* ---- element codecs ----------------------------------------------------- */

/* float -> bfloat16 bits, round to nearest even (the (floatX) cast of a BF16 build). */
uint16_t oracle_bf16_from_f32(float x);
float oracle_bf16_to_f32(uint16_t b);
void oracle_bf16_round_array(const float* in, uint16_t* out, size_t n);
void oracle_bf16_decode_array(const uint16_t* in, float* out, size_t n);

/* kv_w8_encode / kv_w8_decode, Inference_gpt2/attention_kvcache_w8.cuh:55-82.
 * INT8: clamp(rint_half_even(x/scale), -127, 127).  FP8: E4M3 (OCP "FN" variant,
 * max 448, NaN 0x7F/0xFF) of x/scale, round to nearest even, saturating to +-448. */
uint8_t oracle_w8_encode(float x, float scale, int fmt);
float oracle_w8_decode(uint8_t code, int fmt);
uint8_t oracle_fp8_e4m3_from_f32(float y);   /* saturating RNE encode of y itself */
float oracle_fp8_e4m3_to_f32(uint8_t code);  /* exact decode, NaN for 0x7F/0xFF */

/* ---- KV append ---------------------------------------------------------- */

/* kv_cache_write_kernel, Inference_gpt2/attention_kvcache.cuh:46-64: copies the current
 * token's K and V (elem_size bytes each element, any type) from qkv into column
 * cur_lens[b] of each (b,h) slot.  The reference has one cur_len for all rows; here
 * cur_lens holds one entry per sequence. */
void oracle_cache_write(void* kv_cache, const void* qkv, size_t elem_size,
                        const int* cur_lens, int B, int NH, int hs, int maxT);

/* kv_cache_write_kernel_w8, Inference_gpt2/attention_kvcache_w8.cuh:115-155: per row,
 * amax = max|x| over hs channels (x = the bf16 source values, given here as floats),
 * scale = amax / LIMIT (127 or 448), codes = encode(x, scale), or all-zero codes when
 * scale == 0; writes codes and scale into column cur_lens[b]. */
void oracle_cache_write_w8(uint8_t* kv_cache, float* kv_scale, const float* qkv,
                           const int* cur_lens, int B, int NH, int hs, int maxT, int fmt);

/* Dequantise an 8-bit cache to FP32: value = decode(code) * row_scale, the per-element
 * product the reference's V path forms (attention_kvcache_w8.cuh:235). */
void oracle_dequant_w8(float* kv_out, const uint8_t* kv_cache, const float* kv_scale,
                       int B, int NH, int hs, int maxT, int fmt);

/* ---- seeded inputs ------------------------------------------------------ */

/* SplitMix64 stream -> Box-Muller in double -> float: n standard-normal samples. */
void oracle_gen_normal(uint64_t seed, float* out, size_t n);

/* make_random_float after srand(seed), attention_kvcache/attention_kvcache.cu:911-917:
 * (float)(rand() % 10000) / 5000.0f - 1.0f.  The lab calls srand(0) once and then draws
 * the qkv buffer followed by the cache buffer from the same stream (:952,979-980); pass
 * n = n_qkv + n_cache to reproduce both. */
void oracle_lab_rand(unsigned seed, float* out, size_t n);

/* Single-threaded timing helper for the CPU baseline: runs oracle_attention_f32 `reps`
 * times and returns the median wall time of one call in microseconds. */
double oracle_time_attention_f32(float* out, const float* qkv, const float* kv_cache,
                                 int B, int total, int NH, int hs, int maxT, float scale,
                                 int reps);

/* The decode step's fully connected layer (the GEMV after the attention):
 * for b < B, m < M: pre = (sum_{k ascending} W[m*K+k] * x[b*K+k]) * s_m + bias[m] in
 * FP32, s_m = w_scale[m] (8-bit weights, W holding the decoded codes) or 1 (w_scale NULL);
 * pre_gelu[b*M+m] = pre (if non-NULL); out[b*M+m] = gelu ? GELU_tanh(pre) : pre.
 * Follows GEMV6_fused (Inference_gpt2/GEMV.cuh:132-197) and GEMV6_w8x2
 * (Inference_gpt2/GEMV_w8.cuh:64-157).  Outputs are not rounded to the activation type. */
void oracle_gemv(float* out, float* pre_gelu, const float* W, const float* w_scale, const float* x,
                 const float* bias, int B, int M, int K, int gelu);
float oracle_gelu_tanh(float v);

/* Median microseconds of `reps` single-threaded oracle_gemv calls (CPU baseline). */
double oracle_time_gemv(float* out, const float* W, const float* w_scale, const float* x, const float* bias,
                        int B, int M, int K, int reps);

#ifdef __cplusplus
}
#endif
#endif
