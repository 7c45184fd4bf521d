/* kvattn_oracle.c -- CPU oracle for the decode-phase KV-cache attention.
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  See kvattn_oracle.h for the contract and
 * the layouts.  Built with -ffp-contract=off and without fast-math so that every FP32
 * operation is an individually rounded IEEE operation in the loop order written here.
 */
#include "kvattn_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static inline size_t k_index(int b, int h, int j, int NH, int hs, int maxT) {
    return ((size_t)(b * NH + h) * (size_t)maxT + (size_t)j) * (size_t)hs;
}

/* ---------------------------------------------------------------------------------
 * attention_kv_cpu (attention_kvcache/attention_kvcache.cu:74-102).
 * Per (b,h): scores[j] = (sum_d q[d]*K[j][d]) * scale with a running max (:80-89);
 * then for every channel d, acc = sum_j exp(scores[j]-max)*V[j][d] and
 * expsum = sum_j exp(scores[j]-max), out = acc/expsum (:91-99).  The exp is recomputed
 * per channel exactly as the reference does.
 * ------------------------------------------------------------------------------- */
static void attention_one_head_f32(float* out_bh, const float* q, const float* kslot,
                                   const float* vslot, int total, int hs, float scale,
                                   float* scores) {
    float maxval = -FLT_MAX;
    for (int j = 0; j < total; j++) {
        float sum = 0.0f;
        for (int d = 0; d < hs; d++) { sum += q[d] * kslot[(size_t)j * hs + d]; }
        scores[j] = sum * scale;
        maxval = fmaxf(maxval, scores[j]);
    }
    for (int d = 0; d < hs; d++) {
        float acc = 0.0f;
        float expsum = 0.0f;
        for (int j = 0; j < total; j++) {
            float expv = expf(scores[j] - maxval);
            acc += expv * vslot[(size_t)j * hs + d];
            expsum += expv;
        }
        out_bh[d] = acc / expsum;
    }
}

void oracle_attention_f32_ragged(float* out, const float* qkv, const float* kv_cache,
                                 const int* totals, int B, int NH, int hs, int maxT,
                                 float scale) {
    float* scores = (float*)malloc(sizeof(float) * (size_t)(maxT > 0 ? maxT : 1));
    const size_t vblock = (size_t)B * NH * maxT * hs;
    for (int b = 0; b < B; b++) {
        for (int h = 0; h < NH; h++) {
            const float* q = qkv + (size_t)b * 3 * NH * hs + (size_t)h * hs;
            const float* kslot = kv_cache + k_index(b, h, 0, NH, hs, maxT);
            const float* vslot = kv_cache + vblock + k_index(b, h, 0, NH, hs, maxT);
            attention_one_head_f32(out + (size_t)(b * NH + h) * hs, q, kslot, vslot,
                                   totals[b], hs, scale, scores);
        }
    }
    free(scores);
}

void oracle_attention_f32(float* out, const float* qkv, const float* kv_cache,
                          int B, int total, int NH, int hs, int maxT, float scale) {
    int* totals = (int*)malloc(sizeof(int) * (size_t)B);
    for (int b = 0; b < B; b++) totals[b] = total;
    oracle_attention_f32_ragged(out, qkv, kv_cache, totals, B, NH, hs, maxT, scale);
    free(totals);
}

void oracle_attention_f64_ragged(double* out, const float* qkv, const float* kv_cache,
                                 const int* totals, int B, int NH, int hs, int maxT,
                                 double scale) {
    double* scores = (double*)malloc(sizeof(double) * (size_t)(maxT > 0 ? maxT : 1));
    const size_t vblock = (size_t)B * NH * maxT * hs;
    for (int b = 0; b < B; b++) {
        for (int h = 0; h < NH; h++) {
            const float* q = qkv + (size_t)b * 3 * NH * hs + (size_t)h * hs;
            const float* kslot = kv_cache + k_index(b, h, 0, NH, hs, maxT);
            const float* vslot = kv_cache + vblock + k_index(b, h, 0, NH, hs, maxT);
            const int total = totals[b];
            double maxval = -DBL_MAX;
            for (int j = 0; j < total; j++) {
                double sum = 0.0;
                for (int d = 0; d < hs; d++) sum += (double)q[d] * (double)kslot[(size_t)j * hs + d];
                scores[j] = sum * scale;
                if (scores[j] > maxval) maxval = scores[j];
            }
            double expsum = 0.0;
            for (int j = 0; j < total; j++) {
                scores[j] = exp(scores[j] - maxval);
                expsum += scores[j];
            }
            for (int d = 0; d < hs; d++) {
                double acc = 0.0;
                for (int j = 0; j < total; j++) acc += scores[j] * (double)vslot[(size_t)j * hs + d];
                out[(size_t)(b * NH + h) * hs + d] = acc / expsum;
            }
        }
    }
    free(scores);
}

/* ---------------------------------------------------------------------------------
 * Split + merge.
 * Partition (attention_kvcache.cuh:195-200): chunk = ceil(total/S), j_start = s*chunk,
 * j_end = min(j_start+chunk, total).  Empty segment sentinel (:202-207).  Segment max
 * (:235-244), exp-sum and exp numerators (:247-260), exp-weighted V sum (:262-282).
 * ------------------------------------------------------------------------------- */
void oracle_split_partials(float* part_out, float* part_lse, float* part_max,
                           const float* qkv, const float* kv_cache, const int* totals,
                           int B, int NH, int hs, int maxT, int S, float scale) {
    const size_t vblock = (size_t)B * NH * maxT * hs;
    float* scores = (float*)malloc(sizeof(float) * (size_t)(maxT > 0 ? maxT : 1));
    for (int b = 0; b < B; b++) {
        const int total = totals[b];
        const int chunk = (total + S - 1) / S;
        for (int h = 0; h < NH; h++) {
            const float* q = qkv + (size_t)b * 3 * NH * hs + (size_t)h * hs;
            const float* kslot = kv_cache + k_index(b, h, 0, NH, hs, maxT);
            const float* vslot = kv_cache + vblock + k_index(b, h, 0, NH, hs, maxT);
            for (int s = 0; s < S; s++) {
                const size_t pi = (size_t)(b * NH + h) * S + s;
                const int j_start = s * chunk;
                const int j_end = (j_start + chunk < total) ? j_start + chunk : total;
                const int n_local = j_end - j_start;
                if (n_local <= 0) {
                    part_max[pi] = -FLT_MAX;
                    part_lse[pi] = 0.0f;
                    for (int d = 0; d < hs; d++) part_out[pi * hs + d] = 0.0f;
                    continue;
                }
                float mv = -FLT_MAX;
                for (int jj = 0; jj < n_local; jj++) {
                    float sum = 0.0f;
                    const float* k_row = kslot + (size_t)(j_start + jj) * hs;
                    for (int d = 0; d < hs; d++) sum += q[d] * k_row[d];
                    scores[jj] = sum * scale;
                    mv = fmaxf(mv, scores[jj]);
                }
                float ls = 0.0f;
                for (int jj = 0; jj < n_local; jj++) {
                    scores[jj] = expf(scores[jj] - mv);
                    ls += scores[jj];
                }
                for (int d = 0; d < hs; d++) {
                    float acc = 0.0f;
                    for (int jj = 0; jj < n_local; jj++)
                        acc += scores[jj] * vslot[(size_t)(j_start + jj) * hs + d];
                    part_out[pi * hs + d] = acc;
                }
                part_max[pi] = mv;
                part_lse[pi] = ls;
            }
        }
    }
    free(scores);
}

/* attention_kv_merge_kernel (attention_kvcache.cuh:298-318): m = max_s part_max;
 * O = sum_s exp(part_max_s - m) * part_out_s; l = sum_s exp(part_max_s - m) * part_lse_s;
 * out = O / l. */
void oracle_merge(float* out, const float* part_out, const float* part_lse,
                  const float* part_max, int B, int NH, int hs, int S) {
    for (int bh = 0; bh < B * NH; bh++) {
        for (int d = 0; d < hs; d++) {
            float m_global = -FLT_MAX;
            for (int s = 0; s < S; s++) m_global = fmaxf(m_global, part_max[(size_t)bh * S + s]);
            float O = 0.0f, l = 0.0f;
            for (int s = 0; s < S; s++) {
                float rescale = expf(part_max[(size_t)bh * S + s] - m_global);
                O += rescale * part_out[((size_t)bh * S + s) * hs + d];
                l += rescale * part_lse[(size_t)bh * S + s];
            }
            out[(size_t)bh * hs + d] = O / l;
        }
    }
}

/* ---------------------------------------------------------------------------------
 * bfloat16: the upper 16 bits of an IEEE float; the cast rounds to nearest even and
 * keeps NaN a (quiet) NaN.
 * ------------------------------------------------------------------------------- */
static inline uint32_t f32_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float bits_f32(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

uint16_t oracle_bf16_from_f32(float x) {
    uint32_t u = f32_bits(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

void oracle_bf16_round_array(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = oracle_bf16_from_f32(in[i]);
}

void oracle_bf16_decode_array(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = oracle_bf16_to_f32(in[i]);
}

/* ---------------------------------------------------------------------------------
 * FP8 E4M3, OCP 8-bit floating point spec v1.0 (2023), the "FN" variant:
 *   1 sign bit, 4 exponent bits (bias 7), 3 mantissa bits; no infinities;
 *   S.1111.111 is NaN; largest finite 0x7E = 448; subnormals m * 2^-9.
 * Encode rounds to nearest, ties to even, and saturates finite overflow to +-448
 * (the reference requests __NV_SATFINITE, attention_kvcache_w8.cuh:58).
 * ------------------------------------------------------------------------------- */
float oracle_fp8_e4m3_to_f32(uint8_t code) {
    const int sign = code >> 7;
    const int e = (code >> 3) & 0xF;
    const int m = code & 0x7;
    float v;
    if (e == 0xF && m == 0x7) return NAN;
    if (e == 0) v = ldexpf((float)m, -9);
    else v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return sign ? -v : v;
}

uint8_t oracle_fp8_e4m3_from_f32(float y) {
    if (isnan(y)) return 0x7F;
    const uint8_t sign = signbit(y) ? 0x80 : 0x00;
    const float a = fabsf(y);
    if (a >= 448.0f) return sign | 0x7E;                 /* saturate (incl. +-inf) */
    if (a < 0.015625f) {                                 /* below 2^-6: subnormal grid 2^-9 */
        /* a * 512 is exact; rint rounds half to even in the default rounding mode.
         * A result of 8 is the smallest normal 0x08 = 2^-6, which the code below also gives. */
        const int m = (int)rintf(a * 512.0f);
        return sign | (uint8_t)m;
    }
    /* Normal range: round the 23-bit float mantissa to 3 bits, ties to even; a carry out
     * of the mantissa increments the exponent, which is the correct next binade. */
    const uint32_t u = f32_bits(a);
    uint32_t keep = u >> 20;                             /* exponent(8) | mantissa(3) */
    const uint32_t rem = u & 0xFFFFFu;
    if (rem > 0x80000u || (rem == 0x80000u && (keep & 1u))) keep += 1u;
    /* rebias exponent from 127 to 7: subtract (127-7) << 3 */
    const uint32_t code = keep - (120u << 3);
    if (code > 0x7Eu) return sign | 0x7E;                /* rounding reached 480: saturate */
    return sign | (uint8_t)code;
}

/* kv_w8_encode (attention_kvcache_w8.cuh:55-66). */
uint8_t oracle_w8_encode(float x, float scale, int fmt) {
    const float y = x / scale;
    if (fmt == ORACLE_W8_FP8_E4M3) return oracle_fp8_e4m3_from_f32(y);
    /* __float2int_rn: round to nearest, ties to even; then clamp to [-127,127] (:62-63). */
    int q = (int)rintf(y);
    q = (q < -127) ? -127 : ((q > 127) ? 127 : q);
    return (uint8_t)(int8_t)q;
}

/* kv_w8_decode (attention_kvcache_w8.cuh:71-82).  FP8 goes through bf16 in the
 * reference, which is exact for every E4M3 value (3 mantissa bits <= 7). */
float oracle_w8_decode(uint8_t code, int fmt) {
    if (fmt == ORACLE_W8_FP8_E4M3) return oracle_fp8_e4m3_to_f32(code);
    return (float)(int8_t)code;
}

/* ---------------------------------------------------------------------------------
 * KV append.
 * ------------------------------------------------------------------------------- */
void oracle_cache_write(void* kv_cache, const void* qkv, size_t elem_size,
                        const int* cur_lens, int B, int NH, int hs, int maxT) {
    /* attention_kvcache.cuh:59-63: src = b*3*NH*hs + h*hs + d; K at src + NH*hs,
     * V at src + 2*NH*hs; dst = (b*NH+h)*maxT*hs + cur_len*hs + d, V block offset
     * B*NH*maxT*hs. */
    uint8_t* dst = (uint8_t*)kv_cache;
    const uint8_t* src = (const uint8_t*)qkv;
    const size_t vblock = (size_t)B * NH * maxT * hs;
    for (int b = 0; b < B; b++) {
        const int cl = cur_lens[b];
        if (cl < 0 || cl >= maxT) continue;
        for (int h = 0; h < NH; h++) {
            const size_t s0 = (size_t)b * 3 * NH * hs + (size_t)h * hs;
            const size_t d0 = k_index(b, h, cl, NH, hs, maxT);
            memcpy(dst + d0 * elem_size, src + (s0 + (size_t)NH * hs) * elem_size, hs * elem_size);
            memcpy(dst + (vblock + d0) * elem_size, src + (s0 + 2 * (size_t)NH * hs) * elem_size,
                   hs * elem_size);
        }
    }
}

void oracle_cache_write_w8(uint8_t* kv_cache, float* kv_scale, const float* qkv,
                           const int* cur_lens, int B, int NH, int hs, int maxT, int fmt) {
    const float limit = (fmt == ORACLE_W8_FP8_E4M3) ? 448.0f : 127.0f;   /* :45-50 */
    const size_t vblock = (size_t)B * NH * maxT * hs;
    const size_t sblock = (size_t)B * NH * maxT;
    for (int row = 0; row < B * NH * 2; row++) {                     /* :119-123 */
        const int is_v = row >= B * NH;
        const int kh = row - (is_v ? B * NH : 0);
        const int b = kh / NH, h = kh % NH;
        const int cl = cur_lens[b];
        if (cl < 0 || cl >= maxT) continue;
        const float* src = qkv + (size_t)b * 3 * NH * hs + (size_t)h * hs +
                           (is_v ? 2 * (size_t)NH * hs : (size_t)NH * hs);       /* :126-127 */
        uint8_t* dst = kv_cache + (is_v ? vblock : 0) + (size_t)kh * maxT * hs + (size_t)cl * hs;
        float* sc = kv_scale + (is_v ? sblock : 0) + (size_t)kh * maxT + cl;
        float mx = 0.0f;                                                 /* :134-146 */
        for (int d = 0; d < hs; d++) mx = fmaxf(mx, fabsf(src[d]));
        const float scale = mx / limit;                                  /* :148 */
        *sc = scale;
        for (int d = 0; d < hs; d++)                                     /* :151-154 */
            dst[d] = (scale > 0.0f) ? oracle_w8_encode(src[d], scale, fmt) : (uint8_t)0;
    }
}

void oracle_dequant_w8(float* kv_out, const uint8_t* kv_cache, const float* kv_scale,
                       int B, int NH, int hs, int maxT, int fmt) {
    const size_t rows = (size_t)2 * B * NH * maxT;
    for (size_t r = 0; r < rows; r++) {
        const float s = kv_scale[r];
        for (int d = 0; d < hs; d++)
            kv_out[r * hs + d] = oracle_w8_decode(kv_cache[r * hs + d], fmt) * s;
    }
}

/* ---------------------------------------------------------------------------------
 * Seeded inputs.
 * SplitMix64 (Steele, Lea, Flood 2014): state += 0x9E3779B97F4A7C15, then the
 * xor-shift-multiply finaliser.  Uniforms are the top 53 bits scaled to [0,1);
 * Box-Muller: z0 = sqrt(-2 ln u1) cos(2 pi u2), z1 = ... sin(...), with u1 in (0,1].
 * ------------------------------------------------------------------------------- */
static inline uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void oracle_gen_normal(uint64_t seed, float* out, size_t n) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        const double u1 = ((double)(splitmix64(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        const double u2 = (double)(splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
        const double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(r * sin(two_pi * u2));
    }
}

void oracle_lab_rand(unsigned seed, float* out, size_t n) {
    srand(seed);
    for (size_t i = 0; i < n; i++) out[i] = (float)(rand() % 10000) / 5000.0f - 1.0f;
}

static double now_us(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec * 1e6 + (double)ts.tv_nsec * 1e-3;
}

static int cmp_double(const void* a, const void* b) {
    const double x = *(const double*)a, y = *(const double*)b;
    return (x > y) - (x < y);
}

double oracle_time_attention_f32(float* out, const float* qkv, const float* kv_cache,
                                 int B, int total, int NH, int hs, int maxT, float scale,
                                 int reps) {
    if (reps < 1) reps = 1;
    double* t = (double*)malloc(sizeof(double) * (size_t)reps);
    for (int r = 0; r < reps; r++) {
        const double t0 = now_us();
        oracle_attention_f32(out, qkv, kv_cache, B, total, NH, hs, maxT, scale);
        t[r] = now_us() - t0;
    }
    qsort(t, (size_t)reps, sizeof(double), cmp_double);
    const double med = t[reps / 2];
    free(t);
    return med;
}

/* ---------------------------------------------------------------------------------
 * GEMV6_fused / GEMV6_w8x2 per output (Inference_gpt2/GEMV.cuh:132-197,
 * GEMV_w8.cuh:64-157): an FP32 dot product of the row with x, the 8-bit row scale applied
 * once after the sum (GEMV_w8.cuh:136), the bias added (GEMV.cuh:192), the pre-GELU value
 * kept (:193) and GPT-2's tanh GELU with the reference's evaluation order (:195-197).
 * The reference sums in lane-strided order and reduces across a warp; this sums k in
 * ascending order, so the two agree to FP32 rounding of a K-term sum.
 * ------------------------------------------------------------------------------- */
float oracle_gelu_tanh(float v) {
    const float cube = 0.044715f * v * v * v;
    return 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + cube)));
}

void oracle_gemv(float* out, float* pre_gelu, const float* W, const float* w_scale, const float* x,
                 const float* bias, int B, int M, int K, int gelu) {
    for (int b = 0; b < B; b++) {
        const float* xb = x + (size_t)b * K;
        for (int m = 0; m < M; m++) {
            const float* wr = W + (size_t)m * K;
            float sum = 0.0f;
            for (int k = 0; k < K; k++) sum += wr[k] * xb[k];
            if (w_scale) sum *= w_scale[m];
            float pre = sum;
            if (bias) pre += bias[m];
            const size_t o = (size_t)b * M + m;
            if (pre_gelu) pre_gelu[o] = pre;
            out[o] = gelu ? oracle_gelu_tanh(pre) : pre;
        }
    }
}

double oracle_time_gemv(float* out, const float* W, const float* w_scale, const float* x, const float* bias,
                        int B, int M, int K, int reps) {
    if (reps < 1) reps = 1;
    double* t = (double*)malloc(sizeof(double) * (size_t)reps);
    for (int r = 0; r < reps; r++) {
        const double t0 = now_us();
        oracle_gemv(out, NULL, W, w_scale, x, bias, B, M, K, 0);
        t[r] = now_us() - t0;
    }
    qsort(t, (size_t)reps, sizeof(double), cmp_double);
    const double med = t[reps / 2];
    free(t);
    return med;
}
