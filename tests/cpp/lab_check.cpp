// lab_check.cpp -- the reference lab's correctness loop (attention_kvcache/attention_kvcache.cu
// :951-1041), driven through the C++ mirror of the reference entry points (kvattn_gpt2.hpp)
// on the HIP library, with the CPU oracle as the reference routine.
//
// Same inputs as the lab: srand(0), then qkv and the cache drawn from the same rand()
// stream as (rand() % 10000) / 5000 - 1 (B=1, NH=12, hs=64, maxT=1024); same check lengths
// {1, 64, 256, 512, 1024} and split count clamp(ceil(len/128), 4, 32) (:940-945); the lab's
// absolute tolerance 1e-4 (:1038) plus a 1e-5 norm-wise relative bound.  Beyond the lab
// (which only tests FP32): the BF16 cache, and an INT8 / FP8 cache appended one position
// at a time through kv_cache_write_w8.  Exit status 0 iff every check passes.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "kvattn_gpt2.hpp"
#include "kvattn_oracle.h"

#define HIP_OK(x)                                                                       \
    do {                                                                                \
        hipError_t e_ = (x);                                                            \
        if (e_ != hipSuccess) {                                                         \
            printf("HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
            exit(2);                                                                    \
        }                                                                               \
    } while (0)

static const int B = 1, NH = 12, hs = 64, maxT = 1024, MAX_SPLIT_S = 32;

static int calculate_split_S(int len) {
    int s = (len + 127) / 128;
    return s < 4 ? 4 : (s > MAX_SPLIT_S ? MAX_SPLIT_S : s);
}

// max-abs and norm-wise relative error per head; returns the number of failing heads.
static int validate(const char* what, int len, const float* got, const float* want, float abs_tol, float rel_tol) {
    float max_abs = 0.0f;
    double worst_rel = 0.0;
    int bad = 0;
    for (int h = 0; h < B * NH; h++) {
        double num = 0.0, den = 0.0;
        for (int d = 0; d < hs; d++) {
            const float g = got[h * hs + d], w = want[h * hs + d];
            const float diff = fabsf(g - w);
            if (!(diff <= max_abs)) max_abs = diff;
            num += (double)(g - w) * (g - w);
            den += (double)w * w;
        }
        const double rel = sqrt(num / (den > 0 ? den : 1e-30));
        if (rel > worst_rel) worst_rel = rel;
        if (!(rel <= rel_tol) || !(max_abs <= abs_tol)) bad++;
    }
    printf("  %-28s seq_len=%4d | max abs err %.3e | norm-rel %.3e%s\n", what, len, max_abs, worst_rel,
           bad ? "  <-- FAIL" : "");
    return bad;
}

static void to_bf16(const float* in, uint16_t* out, size_t n) { oracle_bf16_round_array(in, out, n); }

int main() {
    const int qkv_elems = B * 3 * NH * hs;
    const int cache_elems = 2 * B * NH * maxT * hs;
    const int out_elems = B * NH * hs;
    std::vector<float> stream((size_t)qkv_elems + cache_elems);
    oracle_lab_rand(0, stream.data(), stream.size());
    const float* qkv = stream.data();
    const float* cache = stream.data() + qkv_elems;

    float *d_qkv, *d_cache, *d_out, *d_po, *d_pl, *d_pm;
    HIP_OK(hipMalloc(&d_qkv, qkv_elems * sizeof(float)));
    HIP_OK(hipMalloc(&d_cache, cache_elems * sizeof(float)));
    HIP_OK(hipMalloc(&d_out, out_elems * sizeof(float)));
    HIP_OK(hipMalloc(&d_po, B * NH * MAX_SPLIT_S * hs * sizeof(float)));
    HIP_OK(hipMalloc(&d_pl, B * NH * MAX_SPLIT_S * sizeof(float)));
    HIP_OK(hipMalloc(&d_pm, B * NH * MAX_SPLIT_S * sizeof(float)));
    HIP_OK(hipMemcpy(d_qkv, qkv, qkv_elems * sizeof(float), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_cache, cache, cache_elems * sizeof(float), hipMemcpyHostToDevice));
    hipStream_t st;
    HIP_OK(hipStreamCreate(&st));

    std::vector<float> want(out_elems), got(out_elems), gotb(out_elems);
    std::vector<uint16_t> outb(out_elems);
    const int lens[] = {1, 64, 256, 512, 1024};
    int bad = 0;

    // ---- FP32 cache: small, large (B=1 -> cooperative), split + merge pair ----------
    printf("=== FP32 KV cache ===\n");
    for (int len : lens) {
        const int S = calculate_split_S(len);
        oracle_attention_f32(want.data(), qkv, cache, B, len, NH, hs, maxT, 1.0f / sqrtf((float)hs));
        kvattn_gpt2::set_cur_len(len - 1);
        for (int v = 0; v < 3; v++) {
            HIP_OK(hipMemset(d_out, 0xFF, out_elems * sizeof(float)));
            const char* name = v == 0 ? "attention_forward_kv_small" : v == 1 ? "attention_forward_kv_large"
                                                                              : "split + merge";
            if (v == 0) {
                kvattn_gpt2::attention_forward_kv_small(d_out, d_qkv, d_cache, B, NH, hs, maxT, st, KVATTN_KV_F32);
            } else if (v == 1) {
                kvattn_gpt2::attention_forward_kv_large(d_out, d_qkv, d_cache, B, NH, hs, maxT, st, d_po, d_pl,
                                                        d_pm, S, KVATTN_KV_F32);
            } else {
                kvattn_gpt2::attention_kv_split(d_po, d_pl, d_pm, d_qkv, d_cache, nullptr, B, NH, hs, maxT, S, st,
                                                KVATTN_KV_F32);
                kvattn_gpt2::attention_kv_merge(d_out, d_po, d_pl, d_pm, B, NH, hs, S, st, KVATTN_KV_F32);
            }
            HIP_OK(hipStreamSynchronize(st));
            HIP_OK(hipMemcpy(got.data(), d_out, out_elems * sizeof(float), hipMemcpyDeviceToHost));
            bad += validate(name, len, got.data(), want.data(), 1e-4f, 1e-5f);
        }
    }

    // ---- BF16 cache: the same inputs rounded to bf16 --------------------------------
    printf("=== BF16 KV cache ===\n");
    std::vector<uint16_t> qb(qkv_elems), cb(cache_elems);
    to_bf16(qkv, qb.data(), qkv_elems);
    to_bf16(cache, cb.data(), cache_elems);
    std::vector<float> qf(qkv_elems), cf(cache_elems);
    oracle_bf16_decode_array(qb.data(), qf.data(), qkv_elems);
    oracle_bf16_decode_array(cb.data(), cf.data(), cache_elems);
    uint16_t *d_qb, *d_cb, *d_ob;
    HIP_OK(hipMalloc(&d_qb, qkv_elems * 2));
    HIP_OK(hipMalloc(&d_cb, cache_elems * 2));
    HIP_OK(hipMalloc(&d_ob, out_elems * 2));
    HIP_OK(hipMemcpy(d_qb, qb.data(), qkv_elems * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_cb, cb.data(), cache_elems * 2, hipMemcpyHostToDevice));
    for (int len : lens) {
        const int S = calculate_split_S(len);
        oracle_attention_f32(want.data(), qf.data(), cf.data(), B, len, NH, hs, maxT, 1.0f / sqrtf((float)hs));
        kvattn_gpt2::set_cur_len(len - 1);
        for (int v = 0; v < 2; v++) {
            if (v == 0) kvattn_gpt2::attention_forward_kv_small(d_ob, d_qb, d_cb, B, NH, hs, maxT, st);
            else kvattn_gpt2::attention_forward_kv_large(d_ob, d_qb, d_cb, B, NH, hs, maxT, st, d_po, d_pl, d_pm, S);
            HIP_OK(hipStreamSynchronize(st));
            HIP_OK(hipMemcpy(outb.data(), d_ob, out_elems * 2, hipMemcpyDeviceToHost));
            oracle_bf16_decode_array(outb.data(), gotb.data(), out_elems);
            bad += validate(v == 0 ? "bf16 forward_kv_small" : "bf16 forward_kv_large", len, gotb.data(),
                            want.data(), 1e-2f, 1e-2f);
        }
    }

    // ---- 8-bit caches appended one position at a time --------------------------------
    for (int fmt = 0; fmt < 2; fmt++) {
        const int dt = fmt == 0 ? KVATTN_KV_INT8 : KVATTN_KV_FP8_E4M3;
        const int ofmt = fmt == 0 ? ORACLE_W8_INT8 : ORACLE_W8_FP8_E4M3;
        const int T8 = 256;
        printf("=== %s KV cache (appended) ===\n", fmt == 0 ? "INT8" : "FP8-E4M3");
        uint8_t* d_c8;
        float* d_sc;
        HIP_OK(hipMalloc(&d_c8, cache_elems / 1));
        HIP_OK(hipMalloc(&d_sc, 2 * B * NH * maxT * sizeof(float)));
        std::vector<uint8_t> c8(cache_elems, 0);
        std::vector<float> sc(2 * B * NH * maxT, 0.0f), tok(qkv_elems);
        std::vector<uint16_t> tokb(qkv_elems);
        for (int j = 0; j < T8; j++) {
            // token j: q from the lab stream, K and V rows = cache column j (bf16-rounded)
            for (int h = 0; h < NH; h++)
                for (int d = 0; d < hs; d++) {
                    tok[h * hs + d] = qkv[h * hs + d];
                    tok[(NH + h) * hs + d] = cache[((size_t)h * maxT + j) * hs + d];
                    tok[(2 * NH + h) * hs + d] = cache[((size_t)(NH + h) * maxT + j) * hs + d];
                }
            to_bf16(tok.data(), tokb.data(), qkv_elems);
            HIP_OK(hipMemcpy(d_qb, tokb.data(), qkv_elems * 2, hipMemcpyHostToDevice));
            kvattn_gpt2::set_cur_len(j);
            kvattn_gpt2::kv_cache_write_w8(d_c8, d_sc, d_qb, B, NH, hs, maxT, st, dt);
            std::vector<float> tf(qkv_elems);
            oracle_bf16_decode_array(tokb.data(), tf.data(), qkv_elems);
            const int cl = j;
            oracle_cache_write_w8(c8.data(), sc.data(), tf.data(), &cl, B, NH, hs, maxT, ofmt);
        }
        HIP_OK(hipStreamSynchronize(st));
        std::vector<uint8_t> gc8(cache_elems);
        std::vector<float> gsc(sc.size());
        HIP_OK(hipMemcpy(gc8.data(), d_c8, cache_elems, hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(gsc.data(), d_sc, gsc.size() * 4, hipMemcpyDeviceToHost));
        size_t code_mismatch = 0, scale_mismatch = 0;
        for (int kvh = 0; kvh < 2 * NH; kvh++)
            for (int j = 0; j < T8; j++) {
                const size_t r = (size_t)kvh * maxT + j;
                if (memcmp(&gsc[r], &sc[r], 4) != 0) scale_mismatch++;
                code_mismatch += memcmp(&gc8[r * hs], &c8[r * hs], hs) != 0;
            }
        printf("  codes: %zu mismatching rows, scales: %zu mismatching rows (of %d)%s\n", code_mismatch,
               scale_mismatch, 2 * NH * T8, (code_mismatch || scale_mismatch) ? "  <-- FAIL" : "");
        bad += (int)(code_mismatch + scale_mismatch);
        std::vector<float> deq(cache_elems);
        oracle_dequant_w8(deq.data(), c8.data(), sc.data(), B, NH, hs, maxT, ofmt);
        std::vector<float> tf(qkv_elems);
        oracle_bf16_decode_array(tokb.data(), tf.data(), qkv_elems);
        oracle_attention_f32(want.data(), tf.data(), deq.data(), B, T8, NH, hs, maxT, 1.0f / sqrtf((float)hs));
        kvattn_gpt2::attention_forward_kv_small_w8(d_ob, d_qb, d_c8, d_sc, B, NH, hs, maxT, st, dt);
        HIP_OK(hipStreamSynchronize(st));
        HIP_OK(hipMemcpy(outb.data(), d_ob, out_elems * 2, hipMemcpyDeviceToHost));
        oracle_bf16_decode_array(outb.data(), gotb.data(), out_elems);
        bad += validate("w8 forward_kv_small", T8, gotb.data(), want.data(), 2e-2f, 2e-2f);
        kvattn_gpt2::attention_forward_kv_large_w8(d_ob, d_qb, d_c8, d_sc, B, NH, hs, maxT, st, d_po, d_pl, d_pm,
                                                   8, dt);
        HIP_OK(hipStreamSynchronize(st));
        HIP_OK(hipMemcpy(outb.data(), d_ob, out_elems * 2, hipMemcpyDeviceToHost));
        oracle_bf16_decode_array(outb.data(), gotb.data(), out_elems);
        bad += validate("w8 forward_kv_large", T8, gotb.data(), want.data(), 2e-2f, 2e-2f);
        HIP_OK(hipFree(d_c8));
        HIP_OK(hipFree(d_sc));
    }

    printf("%s\n", bad ? "-> FAILED" : "-> all passed");
    return bad ? 1 : 0;
}
