// step_check.cpp -- the attention block of the reference engine's decode step
// (forward_kv_graph_ready, inference_gpt2_opt.cu:298-355) on the C ABI, from C++:
// for each of 12 layers, the append and the attention in one launch
// (kvattn_gpt2::kv_append_attention) followed by the attention output projection
// (kvattn_gpt2::launch_GEMV6_fused, bias included), captured ONCE with hipStreamBeginCapture
// and replayed for every token T = 1..1024 with the device length written by
// kvattn_gpt2::set_cur_len_async before each replay.  (The reference captures a small and a
// large graph, :420-449, and writes the length with a blocking cudaMemcpyToSymbol, :548.)
//
// Inputs: every token's q/K/V for every layer ~ N(0,1) (oracle_gen_normal, seed 7), rounded
// to bf16; projection weights ~ N(0,1)/sqrt(768) and biases ~ N(0,1), bf16.  Checks, at 12
// tokens around the plan edges: each layer's attention output against oracle_attention_f32
// on the host's own copy of the appended cache (BF16 bar 1e-2), and each projection output
// against oracle_gemv applied to the GPU's attention output (1e-2); after the last token,
// every appended cache row bit for bit.  Prints the mean GPU time per token.  Exit status 0
// iff every check passes.
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

static const int L = 12, B = 1, NH = 12, hs = 64, C = NH * hs, maxT = 1024;

// Norm-wise relative error and max-abs error relative to max|want| over n values.
static bool close_enough(const float* got, const float* want, int n, double tol, double* nrel) {
    double num = 0.0, den = 0.0, mabs = 0.0, wmax = 0.0;
    for (int i = 0; i < n; i++) {
        const double d = (double)got[i] - want[i];
        if (!(fabs(d) <= mabs)) mabs = fabs(d);
        if (fabs(want[i]) > wmax) wmax = fabs(want[i]);
        num += d * d;
        den += (double)want[i] * want[i];
    }
    *nrel = sqrt(num / (den > 0 ? den : 1e-30));
    return *nrel <= tol && mabs <= tol * (wmax > 0 ? wmax : 1.0);
}

int main() {
    const size_t qkv_elems = (size_t)B * 3 * C;                // one layer, one token
    const size_t cache_elems = (size_t)2 * B * NH * maxT * hs;  // one layer
    // Every token's qkv for every layer, bf16, resident on the device.
    std::vector<float> vals((size_t)maxT * L * qkv_elems);
    oracle_gen_normal(7, vals.data(), vals.size());
    std::vector<uint16_t> qkv_b(vals.size());
    oracle_bf16_round_array(vals.data(), qkv_b.data(), vals.size());
    std::vector<float> qkv_f(vals.size());
    oracle_bf16_decode_array(qkv_b.data(), qkv_f.data(), vals.size());

    std::vector<float> wvals((size_t)L * C * C), bvals((size_t)L * C);
    oracle_gen_normal(8, wvals.data(), wvals.size());
    oracle_gen_normal(9, bvals.data(), bvals.size());
    for (auto& w : wvals) w /= sqrtf((float)C);
    std::vector<uint16_t> w_b(wvals.size()), b_b(bvals.size());
    oracle_bf16_round_array(wvals.data(), w_b.data(), wvals.size());
    oracle_bf16_round_array(bvals.data(), b_b.data(), bvals.size());
    std::vector<float> w_f(wvals.size()), b_f(bvals.size());
    oracle_bf16_decode_array(w_b.data(), w_f.data(), w_b.size());
    oracle_bf16_decode_array(b_b.data(), b_f.data(), b_b.size());

    uint16_t *d_all, *d_qkv, *d_cache, *d_atty, *d_proj, *d_w, *d_bias;
    HIP_OK(hipMalloc(&d_all, qkv_b.size() * 2));
    HIP_OK(hipMalloc(&d_qkv, (size_t)L * qkv_elems * 2));
    HIP_OK(hipMalloc(&d_cache, (size_t)L * cache_elems * 2));
    HIP_OK(hipMalloc(&d_atty, (size_t)L * C * 2));
    HIP_OK(hipMalloc(&d_proj, (size_t)L * C * 2));
    HIP_OK(hipMalloc(&d_w, w_b.size() * 2));
    HIP_OK(hipMalloc(&d_bias, b_b.size() * 2));
    HIP_OK(hipMemcpy(d_all, qkv_b.data(), qkv_b.size() * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_w, w_b.data(), w_b.size() * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_bias, b_b.data(), b_b.size() * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemset(d_cache, 0, (size_t)L * cache_elems * 2));

    hipStream_t st;
    HIP_OK(hipStreamCreate(&st));
    int* d_len = kvattn_gpt2::cur_len_symbol();
    const size_t ws_bytes = kvattn_workspace_bytes(B, NH, hs, maxT, 0);
    void* ws;
    HIP_OK(hipMalloc(&ws, ws_bytes));
    kvattnCheck(kvattn_workspace_init(ws, ws_bytes, st));
    HIP_OK(hipStreamSynchronize(st));

    // The whole block, captured once.
    hipGraph_t graph;
    hipGraphExec_t exec;
    HIP_OK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    for (int l = 0; l < L; l++) {
        uint16_t* qkv_l = d_qkv + (size_t)l * qkv_elems;
        uint16_t* cache_l = d_cache + (size_t)l * cache_elems;   // layer stride 2*B*NH*maxT*hs (:324)
        uint16_t* atty_l = d_atty + (size_t)l * C;
        kvattn_gpt2::kv_append_attention(atty_l, qkv_l, cache_l, nullptr, B, NH, hs, maxT, ws, ws_bytes, st,
                                         KVATTN_KV_BF16, d_len);
        kvattn_gpt2::launch_GEMV6_fused(d_proj + (size_t)l * C, nullptr, d_w + (size_t)l * C * C, atty_l,
                                        d_bias + (size_t)l * C, C, C, false, st);
    }
    HIP_OK(hipStreamEndCapture(st, &graph));
    HIP_OK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));

    const int checks[] = {1, 2, 150, 151, 256, 257, 300, 512, 513, 700, 1023, 1024};
    size_t next_check = 0;
    std::vector<uint16_t> atty_b((size_t)L * C), proj_b((size_t)L * C);
    std::vector<float> atty_f((size_t)L * C), proj_f((size_t)L * C), want(C);
    std::vector<float> host_cache((size_t)L * cache_elems, 0.0f);   // the host's copy of every append
    int bad = 0, checked = 0;
    double worst_att = 0.0, worst_proj = 0.0;
    float gpu_ms = 0.0f;
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    float seg_ms = 0.0f;
    HIP_OK(hipEventRecord(e0, st));
    for (int t = 0; t < maxT; t++) {   // token at position t: attends T = t + 1 positions
        HIP_OK(hipMemcpyAsync(d_qkv, d_all + (size_t)t * L * qkv_elems, (size_t)L * qkv_elems * 2,
                              hipMemcpyDeviceToDevice, st));
        kvattn_gpt2::set_cur_len_async(t, st, d_len);
        HIP_OK(hipGraphLaunch(exec, st));
        for (int l = 0; l < L; l++) {
            const float* tok = qkv_f.data() + ((size_t)t * L + l) * qkv_elems;
            float* hc = host_cache.data() + (size_t)l * cache_elems;
            for (int h = 0; h < NH; h++) {
                memcpy(hc + ((size_t)h * maxT + t) * hs, tok + (size_t)(NH + h) * hs, hs * sizeof(float));
                memcpy(hc + ((size_t)(NH + h) * maxT + t) * hs, tok + (size_t)(2 * NH + h) * hs, hs * sizeof(float));
            }
        }
        if (next_check < sizeof(checks) / sizeof(checks[0]) && checks[next_check] == t + 1) {
            next_check++;
            HIP_OK(hipEventRecord(e1, st));
            HIP_OK(hipEventSynchronize(e1));
            HIP_OK(hipEventElapsedTime(&seg_ms, e0, e1));
            gpu_ms += seg_ms;
            HIP_OK(hipMemcpy(atty_b.data(), d_atty, atty_b.size() * 2, hipMemcpyDeviceToHost));
            HIP_OK(hipMemcpy(proj_b.data(), d_proj, proj_b.size() * 2, hipMemcpyDeviceToHost));
            oracle_bf16_decode_array(atty_b.data(), atty_f.data(), atty_b.size());
            oracle_bf16_decode_array(proj_b.data(), proj_f.data(), proj_b.size());
            for (int l = 0; l < L; l++) {
                const float* tok = qkv_f.data() + ((size_t)t * L + l) * qkv_elems;
                double nrel;
                oracle_attention_f32(want.data(), tok, host_cache.data() + (size_t)l * cache_elems, B, t + 1, NH,
                                     hs, maxT, 1.0f / sqrtf((float)hs));
                if (!close_enough(atty_f.data() + (size_t)l * C, want.data(), C, 1e-2, &nrel)) {
                    printf("  attention layer %d T=%d: norm-rel %.3e  <-- FAIL\n", l, t + 1, nrel);
                    bad++;
                }
                if (nrel > worst_att) worst_att = nrel;
                oracle_gemv(want.data(), nullptr, w_f.data() + (size_t)l * C * C, nullptr,
                            atty_f.data() + (size_t)l * C, b_f.data() + (size_t)l * C, 1, C, C, 0);
                if (!close_enough(proj_f.data() + (size_t)l * C, want.data(), C, 1e-2, &nrel)) {
                    printf("  projection layer %d T=%d: norm-rel %.3e  <-- FAIL\n", l, t + 1, nrel);
                    bad++;
                }
                if (nrel > worst_proj) worst_proj = nrel;
                checked++;
            }
            HIP_OK(hipEventRecord(e0, st));
        }
    }
    HIP_OK(hipStreamSynchronize(st));

    // Every appended row, bit for bit.
    std::vector<uint16_t> cache_b((size_t)L * cache_elems);
    HIP_OK(hipMemcpy(cache_b.data(), d_cache, cache_b.size() * 2, hipMemcpyDeviceToHost));
    size_t row_mismatch = 0;
    for (int t = 0; t < maxT; t++)
        for (int l = 0; l < L; l++)
            for (int kv = 0; kv < 2; kv++)
                for (int h = 0; h < NH; h++) {
                    const uint16_t* want_row = qkv_b.data() + ((size_t)t * L + l) * qkv_elems + (size_t)((1 + kv) * NH + h) * hs;
                    const uint16_t* got_row = cache_b.data() + (size_t)l * cache_elems + ((size_t)(kv * NH + h) * maxT + t) * hs;
                    row_mismatch += memcmp(want_row, got_row, hs * 2) != 0;
                }
    if (row_mismatch) bad++;
    printf("  %d (layer, token) checks: worst attention norm-rel %.3e, worst projection norm-rel %.3e\n", checked,
           worst_att, worst_proj);
    printf("  appended cache rows: %zu mismatching of %d\n", row_mismatch, maxT * L * 2 * NH);
    printf("  12-layer block (append + attention + projection) replayed for T = 1..%d: %.2f us per token "
           "(GPU time, including the per-token qkv copy and length write)\n",
           maxT, gpu_ms * 1000.0 / maxT);
    HIP_OK(hipGraphExecDestroy(exec));
    HIP_OK(hipGraphDestroy(graph));
    printf(bad ? "-> FAILED\n" : "-> all passed\n");
    return bad ? 1 : 0;
}
