// Eager per-call cost of kvattn_decode from C++, the way the reference engine calls its
// attention per layer without --graph (inference_gpt2_opt.cu:298-347): `layers` calls per
// step, one per layer cache, AUTO with the host's length, back to back on one stream.
// Reports, as one JSON line, the GPU clock per call (HIP events around `steps` steps) and
// the host time per call spent enqueueing them.  bench.py runs it next to its own eager
// figure, which goes through Python's ctypes.
//
// Usage: eager_timing <kv_dtype f32|bf16|int8|fp8> <B> <NH> <maxT> <cur_len> <layers> <steps>
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "kvattn.h"

#define CK(x)                                                                                   \
    do {                                                                                        \
        hipError_t e_ = (x);                                                                    \
        if (e_ != hipSuccess) {                                                                 \
            std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            return 1;                                                                           \
        }                                                                                       \
    } while (0)

int main(int argc, char** argv) {
    if (argc != 8) {
        std::fprintf(stderr, "usage: %s <f32|bf16|int8|fp8> <B> <NH> <maxT> <cur_len> <layers> <steps>\n", argv[0]);
        return 2;
    }
    const char* dts = argv[1];
    const int dt = !std::strcmp(dts, "f32") ? KVATTN_KV_F32 : !std::strcmp(dts, "bf16") ? KVATTN_KV_BF16
                 : !std::strcmp(dts, "int8") ? KVATTN_KV_INT8 : !std::strcmp(dts, "fp8") ? KVATTN_KV_FP8_E4M3 : -1;
    const int B = std::atoi(argv[2]), NH = std::atoi(argv[3]), maxT = std::atoi(argv[4]);
    const int cur = std::atoi(argv[5]), layers = std::atoi(argv[6]), steps = std::atoi(argv[7]);
    const int hs = 64;
    if (dt < 0 || B < 1 || NH < 1 || maxT < 1 || cur < 0 || cur >= maxT || layers < 1 || steps < 1) {
        std::fprintf(stderr, "bad arguments\n");
        return 2;
    }
    const bool w8 = dt == KVATTN_KV_INT8 || dt == KVATTN_KV_FP8_E4M3;
    const size_t act = dt == KVATTN_KV_F32 ? 4 : 2;                  // q and out: f32 or bf16
    const size_t elem = dt == KVATTN_KV_F32 ? 4 : (dt == KVATTN_KV_BF16 ? 2 : 1);
    const size_t rows = (size_t)2 * B * NH * maxT;
    const size_t cache_bytes = rows * hs * elem;

    // Seeded bytes for every cache: small finite values in every format (bf16 / f32 halves
    // with a cleared exponent top bit; FP8 codes below 0x78; INT8 any code), row scales 1e-2.
    std::mt19937 rng(7);
    std::vector<uint8_t> host(cache_bytes);
    for (size_t i = 0; i < cache_bytes; ++i) {
        uint8_t v = (uint8_t)(rng() & 0xff);
        if (dt == KVATTN_KV_FP8_E4M3) v &= 0x77;
        else if (!w8 && (i % elem) == elem - 1) v &= 0x3f;   // top byte of each value: |x| < 2
        host[i] = v;
    }
    std::vector<float> scales(w8 ? rows : 0, 1e-2f);
    std::vector<uint8_t> qhost((size_t)B * 3 * NH * hs * act);
    for (auto& v : qhost) v = (uint8_t)(rng() & 0x3f);

    std::vector<void*> cache(layers), out(layers);
    std::vector<float*> scale(layers, nullptr);
    for (int l = 0; l < layers; ++l) {
        CK(hipMalloc(&cache[l], cache_bytes));
        CK(hipMemcpy(cache[l], host.data(), cache_bytes, hipMemcpyHostToDevice));
        CK(hipMalloc(&out[l], (size_t)B * NH * hs * act));
        if (w8) {
            CK(hipMalloc(&scale[l], rows * sizeof(float)));
            CK(hipMemcpy(scale[l], scales.data(), rows * sizeof(float), hipMemcpyHostToDevice));
        }
    }
    void* qkv = nullptr;
    CK(hipMalloc(&qkv, qhost.size()));
    CK(hipMemcpy(qkv, qhost.data(), qhost.size(), hipMemcpyHostToDevice));
    int* len = nullptr;
    CK(hipMalloc(&len, sizeof(int)));
    CK(hipMemcpy(len, &cur, sizeof(int), hipMemcpyHostToDevice));
    const size_t wb = kvattn_workspace_bytes(B, NH, hs, maxT, 0);
    void* ws = nullptr;
    CK(hipMalloc(&ws, wb));
    hipStream_t s;
    CK(hipStreamCreate(&s));
    if (kvattn_workspace_init(ws, wb, s) != KVATTN_OK) {
        std::fprintf(stderr, "kvattn_workspace_init failed\n");
        return 1;
    }
    auto step = [&]() -> int {
        for (int l = 0; l < layers; ++l) {
            const int r = kvattn_decode(out[l], qkv, cache[l], scale[l], B, NH, hs, maxT, len, 0, cur, ws, wb, 0,
                                        KVATTN_AUTO, dt, s);
            if (r != KVATTN_OK) return r;
        }
        return KVATTN_OK;
    };
    for (int w = 0; w < 20; ++w)
        if (int r = step()) {
            std::fprintf(stderr, "kvattn_decode returned %d\n", r);
            return 1;
        }
    CK(hipStreamSynchronize(s));

    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    CK(hipEventRecord(e0, s));
    const auto t0 = std::chrono::steady_clock::now();
    for (int k = 0; k < steps; ++k)
        if (int r = step()) {
            std::fprintf(stderr, "kvattn_decode returned %d\n", r);
            return 1;
        }
    const auto t1 = std::chrono::steady_clock::now();
    CK(hipEventRecord(e1, s));
    CK(hipEventSynchronize(e1));
    float ms = 0.0f;
    CK(hipEventElapsedTime(&ms, e0, e1));
    unsigned status = 0;
    if (kvattn_workspace_status(ws, wb, 0, s, nullptr) != KVATTN_OK) status = 1;
    const double calls = (double)steps * layers;
    std::printf("{\"kv_dtype\": \"%s\", \"B\": %d, \"NH\": %d, \"maxT\": %d, \"cur_len\": %d, \"layers\": %d, "
                "\"steps\": %d, \"us_per_call\": %.4f, \"host_enqueue_us_per_call\": %.4f, \"workspace_status\": %u}\n",
                dts, B, NH, maxT, cur, layers, steps, ms * 1000.0 / calls,
                std::chrono::duration<double, std::micro>(t1 - t0).count() / calls, status);
    return 0;
}
