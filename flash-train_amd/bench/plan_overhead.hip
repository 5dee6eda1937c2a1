// Host-side cost of re-executing a cached Plan: creates one Plan for a small
// GEMM, then times `iters` back-to-back ftrainPlanExecutePrimitive calls
// without synchronizing (host wall clock / iters), plus the convenience
// ftrainGemm call, which re-creates Args and Plan per call (selection-cache
// hit).  Mirrors the reference's L2/L3 tiers
// (benchmarks/csrc/ftrain_bench.cpp:103-177).  For scale it also times bare
// hipLaunchKernel calls of an empty kernel taking an argument block of the
// GEMM kernels' size: the floor under any launch.  Prints one JSON object.
//
// usage: plan_overhead [m n k] [iters]
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include <hip/hip_runtime.h>

#include <flash_train/flash_train.h>

#define CHECK_HIP(x)                                                             \
    do {                                                                         \
        hipError_t e_ = (x);                                                     \
        if (e_ != hipSuccess) {                                                  \
            std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));         \
            return 2;                                                            \
        }                                                                        \
    } while (0)
#define CHECK_FT(x)                                                              \
    do {                                                                         \
        FTrainStatus s_ = (x);                                                   \
        if (s_ != FTRAIN_STATUS_SUCCESS) {                                       \
            std::fprintf(stderr, "%s: %u %s\n", #x, s_, ftrainGetLastMessage()); \
            return 3;                                                            \
        }                                                                        \
    } while (0)

// Same size as the GEMM kernels' parameter block (pointers, scalars, shape,
// leading dimensions).
struct EmptyArgs {
    const void* p[4];
    float s[2];
    int32_t i[6];
    int64_t ld[4];
};
__global__ void empty_kernel(EmptyArgs) {}

static FTrainStorageView mat(void* p, const int64_t* dims) {
    return FTrainStorageView{p, dims, nullptr, 2, FTRAIN_NUMERIC_TYPE_FP32, FTRAIN_INDEX_TYPE_CONTINUOUS, false};
}
static FTrainStorageView scalar(float* p) {
    return FTrainStorageView{p, nullptr, nullptr, 0, FTRAIN_NUMERIC_TYPE_FP32, FTRAIN_INDEX_TYPE_CONTINUOUS, true};
}

int main(int argc, char** argv) {
    const int64_t m = argc > 3 ? std::atoll(argv[1]) : 127;
    const int64_t n = argc > 3 ? std::atoll(argv[2]) : 97;
    const int64_t k = argc > 3 ? std::atoll(argv[3]) : 33;
    const int iters = argc > 4 ? std::atoi(argv[4]) : (argc == 2 ? std::atoi(argv[1]) : 10000);

    float *a = nullptr, *b = nullptr, *d = nullptr;
    CHECK_HIP(hipMalloc(&a, sizeof(float) * m * k));
    CHECK_HIP(hipMalloc(&b, sizeof(float) * k * n));
    CHECK_HIP(hipMalloc(&d, sizeof(float) * m * n));
    CHECK_HIP(hipMemset(a, 0, sizeof(float) * m * k));
    CHECK_HIP(hipMemset(b, 0, sizeof(float) * k * n));
    hipStream_t stream;
    CHECK_HIP(hipStreamCreate(&stream));

    const int64_t ad[2] = {m, k}, bd[2] = {k, n}, cd[2] = {m, n};
    float alpha = 1.f, beta = 0.f;

    FTrainPattern pattern;
    FTrainTensorId ta, tb, tc, td, tal, tbe;
    FTrainGemmOpId op;
    CHECK_FT(ftrainPatternCreate(&pattern));
    for (FTrainTensorId* t : {&ta, &tb, &tc, &td, &tal, &tbe}) CHECK_FT(ftrainPatternAddTensor(pattern, t));
    CHECK_FT(ftrainPatternAddGemm(pattern, &op, ta, tb, tc, td, tal, tbe));
    FTrainOps ops;
    CHECK_FT(ftrainOpsCreate(&ops, pattern));
    FTrainArgs args;
    CHECK_FT(ftrainArgsCreate(&args, ops));
    CHECK_FT(ftrainArgsSetTensor(args, ta, mat(a, ad)));
    CHECK_FT(ftrainArgsSetTensor(args, tb, mat(b, bd)));
    CHECK_FT(ftrainArgsSetTensor(args, tc, mat(nullptr, cd)));
    CHECK_FT(ftrainArgsSetTensor(args, td, mat(d, cd)));
    CHECK_FT(ftrainArgsSetTensor(args, tal, scalar(&alpha)));
    CHECK_FT(ftrainArgsSetTensor(args, tbe, scalar(&beta)));
    CHECK_FT(ftrainArgsSetGemm(args, op, FTRAIN_NUMERIC_TYPE_FP32));
    FTrainPlan plan;
    CHECK_FT(ftrainPlanCreate(&plan, args));
    const char* name = nullptr;
    CHECK_FT(ftrainPlanGetPrimitiveName(plan, 0, &name));

    using clock = std::chrono::steady_clock;
    for (int i = 0; i < 100; ++i) CHECK_FT(ftrainPlanExecutePrimitive(plan, 0, nullptr, 0, stream));
    CHECK_HIP(hipStreamSynchronize(stream));

    // Cached Plan re-execution (host cost per call, no sync inside the loop).
    auto t0 = clock::now();
    for (int i = 0; i < iters; ++i) CHECK_FT(ftrainPlanExecutePrimitive(plan, 0, nullptr, 0, stream));
    auto t1 = clock::now();
    CHECK_HIP(hipStreamSynchronize(stream));
    auto t2 = clock::now();
    const double exec_us = std::chrono::duration<double, std::micro>(t1 - t0).count() / iters;
    const double exec_drain_us = std::chrono::duration<double, std::micro>(t2 - t0).count() / iters;

    // Device time per call with events around a batch.
    hipEvent_t e0, e1;
    CHECK_HIP(hipEventCreate(&e0));
    CHECK_HIP(hipEventCreate(&e1));
    CHECK_HIP(hipEventRecord(e0, stream));
    for (int i = 0; i < 1000; ++i) CHECK_FT(ftrainPlanExecutePrimitive(plan, 0, nullptr, 0, stream));
    CHECK_HIP(hipEventRecord(e1, stream));
    CHECK_HIP(hipEventSynchronize(e1));
    float ms = 0.f;
    CHECK_HIP(hipEventElapsedTime(&ms, e0, e1));

    // Convenience API: Args + Plan per call through the selection cache.
    const int conv_iters = iters / 10 > 0 ? iters / 10 : 1;
    auto t3 = clock::now();
    for (int i = 0; i < conv_iters; ++i)
        CHECK_FT(ftrainGemm(mat(a, ad), mat(b, bd), mat(nullptr, cd), mat(d, cd), scalar(&alpha), scalar(&beta),
                            FTRAIN_NUMERIC_TYPE_FP32, nullptr, 0, stream));
    auto t4 = clock::now();
    CHECK_HIP(hipStreamSynchronize(stream));
    const double conv_us = std::chrono::duration<double, std::micro>(t4 - t3).count() / conv_iters;

    // Bare launch floor: the same number of hipLaunchKernel calls of an empty
    // kernel on the same stream.
    EmptyArgs ea{};
    void* eargs[] = {&ea};
    for (int i = 0; i < 100; ++i)
        CHECK_HIP(hipLaunchKernel(reinterpret_cast<const void*>(&empty_kernel), dim3(1), dim3(64), eargs, 0, stream));
    CHECK_HIP(hipStreamSynchronize(stream));
    auto t5 = clock::now();
    for (int i = 0; i < iters; ++i)
        CHECK_HIP(hipLaunchKernel(reinterpret_cast<const void*>(&empty_kernel), dim3(1), dim3(64), eargs, 0, stream));
    auto t6 = clock::now();
    CHECK_HIP(hipStreamSynchronize(stream));
    const double bare_us = std::chrono::duration<double, std::micro>(t6 - t5).count() / iters;

    std::printf(
        "{\"shape\": [%lld, %lld, %lld], \"primitive\": \"%s\", \"iters\": %d, \"plan_execute_host_us\": %.3f, "
        "\"plan_execute_with_drain_us\": %.3f, \"device_us_per_call\": %.3f, \"convenience_host_us\": %.3f, "
        "\"bare_launch_host_us\": %.3f}\n",
        (long long)m, (long long)n, (long long)k, name, iters, exec_us, exec_drain_us, ms * 1000.0 / 1000, conv_us,
        bare_us);

    ftrainPlanDestroy(plan);
    ftrainArgsDestroy(args);
    ftrainOpsDestroy(ops);
    ftrainPatternDestroy(pattern);
    hipFree(a);
    hipFree(b);
    hipFree(d);
    hipStreamDestroy(stream);
    return 0;
}
