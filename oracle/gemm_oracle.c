/*
 * CPU oracle for the flash-train FP32 GEMM family path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the checker
 * (or the timed CPU baseline) -- never as the product path.
 *
 * Functions:
 *   ft_oracle_gemm_ref   restatement of the reference kernel
 *                        (/root/reference/src/primitive/hygon/gemm/fp32_gemm.hip:18-31):
 *                        one output per (row, col), fp32 accumulator summed
 *                        over k in order, then alpha*acc + (c ? beta*c : 0).
 *   ft_oracle_gemm_f64   the same formula with every product and sum in
 *                        fp64 (the tolerance reference).
 *   ft_oracle_fill       the reference tests' deterministic fill
 *                        ((i * 2654435761) mod 199) / 199 - 0.5
 *                        (/root/reference/tests/api/gemm_numerics_test.cpp:30-32).
 *
 * Pinned by tests/test_oracle.py against: the reference tests' known answers
 * (gemm_api_test.cpp:392-438, :22-138, :330-390), exact integer arithmetic on
 * the deterministic-fill grid (gemm_numerics_test.cpp:129-137), numpy's fp64
 * matmul, and closed forms (identity, all-ones, rank-one).
 */
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

void ft_oracle_gemm_ref(const float* a, const float* b, const float* c, float alpha, float beta, float* d,
                        uint64_t m, uint64_t n, uint64_t k) {
    /* Loop order (row, depth, col) streams b by rows; every output still sums
     * its products in increasing depth order, exactly as the reference's
     * per-output loop does. */
    const int64_t rows = (int64_t)m;
#pragma omp parallel
    {
        float* acc = (float*)malloc(sizeof(float) * (n ? n : 1));
#pragma omp for schedule(dynamic, 1)
        for (int64_t row = 0; row < rows; ++row) {
            for (uint64_t col = 0; col < n; ++col) acc[col] = 0.0f;
            for (uint64_t depth = 0; depth < k; ++depth) {
                const float av    = a[(uint64_t)row * k + depth];
                const float* brow = b + depth * n;
                for (uint64_t col = 0; col < n; ++col) acc[col] += av * brow[col];
            }
            for (uint64_t col = 0; col < n; ++col) {
                const uint64_t i = (uint64_t)row * n + col;
                d[i]             = alpha * acc[col] + (c != NULL ? beta * c[i] : 0.0f);
            }
        }
        free(acc);
    }
}

void ft_oracle_gemm_f64(const float* a, const float* b, const float* c, double alpha, double beta, double* d,
                        uint64_t m, uint64_t n, uint64_t k) {
    const int64_t rows = (int64_t)m;
#pragma omp parallel
    {
        double* acc = (double*)malloc(sizeof(double) * (n ? n : 1));
#pragma omp for schedule(dynamic, 1)
        for (int64_t row = 0; row < rows; ++row) {
            for (uint64_t col = 0; col < n; ++col) acc[col] = 0.0;
            for (uint64_t depth = 0; depth < k; ++depth) {
                const double av   = (double)a[(uint64_t)row * k + depth];
                const float* brow = b + depth * n;
                for (uint64_t col = 0; col < n; ++col) acc[col] += av * (double)brow[col];
            }
            for (uint64_t col = 0; col < n; ++col) {
                const uint64_t i = (uint64_t)row * n + col;
                d[i]             = alpha * acc[col] + (c != NULL ? beta * (double)c[i] : 0.0);
            }
        }
        free(acc);
    }
}

void ft_oracle_fill(float* out, uint64_t count, uint64_t offset) {
    for (uint64_t i = 0; i < count; ++i)
        out[i] = (float)(((i + offset) * 2654435761ULL) % 199ULL) / 199.0f - 0.5f;
}

int ft_oracle_threads(void) {
#ifdef _OPENMP
    extern int omp_get_max_threads(void);
    return omp_get_max_threads();
#else
    return 1;
#endif
}
