// One-pass skinny-m kernel for bf16 / fp16 inputs (fp32 accumulation), the
// 16-bit counterpart of gemv_pass in kernels.hip.  Device code and its
// host-side selector.
#include "half_tile.hpp"

namespace ftrain::gemm {

namespace {

using hdev::from_float;
using hdev::to_float;
using hdev::u32x2;
using hdev::u32x4;

// m <= MR <= kGemvHalfRows, row-major a and b (16-byte aligned rows,
// k % 8 == 0, n % 8 == 0; a column-major a would need m % 8 == 0, more rows
// than the kernel takes).
// Workgroup x owns output columns [64x, 64x + 64) over all of k, so d is
// written directly.  Lane (r = lane / 8, q = lane % 8) of wave w takes
// columns 8q .. 8q+7 and, per step, the 4 consecutive k rows
// 4*(8*(w + NW*j) + r) + t, t = 0..3: one 16-byte load of b per row (8 lanes
// cover a row's 128 bytes) and one 8-byte load of a's 4 values per row of a.
// U steps are loaded before any is used.  Products and sums in fp32;
// reduction in a fixed order: a butterfly over the 8 lanes that share
// columns, then the NW wave sums in wave order through LDS.
template <bool BF16, int NW, int U, int MR>
__global__ __launch_bounds__(NW * 64) void gemv_pass_half(HalfGemmParams p) {
    using u16      = unsigned short;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane >> 3, q = lane & 7;
    const int M = p.m, N = p.n, K = p.k;
    // Columns past n (n % 8 == 0) and rows of a past m are read at a clamped
    // index instead of behind a branch (which would give every load a block
    // of its own); they feed only sums the final store skips.
    const int col0              = min(blockIdx.x * kGemvHalfCols + 8 * q, N - 8);
    const u16* __restrict__ A   = static_cast<const u16*>(p.a);
    const u16* __restrict__ B   = static_cast<const u16*>(p.b);
    const size_t lda = p.lda, ldb = p.ldb;
    constexpr int KSTEP = 32 * NW;  // k rows per step over the workgroup

    float acc[MR][8];
#pragma unroll
    for (int i = 0; i < MR; ++i)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[i][c] = 0.f;

    // b rows k0 .. k0+3 (8 packed values each) and a's values at those rows
    // (k % 8 == 0, so a step is whole or past the end).
    auto load = [&](int k0, u32x4 (&bv)[4], float (&av)[MR][4]) {
#pragma unroll
        for (int t = 0; t < 4; ++t) bv[t] = *reinterpret_cast<const u32x4*>(B + (size_t)(k0 + t) * ldb + col0);
#pragma unroll
        for (int i = 0; i < MR; ++i) {
            const u32x2 v = *reinterpret_cast<const u32x2*>(A + (size_t)min(i, M - 1) * lda + k0);
#pragma unroll
            for (int t = 0; t < 4; ++t) av[i][t] = to_float<BF16>(u16(v[t / 2] >> (16 * (t % 2))));
        }
    };
    auto fma = [&](const u32x4 (&bv)[4], const float (&av)[MR][4]) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float bf[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) bf[c] = to_float<BF16>(u16(bv[t][c / 2] >> (16 * (c % 2))));
#pragma unroll
            for (int i = 0; i < MR; ++i)
#pragma unroll
                for (int c = 0; c < 8; ++c) acc[i][c] += av[i][t] * bf[c];
        }
    };

    int k = 4 * (8 * wave + r);
    for (; k + (U - 1) * KSTEP + 3 < K; k += U * KSTEP) {
        u32x4 bv[U][4];
        float av[U][MR][4];
#pragma unroll
        for (int u = 0; u < U; ++u) load(k + u * KSTEP, bv[u], av[u]);
#pragma unroll
        for (int u = 0; u < U; ++u) fma(bv[u], av[u]);
    }
    for (; k < K; k += KSTEP) {
        u32x4 bv[4];
        float av[MR][4];
        load(k, bv, av);
        fma(bv, av);
    }

#pragma unroll
    for (int sh = 8; sh < 64; sh <<= 1)
#pragma unroll
        for (int i = 0; i < MR; ++i)
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[i][c] += __shfl_xor(acc[i][c], sh);
    __shared__ float part[NW][MR][kGemvHalfCols];
    if (r == 0)
#pragma unroll
        for (int i = 0; i < MR; ++i)
#pragma unroll
            for (int c = 0; c < 8; ++c) part[wave][i][8 * q + c] = acc[i][c];
    __syncthreads();
    if (threadIdx.x < kGemvHalfCols * MR) {
        const int i = threadIdx.x / kGemvHalfCols, c = threadIdx.x % kGemvHalfCols;
        const int col = blockIdx.x * kGemvHalfCols + c;
        if (i < M && col < N) {
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) s += part[w][i][c];
            float out = p.alpha * s;
            const size_t ci = (size_t)i * p.ldc + col, di = (size_t)i * p.ldd + col;
            if (p.c != nullptr)
                out += p.beta * (p.cd_half ? to_float<BF16>(static_cast<const u16*>(p.c)[ci]) : static_cast<const float*>(p.c)[ci]);
            if (p.cd_half)
                static_cast<u16*>(p.d)[di] = from_float<BF16>(out);
            else
                static_cast<float*>(p.d)[di] = out;
        }
    }
}

template <bool BF16>
const void* pick(int m) {
    static_assert(kGemvHalfRows == 2, "one kernel per row count");
    if (m <= 1) return reinterpret_cast<const void*>(&gemv_pass_half<BF16, 8, 2, 1>);
    return reinterpret_cast<const void*>(&gemv_pass_half<BF16, 16, 2, 2>);
}

}  // namespace

const void* gemvHalfKernel(bool bf16, int m) { return bf16 ? pick<true>(m) : pick<false>(m); }

}  // namespace ftrain::gemm
