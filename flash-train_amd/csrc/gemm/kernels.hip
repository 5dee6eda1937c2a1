// FP32 GEMM kernels for MI355X (gfx950 / CDNA4): the row-major a and b
// instantiations of the MFMA tile kernel (gemm/mfma_tile.hpp) and the
// kernels that have no per-layout variants.
//
// Replaces the reference's single SIMT kernel
// (src/primitive/hygon/gemm/fp32_gemm.hip:18-51) with:
//   * MFMA tile kernels built on v_mfma_f32_32x32x2_f32 (gemm/mfma_tile.hpp),
//     whole-k or split over k into partial tiles;
//   * the deterministic split-k reduction;
//   * a streaming split-k kernel for skinny m (GEMV-like, HBM bound);
//   * a general SIMT kernel with 64-bit indexing and arbitrary strides for
//     shapes the others cannot take.
#include "mfma_tile.hpp"

namespace ftrain::gemm {

using namespace dev;

namespace {

// ----------------------------------------------------------------------------
// Skinny-m streaming kernel (m <= 8).  Each workgroup covers 256 columns and
// one k range; its 4 waves interleave over the k rows of that range, each
// lane streaming 4 adjacent columns of b.  The waves' partial sums meet in
// LDS and are stored raw to slice z of the workspace; splitk_reduce then
// forms d in a fixed order (deterministic).  Bound by the one pass over b.
// b is row-major (row stride ldb); a is row-major (TA false) or
// column-major (TA true) with leading dimension lda.
// ----------------------------------------------------------------------------

template <bool VEC, bool TA>
__device__ __forceinline__ void gemv_partial(const GemmParams& p, float* __restrict__ W) {
    const int tid  = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int M = p.m, N = p.n, K = p.k;
    const int col0 = blockIdx.x * kGemvCols + lane * 4;
    const int kbeg = blockIdx.z * p.k_chunk;
    const int kend = min(K, kbeg + p.k_chunk);
    const float* __restrict__ A = p.a;
    const float* __restrict__ B = p.b;

    float acc[kGemvRows][4];
#pragma unroll
    for (int i = 0; i < kGemvRows; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[i][c] = 0.f;

    auto step = [&](int k) {
        floatx4 bv = floatx4{0.f, 0.f, 0.f, 0.f};
        const float* brow = B + (size_t)k * p.ldb;
        if constexpr (VEC) {
            if (col0 < N) bv = *reinterpret_cast<const floatx4*>(brow + col0);
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (col0 + c < N) bv[c] = brow[col0 + c];
        }
#pragma unroll
        for (int i = 0; i < kGemvRows; ++i) {
            if (i < M) {
                const float av = TA ? A[(size_t)k * p.lda + i] : A[(size_t)i * p.lda + k];
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[i][c] += av * bv[c];
            }
        }
    };

    int k = kbeg + wave;
    for (; k + 12 < kend; k += 16) {
        step(k);
        step(k + 4);
        step(k + 8);
        step(k + 12);
    }
    for (; k < kend; k += 4) step(k);

    __shared__ float part[4][kGemvRows][kGemvCols + 4];
#pragma unroll
    for (int i = 0; i < kGemvRows; ++i)
        if (i < M)
#pragma unroll
            for (int c = 0; c < 4; ++c) part[wave][i][lane * 4 + c] = acc[i][c];
    __syncthreads();

    const int col = blockIdx.x * kGemvCols + tid;
    if (col < N) {
        for (int i = 0; i < M; ++i) {
            const float s = part[0][i][tid] + part[1][i][tid] + part[2][i][tid] + part[3][i][tid];
            W[(size_t)blockIdx.z * M * N + (size_t)i * N + col] = s;
        }
    }
}

// Partial slices only (p.d is the workspace); splitk_reduce forms d.
template <bool VEC, bool TA>
__global__ __launch_bounds__(256) void gemv_splitk(GemmParams p) {
    gemv_partial<VEC, TA>(p, p.d);
}

// ----------------------------------------------------------------------------
// One-pass skinny-m kernel (m <= MR <= 8, row-major b with 16-byte aligned
// rows, n % 4 == 0).  Workgroup x owns output columns [32x, 32x + 32) over
// all of k, so no partial sums leave it and d is written directly.  Lane
// (r = lane / 8, q = lane % 8) of wave w takes columns 4q .. 4q+3 and, per
// step, the 4 consecutive k rows 4*(8*(w + NW*j) + r) + t, t = 0..3: one
// 128-bit load of b per row (8 lanes cover a row's 128 bytes, a wave 8
// rows), and for a row-major a one 128-bit load of a's 4 values per row of
// a.  U steps are loaded before any is used, so each wave keeps U*4 KiB of
// b in flight.  Reduction, fixed order: a butterfly over the 8 lanes that
// share columns (lane bits 3..5), then the NW wave sums in wave order
// through LDS.  a row-major (TA false) needs k % 4 == 0 and lda % 4 == 0;
// column-major a is read per element.
// ----------------------------------------------------------------------------
template <int NW, int U, int MR, bool TA>
__global__ __launch_bounds__(NW * 64) void gemv_pass(GemmParams p) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane >> 3, q = lane & 7;
    const int M = p.m, N = p.n, K = p.k;
    // Columns past n (n % 4 == 0) and rows of a past m are read at a clamped
    // index instead of behind a branch, which splits every load into a block
    // of its own: they feed only sums the final store skips (the butterfly
    // combines lanes of the same columns).  Measured at 8192^2: one, two and
    // four rows 38.1 / 39.0 / 39.7 us against 42.9 / 42.9 / 42.4 with the
    // branches; eight rows (at 4096^2) keep them, 18.1 against 29.0 us.
    constexpr bool GUARDED      = MR >= 8;
    const int col               = blockIdx.x * kGemvPassCols + 4 * q;
    const bool col_ok           = col < N;
    const int col0              = GUARDED ? col : min(col, N - 4);
    const float* __restrict__ A   = p.a;
    const float* __restrict__ B   = p.b;
    const size_t lda = p.lda, ldb = p.ldb;
    constexpr int KSTEP = 32 * NW;  // k rows per step over the workgroup

    float acc[MR][4];
#pragma unroll
    for (int i = 0; i < MR; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[i][c] = 0.f;

    // b rows k0 .. k0+3 and a's values at those rows; rows >= K read as 0
    // (only a column-major a allows K % 4 != 0).
    auto load = [&](int k0, floatx4 (&bv)[4], floatx4 (&av)[MR], bool full) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            bv[t] = floatx4{0.f, 0.f, 0.f, 0.f};
            if ((!GUARDED || col_ok) && (full || k0 + t < K))
                bv[t] = *reinterpret_cast<const floatx4*>(B + (size_t)(k0 + t) * ldb + col0);
        }
#pragma unroll
        for (int i = 0; i < MR; ++i) {
            const int row = GUARDED ? i : min(i, M - 1);
            av[i] = floatx4{0.f, 0.f, 0.f, 0.f};
            if (GUARDED && i >= M) continue;
            if constexpr (!TA) {
                if (full || k0 < K) av[i] = *reinterpret_cast<const floatx4*>(A + (size_t)row * lda + k0);
            } else {
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    if (full || k0 + t < K) av[i][t] = A[(size_t)(k0 + t) * lda + row];
            }
        }
    };
    auto fma = [&](const floatx4 (&bv)[4], const floatx4 (&av)[MR]) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < MR; ++i)
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[i][c] += av[i][t] * bv[t][c];
    };

    int k = 4 * (8 * wave + r);
    for (; k + (U - 1) * KSTEP + 3 < K; k += U * KSTEP) {
        floatx4 bv[U][4], av[U][MR];
#pragma unroll
        for (int u = 0; u < U; ++u) load(k + u * KSTEP, bv[u], av[u], true);
#pragma unroll
        for (int u = 0; u < U; ++u) fma(bv[u], av[u]);
    }
    for (; k < K; k += KSTEP) {
        floatx4 bv[4], av[MR];
        load(k, bv, av, false);
        fma(bv, av);
    }

#pragma unroll
    for (int sh = 8; sh < 64; sh <<= 1)
#pragma unroll
        for (int i = 0; i < MR; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[i][c] += __shfl_xor(acc[i][c], sh);
    __shared__ float part[NW][MR][kGemvPassCols];
    if (r == 0)
#pragma unroll
        for (int i = 0; i < MR; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) part[wave][i][4 * q + c] = acc[i][c];
    __syncthreads();
    if (threadIdx.x < kGemvPassCols * MR) {
        const int i = threadIdx.x / kGemvPassCols, c = threadIdx.x % kGemvPassCols;
        const int col = blockIdx.x * kGemvPassCols + c;
        if (i < M && col < N) {
            float s = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) s += part[w][i][c];
            p.d[(size_t)i * p.ldd + col] = p.alpha * s + (p.c != nullptr ? p.beta * p.c[(size_t)i * p.ldc + col] : 0.f);
        }
    }
}

// ----------------------------------------------------------------------------
// Split-k reduction: d = alpha * sum_{z < splits} W[z] + (c ? beta*c : 0) in a
// fixed summation order (deterministic).  The slices are dense m x n fp32; c
// and d are row-major with row strides ldc and ldd, in fp32 or a 16-bit type
// (cd_type).  VEC: units of four adjacent elements (fp32 c and d; n, ldc, ldd
// multiples of 4; 16-byte aligned c, d, W).
// ----------------------------------------------------------------------------
__device__ __forceinline__ float load_cd(const void* p, uint64_t i, int32_t type) {
    if (type == kCdFp32) return static_cast<const float*>(p)[i];
    const unsigned short v = static_cast<const unsigned short*>(p)[i];
    if (type == kCdBf16) return __builtin_bit_cast(float, static_cast<unsigned int>(v) << 16);
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
}

__device__ __forceinline__ void store_cd(void* p, uint64_t i, int32_t type, float x) {
    // Half types round to nearest even (the compiler's conversions).
    if (type == kCdFp32)
        static_cast<float*>(p)[i] = x;
    else if (type == kCdBf16)
        static_cast<unsigned short*>(p)[i] = __builtin_bit_cast(unsigned short, static_cast<__bf16>(x));
    else
        static_cast<unsigned short*>(p)[i] = __builtin_bit_cast(unsigned short, static_cast<_Float16>(x));
}

template <bool VEC>
__global__ __launch_bounds__(256) void splitk_reduce(ReduceParams p) {
    // Each block reduces E output units (VEC: 4 adjacent elements) over the
    // splits with G threads per unit: thread group g sums slices z = g, g+G,
    // ... in increasing z, then one thread adds the G group sums in
    // increasing g.  The order is fixed, so results are deterministic, and
    // the G independent load streams per unit keep enough bytes in flight
    // for deep splits.
    constexpr int G = 16;
    constexpr int E = 256 / G;
    using V         = std::conditional_t<VEC, floatx4, float>;
    __shared__ V part[G][E];
    const int e          = threadIdx.x % E;
    const int g          = threadIdx.x / E;
    const uint64_t units = VEC ? p.count / 4 : p.count;
    const V* __restrict__ W = reinterpret_cast<const V*>(p.partials);
    const int groups        = min(G, p.splits);
    for (uint64_t base = (uint64_t)blockIdx.x * E; base < units; base += (uint64_t)gridDim.x * E) {
        const uint64_t i = base + e;
        if (i < units && g < groups) {
            V s = W[(uint64_t)g * units + i];
#pragma unroll 4
            for (int z = g + G; z < p.splits; z += G) s += W[(uint64_t)z * units + i];
            part[g][e] = s;
        }
        __syncthreads();
        if (g == 0 && i < units) {
            V s = part[0][e];
            for (int q = 1; q < groups; ++q) s += part[q][e];
            if constexpr (VEC) {
                // fp32 c and d, n % 4 == 0.
                const uint64_t row_vecs = p.n / 4;
                const uint64_t r = i / row_vecs, c = 4 * (i - r * row_vecs);
                const float* C = static_cast<const float*>(p.c);
                float* D       = static_cast<float*>(p.d);
                floatx4 out;
                if (C != nullptr) {
                    const floatx4 cv = *reinterpret_cast<const floatx4*>(C + r * p.ldc + c);
#pragma unroll
                    for (int j = 0; j < 4; ++j) out[j] = p.alpha * s[j] + p.beta * cv[j];
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) out[j] = p.alpha * s[j] + 0.f;
                }
                *reinterpret_cast<floatx4*>(D + r * p.ldd + c) = out;
            } else {
                const uint64_t r = i / p.n, c = i - r * p.n;
                const float out = p.alpha * s + (p.c != nullptr ? p.beta * load_cd(p.c, r * p.ldc + c, p.cd_type) : 0.f);
                store_cd(p.d, r * p.ldd + c, p.cd_type, out);
            }
        }
        __syncthreads();
    }
}

// The same reduction with one thread per output unit, summing the slices in
// increasing z: for outputs with enough units to fill the chip on their own
// (the 16-thread form leaves 15 of 16 threads idle at two splits).
template <bool VEC>
__global__ __launch_bounds__(256) void splitk_reduce_wide(ReduceParams p) {
    using V               = std::conditional_t<VEC, floatx4, float>;
    const uint64_t units  = VEC ? p.count / 4 : p.count;
    const V* __restrict__ W = reinterpret_cast<const V*>(p.partials);
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < units; i += (uint64_t)gridDim.x * 256) {
        // Up to 8 slices' loads in flight before their adds (in increasing z): the pass is
        // latency-bound, a load per add kept one or two in flight.
        V s = W[i];
        for (int z = 1; z < p.splits; z += 8) {
            V v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (z + j < p.splits) v[j] = W[(uint64_t)(z + j) * units + i];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (z + j < p.splits) s += v[j];
        }
        if constexpr (VEC) {
            const uint64_t row_vecs = p.n / 4;
            const uint64_t r = i / row_vecs, c = 4 * (i - r * row_vecs);
            const float* C = static_cast<const float*>(p.c);
            floatx4 out;
            if (C != nullptr) {
                const floatx4 cv = *reinterpret_cast<const floatx4*>(C + r * p.ldc + c);
#pragma unroll
                for (int j = 0; j < 4; ++j) out[j] = p.alpha * s[j] + p.beta * cv[j];
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) out[j] = p.alpha * s[j] + 0.f;
            }
            *reinterpret_cast<floatx4*>(static_cast<float*>(p.d) + r * p.ldd + c) = out;
        } else {
            const uint64_t r = i / p.n, c = i - r * p.n;
            const float out = p.alpha * s + (p.c != nullptr ? p.beta * load_cd(p.c, r * p.ldc + c, p.cd_type) : 0.f);
            store_cd(p.d, r * p.ldd + c, p.cd_type, out);
        }
    }
}

// ----------------------------------------------------------------------------
// General SIMT kernel: 64x64 tiles, 4x4 outputs per thread, 64-bit indices,
// grid-stride over tiles.  Any shape, 4-byte alignment, any element strides
// for a and b, row strides for c and d.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void simt_gemm(WideParams p) {
    constexpr int T = 64, BK = 16;
    __shared__ float As[BK][T + 4];
    __shared__ float Bs[BK][T + 4];
    const int tid = threadIdx.x;
    const int tx = tid % 16, ty = tid / 16;
    const uint64_t M = p.m, N = p.n, K = p.k;
    const uint64_t tiles_n = (N + T - 1) / T;
    const uint64_t tiles   = ((M + T - 1) / T) * tiles_n;
    for (uint64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
        const uint64_t m0 = (t / tiles_n) * T;
        const uint64_t n0 = (t % tiles_n) * T;
        float acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
        for (uint64_t k0 = 0; k0 < K; k0 += BK) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int idx = tid + j * 256;
                const int r = idx / BK, kk = idx % BK;
                const uint64_t gm = m0 + r, gk = k0 + kk;
                As[kk][r] = (gm < M && gk < K) ? p.a[gm * p.a_rs + gk * p.a_cs] : 0.f;
                const int rb = idx / T, cb = idx % T;
                const uint64_t bk = k0 + rb, bn = n0 + cb;
                Bs[rb][cb] = (bk < K && bn < N) ? p.b[bk * p.b_rs + bn * p.b_cs] : 0.f;
            }
            __syncthreads();
#pragma unroll
            for (int kk = 0; kk < BK; ++kk) {
                float av[4], bv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) av[i] = As[kk][ty * 4 + i];
#pragma unroll
                for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx * 4 + j];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] += av[i] * bv[j];
            }
            __syncthreads();
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint64_t row = m0 + ty * 4 + i;
            if (row >= M) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint64_t c = n0 + tx * 4 + j;
                if (c >= N) continue;
                p.d[row * p.ldd + c] =
                    p.alpha * acc[i][j] + (p.c != nullptr ? p.beta * p.c[row * p.ldc + c] : 0.f);
            }
        }
    }
}


}  // namespace

// Waves and steps in flight per row count, measured at n = k = 8192 (fp32):
// one row 8 waves x 2 steps (37.8 us), two and four rows 16 x 2 (38.9 /
// 38.8), eight rows 8 x 2 (the configurations with more in flight, 8 x 4
// and 16 x 2, spill registers there).  The 16-bit kernel uses the same.
int gemvPassThreads(int m) { return m <= 1 || m > 4 ? 512 : 1024; }

const void* gemvKernel(Variant v, int m, bool ta, int& threads) {
    threads = gemvPassThreads(m);
    if (v == Variant::kBf16Gemv || v == Variant::kFp16Gemv) return ta ? nullptr : gemvHalfKernel(v == Variant::kBf16Gemv, m);
    if (m <= 1) return ta ? reinterpret_cast<const void*>(&gemv_pass<8, 2, 1, true>) : reinterpret_cast<const void*>(&gemv_pass<8, 2, 1, false>);
    if (m <= 2) return ta ? reinterpret_cast<const void*>(&gemv_pass<16, 2, 2, true>) : reinterpret_cast<const void*>(&gemv_pass<16, 2, 2, false>);
    if (m <= 4) return ta ? reinterpret_cast<const void*>(&gemv_pass<16, 2, 4, true>) : reinterpret_cast<const void*>(&gemv_pass<16, 2, 4, false>);
    return ta ? reinterpret_cast<const void*>(&gemv_pass<8, 2, 8, true>) : reinterpret_cast<const void*>(&gemv_pass<8, 2, 8, false>);
}

const void* kernelFor(Variant v, bool ta, bool tb, bool prefetch_b) {
    if (info(v).gemv && info(v).split == SplitKind::kNone) {
        if (tb) return nullptr;
        int threads = 0;
        return gemvKernel(v, kGemvRows, ta, threads);
    }
    if (v >= Variant::kMfma16_256x256 && v <= Variant::kMfma16_256x64S) {
        using Fn                     = const void* (*)(int);
        static constexpr Fn table[4] = {mfma16KernelNN, mfma16KernelTN, mfma16KernelNT, mfma16KernelTT};
        return table[(ta ? 1 : 0) + (tb ? 2 : 0)](static_cast<int>(v) - static_cast<int>(Variant::kMfma16_256x256));
    }
    if (v >= Variant::kBf16Mfma256x256 && v <= Variant::kFp16Mfma64x64U) {
        const int i    = static_cast<int>(v) - static_cast<int>(Variant::kBf16Mfma256x256);
        const int tile = i % kHalfTiles;
        using Fn       = const void* (*)(int);
        static constexpr Fn table[2][4] = {
            {halfKernelBf16NN, halfKernelBf16TN, halfKernelBf16NT, halfKernelBf16TT},
            {halfKernelFp16NN, halfKernelFp16TN, halfKernelFp16NT, halfKernelFp16TT}};
        return table[i / kHalfTiles][(ta ? 1 : 0) + (tb ? 2 : 0)](tile);
    }
    if (v >= Variant::kMfma16Dma256x256 && v <= Variant::kMfma16Dma128x64) return ta ? dma32KernelTA(v, tb) : tb ? dma32KernelTB(v) : dma32Kernel(v);
    if (v == Variant::kBf16MfmaDma256x256) return dmaKernelBf16(ta, tb, prefetch_b);
    if (v == Variant::kFp16MfmaDma256x256) return dmaKernelFp16(ta, tb, prefetch_b);
    if (v == Variant::kBf16MfmaDma128x128 || v == Variant::kBf16MfmaDma128x128S)
        return dma128KernelBf16(ta, tb, v == Variant::kBf16MfmaDma128x128S);
    if (v == Variant::kFp16MfmaDma128x128 || v == Variant::kFp16MfmaDma128x128S)
        return dma128KernelFp16(ta, tb, v == Variant::kFp16MfmaDma128x128S);
    if (v == Variant::kBf16MfmaDma64x128S) return dma64x128KernelBf16(ta, tb);
    if (v == Variant::kFp16MfmaDma64x128S) return dma64x128KernelFp16(ta, tb);
    if (ta || tb) {
        if (v == Variant::kSimt) return reinterpret_cast<const void*>(&simt_gemm);  // strides are runtime values
        if (v == Variant::kGemvS && !tb && ta) return reinterpret_cast<const void*>(&gemv_splitk<true, true>);
        if (v == Variant::kGemvUS && !tb && ta) return reinterpret_cast<const void*>(&gemv_splitk<false, true>);
        if (!info(v).layouts) return nullptr;
        return ta ? (tb ? layoutKernelTT(v) : layoutKernelTN(v)) : layoutKernelNT(v);
    }
    switch (v) {
        case Variant::kMfma256x256: return reinterpret_cast<const void*>(&mfma_gemm<256, 256, 16, 2, 2, 3, 1, true, kWhole, false, false>);
        case Variant::kMfma256x256S: return reinterpret_cast<const void*>(&mfma_gemm<256, 256, 16, 2, 2, 3, 1, true, kPartial, false, false>);
        case Variant::kMfma256x128: return reinterpret_cast<const void*>(&mfma_gemm<256, 128, 16, 2, 2, 2, 2, true, kWhole, false, false>);
        case Variant::kMfma64x256: return reinterpret_cast<const void*>(&mfma_gemm<64, 256, 16, 1, 4, 3, 1, true, kWhole, false, false>);
        case Variant::kMfma64x256S: return reinterpret_cast<const void*>(&mfma_gemm<64, 256, 16, 1, 4, 3, 1, true, kPartial, false, false>);
        case Variant::kMfma256x64: return reinterpret_cast<const void*>(&mfma_gemm<256, 64, 16, 4, 1, 3, 1, true, kWhole, false, false>);
        case Variant::kMfma256x64S: return reinterpret_cast<const void*>(&mfma_gemm<256, 64, 16, 4, 1, 3, 1, true, kPartial, false, false>);
        case Variant::kGemvS: return reinterpret_cast<const void*>(&gemv_splitk<true, false>);
        case Variant::kGemvUS: return reinterpret_cast<const void*>(&gemv_splitk<false, false>);
        case Variant::kSimt: return reinterpret_cast<const void*>(&simt_gemm);
        case Variant::kDeepK64x64: return deepkKernel();
        default: return layoutKernel<false, false>(v);
    }
}

const void* groupedKernelNN(int which) { return groupedLayoutKernel<false, false>(which); }

const void* groupedKernelFor(FTrainNumericType input, int which, bool ta, bool tb, bool prefetch_b) {
    using Fn                        = const void* (*)(int);
    static constexpr Fn table[3][4] = {
        {groupedKernelNN, groupedKernelTN, groupedKernelNT, groupedKernelTT},
        {groupedHalfKernelBf16NN, groupedHalfKernelBf16TN, groupedHalfKernelBf16NT, groupedHalfKernelBf16TT},
        {groupedHalfKernelFp16NN, groupedHalfKernelFp16TN, groupedHalfKernelFp16NT, groupedHalfKernelFp16TT}};
    const int t = input == FTRAIN_NUMERIC_TYPE_FP32 ? 0 : input == FTRAIN_NUMERIC_TYPE_BF16 ? 1 : 2;
    const int o = (ta ? 1 : 0) + (tb ? 2 : 0);
    if (t != 0 && which == 3)
        return t == 1 ? groupedDmaKernelBf16(ta, tb, prefetch_b) : groupedDmaKernelFp16(ta, tb, prefetch_b);
    if (t != 0 && which == 4) return t == 1 ? groupedDma128KernelBf16(ta, tb) : groupedDma128KernelFp16(ta, tb);
    if (t == 0 && which == 4) return ta || tb ? nullptr : groupedDma32Kernel();
    if (t == 0 && which == 5) return groupedDma32Kernel128(ta, tb);
    if (t == 0 && which == 6) return ta ? nullptr : groupedDma32Kernel64x128(tb);
    if (t == 0 && (which == 2 || which == 3)) {
        // The fp32 256x128 / 128x256 tiles of the 16x16x4 family (grouped entries 16 and 17).
        static constexpr Fn m16[4] = {mfma16KernelNN, mfma16KernelTN, mfma16KernelNT, mfma16KernelTT};
        return m16[o](which + 14);
    }
    return table[t][o](which);
}

const void* reduceKernel(bool vec, bool wide) {
    if (wide)
        return vec ? reinterpret_cast<const void*>(&splitk_reduce_wide<true>)
                   : reinterpret_cast<const void*>(&splitk_reduce_wide<false>);
    return vec ? reinterpret_cast<const void*>(&splitk_reduce<true>) : reinterpret_cast<const void*>(&splitk_reduce<false>);
}

}  // namespace ftrain::gemm
