// FP32 deep-k kernel on v_mfma_f32_16x16x4_f32 for shapes with few output
// tiles and a long reduction (skinny m or n, deep k), with the split-k
// reduction done inside the same launch.  Device code only.
//
// Replaces the reference's SIMT kernel (src/primitive/hygon/gemm/
// fp32_gemm.hip:18-31) with the same formula: d = alpha*(a@b) + beta*c, the
// beta term dropped for a null c and always evaluated otherwise.
//
// Geometry: a 64 x 64 output tile per workgroup of 4 waves.  The waves split
// k, not the tile: the workgroup's k range is cut into slices of 32, wave w
// takes slices w, w+4, w+8, ... and accumulates the whole 64 x 64 tile (16
// blocks of 16 x 16, 64 accumulators per lane).  No wave shares operands
// with another, so the main loop has no LDS traffic and no barrier: each
// wave loads its MFMA operands straight from global memory into registers
// with 128-bit loads and refills each register with the next slice's data
// right after its last MFMA, so loads stream out evenly and every operand
// has a whole slice (128 MFMAs) of time to arrive.
//
// v_mfma_f32_16x16x4_f32, one block (16 x 16 output, k = 4):
//   A operand: lane l holds A[row = l % 16][k slot g = l / 16]
//   B operand: lane l holds B[k slot g][col = l % 16]
//   result   : lane l, register r holds D[row = 4*g + r][col = l % 16]
// Slice layout per lane (j16 = lane % 16, g = lane / 16, slice start k0):
//   a[bi][h] = A[16bi + j16][k0 + 8g + 4h .. +3]   (rows of a: full 128-byte
//              lines over the 4 lane groups)
//   b[s]     = B[k0 + 8g + s][4 j16 .. +3]          (256 contiguous bytes of
//              a row of b per lane group)
// At step s (0..7) k slot g is k0 + 8g + s.  Block bj's MFMA column j is
// tile column 4j + bj, so one 128-bit load of a b row gives a lane its
// operands for all four column blocks of a step.
//
// Split-k inside the launch.  The grid is tiles x splits workgroups; split
// z reduces k in [z*k_chunk, (z+1)*k_chunk).  Every workgroup sums its 4
// waves' tiles through LDS (wave order 0..3); with more than one split it
// then
//   1. stores its 64 x 64 partial to slot (z, tile) with agent-scope
//      coherent stores (each visible device-wide once complete),
//   2. waits for them to complete and increments the tile's arrival counter
//      (agent-scope atomic),
//   3. if it arrived last, reads every other split's partial with
//      agent-scope coherent loads, sums the partials in split order 0..S-1
//      (its own from registers), writes d = alpha*sum + beta*c and sets the
//      counter back to 0.
// No workgroup waits for another, so nothing depends on co-residency, and
// no cache writeback or invalidate is needed: every access that crosses
// workgroups is coherent at device scope by itself.  The summation order is
// fixed, so results are bit-identical from run to run whatever the arrival
// order.  Counters must be 0 when a launch starts; every launch leaves them
// 0.
#pragma once

#include <hip/hip_runtime.h>

#include "ft/gemm_kernels.hpp"

namespace ftrain::gemm::deepk {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned long long u64;

constexpr int BM = 64, BN = 64, KW = 32, NT = 256;
constexpr int SR = BN + 4;  // LDS row stride of the wave tiles in the epilogue

// Work item of hardware workgroup `bid`: with the total a multiple of 8,
// workgroup b runs on XCD b % 8, so XCD x is given the contiguous range
// [x*total/8, (x+1)*total/8) of (split, tile) pairs, split-major: the
// workgroups of one split, which read the same slice of the shared operand,
// share an L2.
__device__ __forceinline__ void work_of(int bid, int tiles, int total, int& tile, int& split) {
    int o = bid;
    if ((total & 7) == 0) o = (bid & 7) * (total >> 3) + (bid >> 3);
    split = o / tiles;
    tile  = o - split * tiles;
}

struct Slice {
    floatx4 a[4][2];
    floatx4 b[8];
};

__device__ __forceinline__ void deepk_gemm_body(const DeepKParams& P) {
    const GemmParams& p = P.g;
    const int tid  = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6, j16 = lane & 15, g = lane >> 4;
    const int tiles = p.tiles_m * p.tiles_n;
    int tile, split;
    work_of(blockIdx.x, tiles, tiles * P.splits, tile, split);
    const int tm = tile / p.tiles_n, tn = tile - tm * p.tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;
    const int M = p.m, N = p.n;
    const int kbeg = split * p.k_chunk;
    const int kend = min(p.k, kbeg + p.k_chunk);
    const size_t ldb = p.ldb;

    // Rows of a and columns of b past the matrix edge are read at a clamped
    // index (a 4-column run of b stays inside, n % 4 == 0): their products
    // only reach outputs the epilogue does not store.
    const float* arow[4];
#pragma unroll
    for (int bi = 0; bi < 4; ++bi) arow[bi] = p.a + (size_t)min(m0 + 16 * bi + j16, M - 1) * p.lda + 8 * g;
    const float* bcol = p.b + (size_t)(8 * g) * ldb + min(n0 + 4 * j16, N - 4);

    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    auto mfma_step = [&](const Slice& S, int s) {
#pragma unroll
        for (int bi = 0; bi < 4; ++bi)
#pragma unroll
            for (int bj = 0; bj < 4; ++bj)
                acc[bi][bj] = __builtin_amdgcn_mfma_f32_16x16x4f32(S.a[bi][s >> 2][s & 3], S.b[s][bj], acc[bi][bj], 0, 0, 0);
    };

    const int nfull = (kend - kbeg) / KW;  // whole slices; a partial one (the k tail) follows
    // Slice index past the last whole one: clamped (the loads re-read valid
    // memory and are never used).
    auto slice_k0 = [&](int sl) { return kbeg + min(sl, nfull - 1) * KW; };
    const int nw = nfull > wave ? (nfull - wave + 3) / 4 : 0;  // whole slices of this wave
    Slice R;
    if (nw > 0) {
        {
            const int k0 = slice_k0(wave);
#pragma unroll
            for (int bi = 0; bi < 4; ++bi)
#pragma unroll
                for (int h = 0; h < 2; ++h) R.a[bi][h] = *reinterpret_cast<const floatx4*>(arow[bi] + k0 + 4 * h);
#pragma unroll
            for (int s = 0; s < 8; ++s) R.b[s] = *reinterpret_cast<const floatx4*>(bcol + (size_t)(k0 + s) * ldb);
        }
        for (int i = 0; i < nw; ++i) {
            // Compute slice wave + 4i; refill each register with slice
            // wave + 4(i+1) after its last use: b[s] after step s, a[.][0]
            // after step 3, a[.][1] after step 7.
            const int k0 = slice_k0(wave + 4 * (i + 1));
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                mfma_step(R, s);
                R.b[s] = *reinterpret_cast<const floatx4*>(bcol + (size_t)(k0 + s) * ldb);
                if (s == 3 || s == 7) {
#pragma unroll
                    for (int bi = 0; bi < 4; ++bi)
                        R.a[bi][s >> 2] = *reinterpret_cast<const floatx4*>(arow[bi] + k0 + 4 * (s >> 2));
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);  // the step's MFMAs
                if (s == 3 || s == 7)
                    __builtin_amdgcn_sched_group_barrier(0x020, 5, 0);  // then its refills
                else
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
        }
    }
    // The k tail (fewer than KW values, zero-filled), by the wave whose turn
    // it is.  k % 4 == 0 and kend % 4 == 0, so a 4-run of a is all in or out.
    if (nfull * KW < kend - kbeg && wave == (nfull & 3)) {
        const int k0 = kbeg + nfull * KW;
#pragma unroll
        for (int bi = 0; bi < 4; ++bi)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                R.a[bi][h] = k0 + 8 * g + 4 * h < kend ? *reinterpret_cast<const floatx4*>(arow[bi] + k0 + 4 * h)
                                                       : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; ++s)
            R.b[s] = k0 + 8 * g + s < kend ? *reinterpret_cast<const floatx4*>(bcol + (size_t)(k0 + s) * ldb)
                                           : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 8; ++s) mfma_step(R, s);
    }

    // ---- the 4 waves' tiles summed through LDS in wave order ----
    __shared__ __attribute__((aligned(16))) float red[4 * BM * SR];
#pragma unroll
    for (int bi = 0; bi < 4; ++bi)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            *reinterpret_cast<floatx4*>(red + (wave * BM + bi * 16 + 4 * g + r) * SR + 4 * j16) =
                floatx4{acc[bi][0][r], acc[bi][1][r], acc[bi][2][r], acc[bi][3][r]};
    __syncthreads();
    // Thread t owns tile row t / 4, columns 16 (t % 4) .. +15.
    const int orow = tid >> 2, ocol = 16 * (tid & 3);
    floatx4 sum[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        sum[q] = *reinterpret_cast<const floatx4*>(red + orow * SR + ocol + 4 * q);
#pragma unroll
        for (int w = 1; w < 4; ++w) sum[q] += *reinterpret_cast<const floatx4*>(red + (w * BM + orow) * SR + ocol + 4 * q);
    }

    const int S = P.splits;
    if (S > 1) {
        // Slot (split, tile) holds 2048 64-bit words; word 256 q + t is
        // thread t's pair q (q = 0..7), so each store or load instruction of
        // a wave covers 512 contiguous bytes.
        u64* const slots          = reinterpret_cast<u64*>(P.partials);
        const size_t tile_words   = BM * BN / 2;
        const size_t split_stride = (size_t)tiles * tile_words;
        u64* const mine           = slots + split * split_stride + tile * tile_words + tid;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            __hip_atomic_store(mine + (2 * q) * NT, __builtin_bit_cast(u64, float2{sum[q][0], sum[q][1]}),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(mine + (2 * q + 1) * NT, __builtin_bit_cast(u64, float2{sum[q][2], sum[q][3]}),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // This thread's stores are complete (so visible device-wide) before
        // the barrier; the arrival is counted after every thread's are.
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __syncthreads();
        __shared__ unsigned int arrived;
        if (tid == 0)
            arrived = __hip_atomic_fetch_add(P.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (arrived != unsigned(S - 1)) return;
        // Last arrival: every other split's partial, 8 splits' loads in
        // flight at a time, summed in split order.
        const u64* const base = slots + tile * tile_words + tid;
        floatx4 total[4];
        for (int s0 = 0; s0 < S; s0 += 8) {
            floatx4 part[8][4];
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const int z = s0 + b;
                if (z >= S || z == split) continue;
                const u64* src = base + z * split_stride;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float2 lo = __builtin_bit_cast(
                        float2, __hip_atomic_load(src + (2 * q) * NT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
                    const float2 hi = __builtin_bit_cast(
                        float2, __hip_atomic_load(src + (2 * q + 1) * NT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
                    part[b][q] = floatx4{lo.x, lo.y, hi.x, hi.y};
                }
            }
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const int z = s0 + b;
                if (z >= S) break;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const floatx4 v = z == split ? sum[q] : part[b][q];
                    total[q] = z == 0 ? v : total[q] + v;
                }
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) sum[q] = total[q];
        if (tid == 0) __hip_atomic_store(P.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // d = alpha*sum + beta*c (n % 4 == 0: a run of 4 columns is all in or out).
    const int row = m0 + orow;
    if (row >= M) return;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int col = n0 + ocol + 4 * q;
        if (col >= N) continue;
        floatx4 out = p.alpha * sum[q];
        if (p.c != nullptr) out += p.beta * *reinterpret_cast<const floatx4*>(p.c + (size_t)row * p.ldc + col);
        *reinterpret_cast<floatx4*>(p.d + (size_t)row * p.ldd + col) = out;
    }
}

__global__ __launch_bounds__(NT, 1) void deepk_gemm(DeepKParams P) { deepk_gemm_body(P); }

// Sets n arrival counters to 0 (a caller's workspace starts with arbitrary
// contents).
__global__ __launch_bounds__(256) void deepk_clear_counters(unsigned int* counters, int n) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) counters[i] = 0u;
}

}  // namespace ftrain::gemm::deepk
