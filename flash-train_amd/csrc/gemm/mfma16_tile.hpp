// FP32 MFMA tile kernel on v_mfma_f32_16x16x4_f32 for large shapes, shared
// by the per-layout HIP translation units.  Device code only.
//
// Replaces the reference's SIMT kernel (src/primitive/hygon/gemm/
// fp32_gemm.hip:18-31) with the same formula: d = alpha*(a@b) + beta*c, the
// beta term dropped for a null c and always evaluated otherwise.
//
// Geometry: a 256 x 256 output tile per workgroup of 4 waves (one per
// SIMD), each wave a 128 x 128 sub-tile of 16 x 16 MFMA blocks (8 x 8
// blocks, 256 fp32 accumulators per lane, held in the accumulation
// registers).  A stage (BK = 16) is 256 MFMAs per wave, so the one barrier
// per stage is amortised over ~8k cycles.  With 8192^3 that is 1024 tiles,
// exactly four rounds over 256 CUs, and every A/B element fetched from L2
// feeds 256 outputs.  Measured on MI355X: 88% MFMA busy at 8192^3.
//
// v_mfma_f32_16x16x4_f32, one block (16 x 16 output, k = 4):
//   A operand: lane l holds A[row = l % 16][k slot g = l / 16]
//   B operand: lane l holds B[k slot g][col = l % 16]
//   result   : lane l, register r holds D[row = 4*g + r][col = l % 16]
// Lane group g takes k = g*KS + s at step s (KS = BK/4 steps per stage), so
// over one stage a lane's A values are KS consecutive k: one 128-bit LDS
// read per row block.  Column interleave in groups of four blocks: block
// bj, MFMA column j maps to wave-tile column (bj/4)*64 + 4*j + bj%4, so a
// lane owns TN/4 runs of 4 adjacent columns.  The B operands of all TN
// blocks of one step are then TN/4 128-bit LDS reads that the 16 lanes of a
// group take from one contiguous 256-byte span (conflict free), and each
// 128-bit store of the epilogue covers 256 contiguous bytes of a d row.
//
// Operand layouts (TA, TB) and their LDS staging are those of mfma_tile.hpp:
// each tile is stored with its memory-contiguous dimension innermost so
// 128-bit global loads become 128-bit LDS writes; a column-major A tile is
// then read one k per 32-bit read, a column-major B tile one column's KS
// consecutive k per 128-bit read.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "ft/gemm_kernels.hpp"

namespace ftrain::gemm::m16 {

typedef float floatx4 __attribute__((ext_vector_type(4)));

enum SplitMode : int { kWhole = 0, kPartial = 2 };

// XCD-aware tile order (see mfma_tile.hpp): each XCD gets a contiguous range
// of tiles, walked in column sweeps over bands of kBand tile rows.  Measured
// at 8192^3 (FETCH_SIZE per launch): bands of 4 rows fetch 5.3 GB for the
// 256x128 tile and 3.2 GB for the 256x256 tile, against 12.3 GB and 3.5 GB
// with bands of 8, at the same speed.
template <int kBand>
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int tiles = tiles_m * tiles_n;
    const int per   = tiles >> 3;
    int t           = bid;
    if (bid < (per << 3)) t = (bid & 7) * per + (bid >> 3);
    const int band_span = kBand * tiles_n;
    const int band      = t / band_span;
    const int first_m   = band * kBand;
    const int band_rows = min(tiles_m - first_m, kBand);
    const int within    = t - band * band_span;
    tm                  = first_m + within % band_rows;
    tn                  = within / band_rows;
}

// MINB workgroups per CU bound the registers; SIMPLE selects the plain
// stage loop (operands read after the barrier, then the stage's MFMAs, then
// the next stage's LDS writes and global loads), for tiles that run two
// workgroups per CU: the other workgroup's MFMAs cover this one's reads and
// barrier, and the single operand set fits the halved register budget.
template <int BM, int BN, int BK, int WM, int WN, int SPLIT, bool TA, bool TB, int MINB = 1, bool SIMPLE = false,
          int BAND = 4>
__device__ __forceinline__ void mfma16_gemm_tile(const GemmParams& p, int bid, int z) {
    constexpr int NT  = WM * WN * 64;
    constexpr int WTM = BM / WM;
    constexpr int WTN = BN / WN;
    constexpr int TM  = WTM / 16;
    constexpr int TN  = WTN / 16;
    constexpr int KS  = BK / 4;  // k-steps per stage
    // LDS row strides (floats).  A 128-bit LDS read is conflict-free when each
    // half-wave's 32 lanes cover 128 distinct banks; a 128-bit write when each
    // 8 consecutive lanes cover 32 (measured on MI355X with SQ_LDS_BANK_CONFLICT).
    // Row-major A: a half-wave reads 16 rows at two 4-float k offsets, so
    // rows 24 floats apart land on 16 distinct 8-bank slots.  Row-major B: a
    // half-wave reads two k rows 4 apart, which BN + 16 places 64 banks apart.
    constexpr int A_LD = BM * BK / 4 / NT;
    constexpr int B_LD = BK * BN / 4 / NT;
    // Column-major A with four staging vectors per thread (BK = 16): a
    // thread loads 4 consecutive k of one 4-row run, which transposes in
    // registers (fp32 elements are whole registers) into the k-contiguous
    // layout of a row-major A, read with the same 128-bit operand reads.
    // Other column-major tiles, and the split-k ones (whose registers the
    // transpose overflows), store A k-major and read one k per read.
    constexpr bool TAX = TA && A_LD == 4 && BK == 16 && SPLIT == kWhole;
    constexpr bool A_KMAJ = TA && !TAX;
    constexpr int SA  = A_KMAJ ? BM + 4 : BK + 8;
    constexpr int SB  = TB ? BK + 4 : BN + 16;
    constexpr int A_ELEMS = A_KMAJ ? BK * SA : BM * SA;
    constexpr int B_ELEMS = TB ? BN * SB : BK * SB;
    static_assert(TN % 4 == 0 && KS % 4 == 0, "128-bit operand reads");
    static_assert(A_LD >= 1 && B_LD >= 1 && BM * BK / 4 % NT == 0 && BK * BN / 4 % NT == 0, "staging");

    __shared__ __attribute__((aligned(16))) float As[2][A_ELEMS];
    __shared__ __attribute__((aligned(16))) float Bs[2][B_ELEMS];

    const int tid  = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int j16  = lane & 15;
    const int g    = lane >> 4;
    const int wrow = (wave / WN) * WTM;
    const int wcol = (wave % WN) * WTN;

    int tm, tn;
    tile_of<BAND>(bid, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int M = p.m, N = p.n, K = p.k;
    const int kbeg = SPLIT != kWhole ? z * p.k_chunk : 0;
    const int kend = SPLIT != kWhole ? min(K, kbeg + p.k_chunk) : K;
    const int nst  = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

    const float* __restrict__ A = p.a;
    const float* __restrict__ B = p.b;
    const size_t lda = p.lda, ldb = p.ldb;

    // Staging slot j of this thread: tile-local coordinates, consecutive
    // threads along each matrix's contiguous dimension.
    auto a_coord = [&](int j, int& r, int& k) {
        const int idx = tid + j * NT;
        if constexpr (TAX) {
            // Slot j: k = 4*(tid % 4) + j of rows 4*(tid / 4) .. +3.  The 8
            // lanes of one LDS write group then cover 2 row runs x 4 k
            // quarters: after the transpose each write hits 128 distinct
            // bytes (rows 4 apart, SA = 24: 384 bytes; k quarters 16 bytes).
            r = 4 * (tid >> 2);
            k = 4 * (tid & 3) + j;
        } else if constexpr (TA) {
            r = 4 * (idx % (BM / 4));
            k = idx / (BM / 4);
        } else {
            // Four threads per row of BK = 16.  Within each group of 16 rows
            // the even rows go to the first half-wave and the odd rows to the
            // second, so the 8 lanes of one write group cover rows 2 apart
            // (48 floats: disjoint 32-bank sets at stride 24).
            static_assert(BK == 16 && NT % 64 == 0, "row permutation assumes BK = 16");
            const int q = idx >> 2;  // consecutive row slot
            r = (q & ~15) | ((q & 7) << 1) | ((q >> 3) & 1);
            k = 4 * (idx & 3);
        }
    };
    auto b_coord = [&](int j, int& k, int& c) {
        const int idx = tid + j * NT;
        if constexpr (TB) {
            k = 4 * (idx % (BK / 4));
            c = idx / (BK / 4);
        } else {
            k = idx / (BN / 4);
            c = 4 * (idx % (BN / 4));
        }
    };
    auto a_lds = [&](int r, int k) { return A_KMAJ ? k * SA + r : r * SA + k; };
    auto b_lds = [&](int k, int c) { return TB ? c * SB + k : k * SB + c; };

    floatx4 ra[A_LD], rb[B_LD];
    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Stages [k_lo, k_lo + n_st * BK), the last one cut at kend.
    auto main_loop = [&](auto checked_tag, const int k_lo, const int n_st) {
        constexpr bool CHECKED = decltype(checked_tag)::value;
        // m / n index of a load.  The unchecked loop clamps it into the matrix
        // (a vector of `run` elements stays inside): an edge tile then reads
        // valid memory for rows and columns past the edge, whose products
        // land only in outputs the epilogue does not store.  Only a k tail
        // needs the zero-filling checked loop.
        auto row_at = [](int i, int extent, int run) { return CHECKED ? i : min(i, extent - run); };
        auto a_at = [&](int gm, int gk) { return A + (TA ? (size_t)gk * lda + gm : (size_t)gm * lda + gk); };
        auto b_at = [&](int gk, int gn) { return B + (TB ? (size_t)gn * ldb + gk : (size_t)gk * ldb + gn); };

        auto load_stage = [&](int k0) {
#pragma unroll
            for (int j = 0; j < A_LD; ++j) {
                int r, k;
                a_coord(j, r, k);
                const int gm = row_at(m0 + r, M, TA ? 4 : 1), gk = k0 + k;
                ra[j] = floatx4{0.f, 0.f, 0.f, 0.f};
                if (!CHECKED || (gm < M && gk < kend)) ra[j] = *reinterpret_cast<const floatx4*>(a_at(gm, gk));
            }
#pragma unroll
            for (int j = 0; j < B_LD; ++j) {
                int k, c;
                b_coord(j, k, c);
                const int gk = k0 + k, gn = row_at(n0 + c, N, TB ? 1 : 4);
                rb[j] = floatx4{0.f, 0.f, 0.f, 0.f};
                if (!CHECKED || (gk < kend && gn < N)) rb[j] = *reinterpret_cast<const floatx4*>(b_at(gk, gn));
            }
        };
        auto store_stage = [&](int buf) {
            if constexpr (TAX) {
                // ra[j] holds rows r .. r+3 at k = k0 + j: row r + i gets
                // k0 .. k0+3 from element i of each.
                int r, k0;
                a_coord(0, r, k0);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    *reinterpret_cast<floatx4*>(&As[buf][(r + i) * SA + k0]) = floatx4{ra[0][i], ra[1][i], ra[2][i], ra[3][i]};
            } else {
#pragma unroll
                for (int j = 0; j < A_LD; ++j) {
                    int r, k;
                    a_coord(j, r, k);
                    *reinterpret_cast<floatx4*>(&As[buf][a_lds(r, k)]) = ra[j];
                }
            }
#pragma unroll
            for (int j = 0; j < B_LD; ++j) {
                int k, c;
                b_coord(j, k, c);
                *reinterpret_cast<floatx4*>(&Bs[buf][b_lds(k, c)]) = rb[j];
            }
        };

        // A operands of a whole stage: av[bi][q] holds k = g*KS + 4q .. +3.
        auto read_a = [&](int buf, floatx4 (&av)[TM][KS / 4]) {
#pragma unroll
            for (int bi = 0; bi < TM; ++bi) {
                const int r = wrow + bi * 16 + j16;
#pragma unroll
                for (int q = 0; q < KS / 4; ++q) {
                    if constexpr (A_KMAJ) {
#pragma unroll
                        for (int t = 0; t < 4; ++t) av[bi][q][t] = As[buf][(g * KS + 4 * q + t) * SA + r];
                    } else {
                        av[bi][q] = *reinterpret_cast<const floatx4*>(&As[buf][r * SA + g * KS + 4 * q]);
                    }
                }
            }
        };
        // B operands of the whole stage: bv[s][bj] for k = g*KS + s and
        // column (bj/4)*64 + 4*j16 + bj%4.
        auto read_b = [&](int buf, float (&bv)[KS][TN]) {
            if constexpr (TB) {
                // Column-major tile: one column's KS consecutive k per read.
#pragma unroll
                for (int bj = 0; bj < TN; ++bj)
#pragma unroll
                    for (int q = 0; q < KS / 4; ++q) {
                        const int c = wcol + (bj / 4) * 64 + 4 * j16 + bj % 4;
                        const floatx4 v = *reinterpret_cast<const floatx4*>(&Bs[buf][c * SB + g * KS + 4 * q]);
#pragma unroll
                        for (int t = 0; t < 4; ++t) bv[4 * q + t][bj] = v[t];
                    }
            } else {
#pragma unroll
                for (int s = 0; s < KS; ++s)
#pragma unroll
                    for (int q = 0; q < TN / 4; ++q) {
                        const floatx4 v =
                            *reinterpret_cast<const floatx4*>(&Bs[buf][(g * KS + s) * SB + wcol + 64 * q + 4 * j16]);
#pragma unroll
                        for (int t = 0; t < 4; ++t) bv[s][4 * q + t] = v[t];
                    }
            }
        };

        auto mfmas = [&](const floatx4 (&av)[TM][KS / 4], const float (&bv)[KS][TN], int first, int last) {
#pragma unroll
            for (int i = 0; i < KS * TM * TN; ++i) {
                if (i < first || i >= last) continue;
                const int s = i / (TM * TN), bi = (i / TN) % TM, bj = i % TN;
                acc[bi][bj] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[bi][s / 4][s % 4], bv[s][bj], acc[bi][bj], 0, 0, 0);
            }
        };

        // Software pipeline over two LDS buffers and two operand register
        // sets.  Iteration st holds stage st's operands in registers (read
        // at the end of the previous iteration) and the global data of
        // stage st+1 in the staging registers:
        //   1. the first MFMAs of stage st run while stage st+1 is written to
        //      the other LDS buffer and stage st+2's global loads are issued;
        //   2. barrier (stage st+1 visible; its buffer's previous contents,
        //      stage st-1, were read before the previous barrier);
        //   3. stage st+1's operands are read into the other register set
        //      under the remaining MFMAs of stage st.
        // sched_barrier(0) keeps each phase where it is written.  Past the
        // last stage the loads re-read the final stage and the extra LDS
        // writes land in a buffer nobody reads again.
        constexpr int NM    = KS * TM * TN;
        // MFMAs before the barrier; the rest cover the next stage's operand
        // reads.  Measured on the 256x256 tile at 8192^3: 7/8 of the stage
        // 142.0 TFLOP/s, 1/2 141.5, 1/4 140.8.  A column-major A keeps 1/2:
        // with 7/8 its k-major reads spill registers, and its transposed
        // staging runs at 120 TFLOP/s against 139 with 1/2.
        constexpr int FIRST = TA ? NM / 2 : NM * 7 / 8;
        floatx4 av[2][TM][KS / 4];
        float bv[2][KS][TN];
        auto clamp_k0 = [&](int stage) { return k_lo + min(stage, n_st - 1) * BK; };
        if (n_st > 0) {
            load_stage(k_lo);
            store_stage(0);
            load_stage(clamp_k0(1));
        }
        __syncthreads();
        if (n_st > 0) {
            read_a(0, av[0]);
            read_b(0, bv[0]);
        }
        auto iteration = [&](int st, const floatx4 (&ac)[TM][KS / 4], const float (&bc)[KS][TN],
                             floatx4 (&an)[TM][KS / 4], float (&bn)[KS][TN]) {
            const int nxt = (st + 1) & 1;
            store_stage(nxt);
            load_stage(clamp_k0(st + 2));
            mfmas(ac, bc, 0, FIRST);
            constexpr int MEM = A_LD + B_LD;  // LDS writes, then global loads, spread over the MFMAs
#pragma unroll
            for (int i = 0; i < MEM; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, FIRST / (2 * MEM), 0);
                __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, FIRST / (2 * MEM), 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
            read_a(nxt, an);
            read_b(nxt, bn);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(ac, bc, FIRST, NM);
            __builtin_amdgcn_sched_barrier(0);
        };
        if constexpr (SIMPLE) {
            for (int st = 0; st < n_st; ++st) {
                read_a(st & 1, av[0]);
                read_b(st & 1, bv[0]);
                mfmas(av[0], bv[0], 0, NM);
                store_stage((st + 1) & 1);
                load_stage(clamp_k0(st + 2));
                __syncthreads();
            }
        } else {
            for (int st = 0; st < n_st; ++st) {
                iteration(st, av[0], bv[0], av[1], bv[1]);
                // Rotate the register sets by copying (the allocator coalesces
                // the copies; swapping references across an unrolled pair made
                // it keep both sets live in separate registers and spill).
    #pragma unroll
                for (int i = 0; i < TM; ++i)
    #pragma unroll
                    for (int q = 0; q < KS / 4; ++q) av[0][i][q] = av[1][i][q];
    #pragma unroll
                for (int i = 0; i < KS; ++i)
    #pragma unroll
                    for (int j = 0; j < TN; ++j) bv[0][i][j] = bv[1][i][j];
            }
        }
    };

    // A k tail: the whole stages run the unchecked loop and the last, partial one a checked pass of
    // its own (zeros past kend) instead of checking every stage.  The split-k tiles keep one
    // checked loop (a second loop copy made the 256x256 one spill registers).
    const int full = (kend - kbeg) / BK;
    if (full == nst) {
        main_loop(std::false_type{}, kbeg, nst);
    } else if constexpr (SPLIT != kWhole) {
        main_loop(std::true_type{}, kbeg, nst);
    } else {
        if (full > 0) {
            main_loop(std::false_type{}, kbeg, full);
            __syncthreads();  // the checked pass rewrites the LDS buffers the last stage read
        }
        main_loop(std::true_type{}, kbeg + full * BK, 1);
    }

    // Epilogue: block (bi, bj) register r is D[row 4g + r][col (bj/4)*64 +
    // 4*j16 + bj%4]: run q of the lane is bj = 4q .. 4q+3.
    const float alpha = p.alpha, beta = p.beta;
    const float* __restrict__ C = p.c;
    float* __restrict__ D       = p.d;
    const size_t ldc = p.ldc, ldd = p.ldd;
    const int col = n0 + wcol + 4 * j16;
    if constexpr (SPLIT == kPartial) {
#pragma unroll
        for (int bi = 0; bi < TM; ++bi) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wrow + bi * 16 + 4 * g + r;
                if (row >= M) continue;
#pragma unroll
                for (int q = 0; q < TN / 4; ++q) {
                    if (col + 64 * q >= N) continue;  // n % 4 == 0: a run of 4 columns is all in or all out
                    floatx4 out;
#pragma unroll
                    for (int t = 0; t < 4; ++t) out[t] = acc[bi][4 * q + t][r];
                    *reinterpret_cast<floatx4*>(D + (size_t)z * M * N + (size_t)row * N + col + 64 * q) = out;
                }
            }
        }
    } else {
        // One row block at a time, the c values of row block bi + 1 loaded
        // while row block bi is written (the barriers keep the scheduler
        // from hoisting every c load of the tile into registers at once).
        auto run = [&](auto c_tag) {
            constexpr bool HAS_C = decltype(c_tag)::value;
            floatx4 cv[HAS_C ? 2 : 1][4][TN / 4];
            auto load_c = [&](int bi, floatx4 (&dst)[4][TN / 4]) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = m0 + wrow + bi * 16 + 4 * g + r;
#pragma unroll
                    for (int q = 0; q < TN / 4; ++q)
                        dst[r][q] = row < M && col + 64 * q < N
                                        ? *reinterpret_cast<const floatx4*>(C + (size_t)row * ldc + col + 64 * q)
                                        : floatx4{0.f, 0.f, 0.f, 0.f};
                }
            };
            if constexpr (HAS_C) load_c(0, cv[0]);
#pragma unroll
            for (int bi = 0; bi < TM; ++bi) {
                if constexpr (HAS_C)
                    if (bi + 1 < TM) load_c(bi + 1, cv[(bi + 1) & 1]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = m0 + wrow + bi * 16 + 4 * g + r;
                    if (row >= M) continue;
#pragma unroll
                    for (int q = 0; q < TN / 4; ++q) {
                        if (col + 64 * q >= N) continue;  // n % 4 == 0: a run of 4 columns is all in or all out
                        floatx4 out;
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            out[t] = alpha * acc[bi][4 * q + t][r];
                            if constexpr (HAS_C) out[t] += beta * cv[HAS_C ? bi & 1 : 0][r][q][t];
                        }
                        *reinterpret_cast<floatx4*>(D + (size_t)row * ldd + col + 64 * q) = out;
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        if (C != nullptr)
            run(std::true_type{});
        else
            run(std::false_type{});
    }
}

template <int BM, int BN, int BK, int WM, int WN, int SPLIT, bool TA, bool TB, int MINB = 1, bool SIMPLE = false,
          int BAND = 4>
__global__ __launch_bounds__(WM* WN * 64, MINB) void mfma16_gemm(GemmParams p) {
    int bid = blockIdx.x, z = blockIdx.z;
    if constexpr (SPLIT != kWhole) {
        // Workgroups are dispatched in grid order (x fastest) and dealt to the 8 XCDs in turn, so
        // the tiles of one k split would land on different XCDs and each fetch the split's
        // shared operand slice into its own L2.  Renumber: the s-th workgroup on XCD x takes
        // work item x * (total / 8) + s, items ordered split-major, so each XCD runs whole splits
        // and every tile of a split reuses the slice from the same L2.
        const int tiles = gridDim.x, total = tiles * gridDim.z;
        // The tile index t is then handed to tile_of as the id whose XCD spreading yields t
        // back, so the tiles a workgroup walks stay in tile_of's band order.
        if ((total & 7) == 0) {
            const int lin = blockIdx.x + tiles * blockIdx.z;
            const int w   = (lin & 7) * (total >> 3) + (lin >> 3);
            z             = w / tiles;
            const int t   = w - z * tiles, per = tiles >> 3;
            bid           = t < (per << 3) ? ((t % per) << 3) + t / per : t;
        }
    }
    mfma16_gemm_tile<BM, BN, BK, WM, WN, SPLIT, TA, TB, MINB, SIMPLE, BAND>(p, bid, z);
}

// Index of the group that owns workgroup `bid`: the last g with
// start[g] <= bid (groups are listed with ascending, distinct starts).
__device__ __forceinline__ int find_group(const int32_t* __restrict__ start, int groups, int bid) {
    int lo = 0, hi = groups - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (start[mid] <= bid)
            lo = mid;
        else
            hi = mid - 1;
    }
    return lo;
}

// Grouped GEMM: workgroup bid runs tile bid - start[g] of group g, whose
// parameters sit in a device table.
template <int BM, int BN, int BK, int WM, int WN, bool TA, bool TB, int MINB, bool SIMPLE>
__global__ __launch_bounds__(WM* WN * 64, MINB) void grouped_mfma16_gemm(GroupedGemmArgs g) {
    const int bid = blockIdx.x;
    const int grp = find_group(g.tile_start, g.groups, bid);
    const GemmParams p = g.params[grp];
    // Group starts are multiples of 8, so the group-local id keeps the
    // hardware id's XCD (id mod 8); ids past the group's tiles are padding.
    const int local = bid - g.tile_start[grp];
    if (local >= p.tiles_m * p.tiles_n) return;
    mfma16_gemm_tile<BM, BN, BK, WM, WN, kWhole, TA, TB, MINB, SIMPLE>(p, local, 0);
}

// The 16x16x4 variants for one operand orientation: 0 = 256x256 whole-k,
// 1 = 256x256 split-k, 2 = 256x128 whole-k (two workgroups per CU),
// 3 = 256x128 split-k, 4 = 128x256 whole-k (two workgroups per CU),
// 5 / 6 = 64x256 whole-k / split-k, 7 / 8 = 256x64 whole-k / split-k (4 waves
// of 64x64, two workgroups per CU, pipelined loop); grouped: 16 = 256x128,
// 17 = 128x256.
template <bool TA, bool TB>
const void* mfma16Kernel(int which) {
    switch (which) {
        case 0: return reinterpret_cast<const void*>(&mfma16_gemm<256, 256, 16, 2, 2, kWhole, TA, TB>);
        case 1: return reinterpret_cast<const void*>(&mfma16_gemm<256, 256, 16, 2, 2, kPartial, TA, TB>);
        case 2: return reinterpret_cast<const void*>(&mfma16_gemm<256, 128, 16, 2, 2, kWhole, TA, TB, 2, true>);
        case 3: return reinterpret_cast<const void*>(&mfma16_gemm<256, 128, 16, 2, 2, kPartial, TA, TB, 2, true>);
        case 4: return reinterpret_cast<const void*>(&mfma16_gemm<128, 256, 16, 2, 2, kWhole, TA, TB, 2, true>);
        case 5: return reinterpret_cast<const void*>(&mfma16_gemm<64, 256, 16, 1, 4, kWhole, TA, TB, 2>);
        case 6: return reinterpret_cast<const void*>(&mfma16_gemm<64, 256, 16, 1, 4, kPartial, TA, TB, 2>);
        case 7: return reinterpret_cast<const void*>(&mfma16_gemm<256, 64, 16, 4, 1, kWhole, TA, TB, 2>);
        case 8: return reinterpret_cast<const void*>(&mfma16_gemm<256, 64, 16, 4, 1, kPartial, TA, TB, 2>);
        case 16: return reinterpret_cast<const void*>(&grouped_mfma16_gemm<256, 128, 16, 2, 2, TA, TB, 2, true>);
        case 17: return reinterpret_cast<const void*>(&grouped_mfma16_gemm<128, 256, 16, 2, 2, TA, TB, 2, true>);
        default: return nullptr;
    }
}

}  // namespace ftrain::gemm::m16
