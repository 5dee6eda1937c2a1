// BF16 / FP16 MFMA tile kernel template (fp32 accumulation), shared by the
// per-type, per-layout HIP translation units kernels_half_*.hip.  Device
// code only.
//
// d = alpha * (a @ b) + beta * c with a, b in bf16 or fp16 (one type for
// both), products accumulated in fp32, the epilogue evaluated in fp32, and
// c / d either fp32 or the input type (rounded to nearest even).  The
// reference's numeric-type enum names both input types
// (include/flash_train/common.h:38-65); its only kernel is fp32
// (src/primitive/hygon/gemm/fp32_gemm.hip:18-31), whose semantics this
// follows: with a null c the beta term is dropped, with a non-null c it is
// always evaluated.
//
// MFMA: v_mfma_f32_32x32x16_{bf16,f16} (gfx950).  One instruction multiplies
// a 32x16 block of A by a 16x32 block of B into a 32x32 fp32 block:
//   A operand: lane l holds 8 values A[row = l % 32][one k group of 8]
//   B operand: lane l holds 8 values B[same k group][col = l % 32]
//   result   : lane l, register r holds D[row = 8*(r/4) + 4*(l/32) + r%4][col = l % 32]
// The k group of lane half h = l / 32 at step s is assigned
// k = h*BK/2 + 8*s + (0..7): the pairing only has to agree between A and B,
// and this choice makes each lane's operand one 16-byte LDS read.
//
// LDS: a k-contiguous operand is stored as [rows][BK + 8]; the 8-element pad
// makes the row stride 36 dwords, so the 16 lanes of one 128-bit read pass
// (consecutive rows) hit 16 disjoint 4-bank groups.
//
// Global -> LDS, per operand orientation:
//   k-contiguous in memory (row-major a, column-major b): 16-byte loads of 8
//     consecutive k, written to LDS as they are;
//   row/column-contiguous (column-major a, row-major b): 16-byte loads of 8
//     consecutive m (or n) at one k, written as they are into a k-major
//     tile, whose operands are then read with ds_read_b64_tr_b16 (TR);
//   per-element tiles (any shape): one element per load, stored k-contiguous.
// Consecutive threads walk each matrix's contiguous dimension, so the loads
// stay coalesced for every orientation.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "ft/gemm_kernels.hpp"

namespace ftrain::gemm::hdev {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));

enum SplitMode : int { kWhole = 0, kPartial = 2 };

// 16-bit storage <-> fp32.
template <bool BF16>
__device__ __forceinline__ float to_float(unsigned short v) {
    if constexpr (BF16)
        return __builtin_bit_cast(float, static_cast<unsigned int>(v) << 16);
    else
        return static_cast<float>(__builtin_bit_cast(_Float16, v));
}
template <bool BF16>
__device__ __forceinline__ unsigned short from_float(float v) {
    // Round to nearest even (the compiler's conversions; NaN stays NaN).
    if constexpr (BF16)
        return __builtin_bit_cast(unsigned short, static_cast<__bf16>(v));
    else
        return __builtin_bit_cast(unsigned short, static_cast<_Float16>(v));
}

template <bool BF16>
__device__ __forceinline__ floatx16 mfma(u32x4 a, u32x4 b, floatx16 acc) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       acc, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(halfx8, a), __builtin_bit_cast(halfx8, b),
                                                      acc, 0, 0, 0);
}

// Same XCD-aware tile order as the fp32 kernels: each XCD (workgroup id mod
// 8) receives a contiguous range of tiles, walked in bands of 8 tile rows.
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int tiles = tiles_m * tiles_n;
    const int per   = tiles >> 3;
    int t           = bid;
    if (bid < (per << 3)) t = (bid & 7) * per + (bid >> 3);
    constexpr int kBand = 8;
    const int band_span = kBand * tiles_n;
    const int band      = t / band_span;
    const int first_m   = band * kBand;
    const int band_rows = min(tiles_m - first_m, kBand);
    const int within    = t - band * band_span;
    tm                  = first_m + within % band_rows;
    tn                  = within / band_rows;
}

// ----------------------------------------------------------------------------
// BM x BN tile, BK k per stage, WM x WN waves (each (BM/WM) x (BN/WN) of
// 32x32 blocks), two LDS stages, one barrier per stage.  VEC: 16-byte global
// accesses (bases 16-byte aligned, leading dimensions and each matrix's
// contiguous extent multiples of 8); otherwise per-element loads, any shape.
// SPLIT: kWhole writes d; kPartial writes the raw fp32 partial tile to slice
// z of the workspace (dense m x n) for splitk_reduce.
// ----------------------------------------------------------------------------
// The tile body (see mfma_tile.hpp): tile `bid` of p's grid, split `z`.
template <bool BF16, int BM, int BN, int BK, int WM, int WN, int MINB, bool VEC, int SPLIT, bool TA, bool TB>
__device__ __forceinline__ void half_gemm_tile(const HalfGemmParams& p, int bid, int z) {
    using u16           = unsigned short;
    constexpr int NT    = WM * WN * 64;
    constexpr int WTM   = BM / WM;
    constexpr int WTN   = BN / WN;
    constexpr int TM    = WTM / 32;
    constexpr int TN    = WTN / 32;
    constexpr int STEPS = BK / 16;  // MFMA k-steps per stage
    constexpr int SK    = BK + 8;   // LDS row stride (elements)
    static_assert(TM >= 1 && TN >= 1 && BK % 16 == 0, "tile");
    // A transposed operand (column-major a, row-major b) of a 16-byte tile is
    // stored as it lies in memory, k-major, and read with transposing LDS
    // reads (TR); the per-element tile transposes while staging.
    constexpr bool A_TR = VEC && TA;
    constexpr bool B_TR = VEC && !TB;
    constexpr int A_LDS = A_TR ? (BM >= 256 ? BK * (BM + 32) + 128 : BK * BM) : BM * SK;
    constexpr int B_LDS = B_TR ? (BN >= 256 ? BK * (BN + 32) + 128 : BK * BN) : BN * SK;

    __shared__ __attribute__((aligned(16))) u16 As[2][A_LDS];
    __shared__ __attribute__((aligned(16))) u16 Bs[2][B_LDS];
    // Element (k, x) of a k-major tile with rows of W elements.  One
    // transposing read covers 64 bytes of 4 consecutive rows per lane half,
    // the halves BK/2 rows apart; the layout puts those 8 row pieces on
    // distinct banks.  W >= 256: row stride W + 32 elements, and the second
    // half of the k range 256 bytes further on.  W = 128 (rows of 256
    // bytes, no pad): 64-byte group g of row k is stored at group
    // g ^ (k & 3) ^ ((k / (BK/2)) & 1); 16-byte writes of 8 consecutive
    // lanes stay inside one aligned 128-byte run.
    static_assert((!A_TR || BM == 128 || BM >= 256) && (!B_TR || BN == 128 || BN >= 256), "TR tile width");
    auto tr_at = [](int k, int x, int W) {
        if (W >= 256) return k * (W + 32) + (k >= BK / 2 ? 128 : 0) + x;
        const int f = (k & 3) ^ ((k / (BK / 2)) & 1);
        return k * W + (x ^ (32 * f));
    };

    const int tid  = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int li   = lane & 31;
    const int h    = lane >> 5;
    const int wrow = (wave / WN) * WTM;
    const int wcol = (wave % WN) * WTN;

    int tm, tn;
    tile_of(bid, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int M = p.m, N = p.n, K = p.k;
    const int kbeg = SPLIT != kWhole ? z * p.k_chunk : 0;
    const int kend = SPLIT != kWhole ? min(K, kbeg + p.k_chunk) : K;
    const int nst  = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

    const u16* __restrict__ A = static_cast<const u16*>(p.a);
    const u16* __restrict__ B = static_cast<const u16*>(p.b);
    const size_t lda = p.lda, ldb = p.ldb;

    // Element (r, k) of a and (k, c) of b in global memory.
    auto a_at = [&](int gm, int gk) { return A + (TA ? (size_t)gk * lda + gm : (size_t)gm * lda + gk); };
    auto b_at = [&](int gk, int gn) { return B + (TB ? (size_t)gn * ldb + gk : (size_t)gk * ldb + gn); };

    // Staging registers.  VEC: ROWS*BK/8 vectors of 8 elements (8 k of a
    // k-contiguous operand, 8 m or n of a transposed one); scalar: ROWS*BK
    // elements.  Threads beyond the count idle for that operand.
    constexpr int A_VECS = VEC ? BM * BK / 8 : 0;
    constexpr int B_VECS = VEC ? BN * BK / 8 : 0;
    constexpr int A_PER  = VEC ? (A_VECS + NT - 1) / NT : BM * BK / NT;
    constexpr int B_PER  = VEC ? (B_VECS + NT - 1) / NT : BN * BK / NT;
    static_assert(VEC || (BM * BK % NT == 0 && BN * BK % NT == 0), "scalar staging");
    u32x4 ra[VEC ? A_PER : 1][1];
    u32x4 rb[VEC ? B_PER : 1][1];
    u16 sa[VEC ? 1 : A_PER];
    u16 sb[VEC ? 1 : B_PER];

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const u32x4 zero4 = u32x4{0u, 0u, 0u, 0u};

    // Stages [k_lo, k_lo + n_st * BK), the last one cut at kend.
    auto main_loop = [&](auto checked_tag, const int k_lo, const int n_st) {
        constexpr bool CHECKED = decltype(checked_tag)::value;
        // m / n index of a load.  The unchecked loop clamps it into the matrix
        // (a run of `run` elements stays inside): an edge tile then reads
        // valid memory for rows and columns past the edge, whose products
        // land only in outputs the epilogue does not store.  Only a k tail
        // needs the zero-filling checked loop.
        auto row_at = [](int i, int extent, int run) { return CHECKED ? i : min(i, extent - run); };

        // Global loads of one stage (k range [k0, k0 + BK)) into registers.
        // Entries: A staging slots 0 .. A_PER-1, then B slots; [first, last)
        // selects a part (the whole stage by default).
        auto load_stage = [&](int k0, int first = 0, int last = 1 << 20) {
            if constexpr (VEC) {
#pragma unroll
                for (int j = 0; j < A_PER; ++j) {
                    const int idx = tid + j * NT;
                    if (j < first || j >= last) continue;
                    if (A_VECS % NT != 0 && idx >= A_VECS) continue;
                    if constexpr (!TA) {  // (r, 8 k) vectors, 8 threads per row of BK = 64
                        const int r = idx / (BK / 8), kq = 8 * (idx % (BK / 8));
                        const int gm = row_at(m0 + r, M, 1), gk = k0 + kq;
                        ra[j][0] = zero4;
                        if (!CHECKED || (gm < M && gk < kend)) ra[j][0] = *reinterpret_cast<const u32x4*>(a_at(gm, gk));
                    } else {  // (k, 8 m) vectors along the contiguous m
                        const int k = idx / (BM / 8), mq = 8 * (idx % (BM / 8));
                        const int gm = row_at(m0 + mq, M, 8), gk = k0 + k;
                        ra[j][0] = zero4;
                        if (!CHECKED || (gm < M && gk < kend)) ra[j][0] = *reinterpret_cast<const u32x4*>(a_at(gm, gk));
                    }
                }
#pragma unroll
                for (int j = 0; j < B_PER; ++j) {
                    const int idx = tid + j * NT;
                    if (A_PER + j < first || A_PER + j >= last) continue;
                    if (B_VECS % NT != 0 && idx >= B_VECS) continue;
                    if constexpr (TB) {  // (c, 8 k) vectors
                        const int c = idx / (BK / 8), kq = 8 * (idx % (BK / 8));
                        const int gn = row_at(n0 + c, N, 1), gk = k0 + kq;
                        rb[j][0] = zero4;
                        if (!CHECKED || (gn < N && gk < kend)) rb[j][0] = *reinterpret_cast<const u32x4*>(b_at(gk, gn));
                    } else {  // (k, 8 n) vectors along the contiguous n
                        const int k = idx / (BN / 8), nq = 8 * (idx % (BN / 8));
                        const int gn = row_at(n0 + nq, N, 8), gk = k0 + k;
                        rb[j][0] = zero4;
                        if (!CHECKED || (gn < N && gk < kend)) rb[j][0] = *reinterpret_cast<const u32x4*>(b_at(gk, gn));
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < A_PER; ++j) {
                    const int idx = tid + j * NT;
                    const int r = TA ? idx % BM : idx / BK, k = TA ? idx / BM : idx % BK;
                    const int gm = row_at(m0 + r, M, 1), gk = k0 + k;
                    sa[j]        = (!CHECKED || (gm < M && gk < kend)) ? *a_at(gm, gk) : u16(0);
                }
#pragma unroll
                for (int j = 0; j < B_PER; ++j) {
                    const int idx = tid + j * NT;
                    const int c = TB ? idx / BK : idx % BN, k = TB ? idx % BK : idx / BN;
                    const int gn = row_at(n0 + c, N, 1), gk = k0 + k;
                    sb[j]        = (!CHECKED || (gk < kend && gn < N)) ? *b_at(gk, gn) : u16(0);
                }
            }
        };

        // Registers -> LDS buffer `buf` (k-contiguous rows).
        auto store_stage = [&](int buf, int first = 0, int last = 1 << 20) {
            if constexpr (VEC) {
#pragma unroll
                for (int j = 0; j < A_PER; ++j) {
                    const int idx = tid + j * NT;
                    if (j < first || j >= last) continue;
                    if (A_VECS % NT != 0 && idx >= A_VECS) continue;
                    if constexpr (!TA) {
                        const int r = idx / (BK / 8), kq = 8 * (idx % (BK / 8));
                        *reinterpret_cast<u32x4*>(&As[buf][r * SK + kq]) = ra[j][0];
                    } else {
                        const int k = idx / (BM / 8), mq = 8 * (idx % (BM / 8));
                        *reinterpret_cast<u32x4*>(&As[buf][tr_at(k, mq, BM)]) = ra[j][0];
                    }
                }
#pragma unroll
                for (int j = 0; j < B_PER; ++j) {
                    const int idx = tid + j * NT;
                    if (A_PER + j < first || A_PER + j >= last) continue;
                    if (B_VECS % NT != 0 && idx >= B_VECS) continue;
                    if constexpr (TB) {
                        const int c = idx / (BK / 8), kq = 8 * (idx % (BK / 8));
                        *reinterpret_cast<u32x4*>(&Bs[buf][c * SK + kq]) = rb[j][0];
                    } else {
                        const int k = idx / (BN / 8), nq = 8 * (idx % (BN / 8));
                        *reinterpret_cast<u32x4*>(&Bs[buf][tr_at(k, nq, BN)]) = rb[j][0];
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < A_PER; ++j) {
                    const int idx = tid + j * NT;
                    const int r = TA ? idx % BM : idx / BK, k = TA ? idx / BM : idx % BK;
                    As[buf][r * SK + k] = sa[j];
                }
#pragma unroll
                for (int j = 0; j < B_PER; ++j) {
                    const int idx = tid + j * NT;
                    const int c = TB ? idx / BK : idx % BN, k = TB ? idx % BK : idx / BN;
                    Bs[buf][c * SK + k] = sb[j];
                }
            }
        };

        // All MFMAs of one stage; operands of step s+1 are read while step
        // s's MFMAs run (the compiler hoists the reads of the unrolled loop).
        // Operands of k-step s of LDS buffer `buf`.
        // A k-major (TR) tile is read with ds_read_b64_tr_b16: within each
        // group of 16 lanes, lane 4j + a reads 4 consecutive elements of k
        // row j, and lane 4a + e receives element e of lanes a, 4 + a, 8 + a,
        // 12 + a, i.e. 4 consecutive k of one column.  Lane l's source row
        // and column offset are j = (l & 15) >> 2 and 16 * ((l >> 4) & 1) +
        // 4 * (l & 3); two reads (k + 0..3, k + 4..7) make one operand.
        const int tr_k = (lane & 15) >> 2, tr_x = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
        auto read_tr = [&](const u16* tile, int W, int kk, int x) {
            typedef short v4i16 __attribute__((ext_vector_type(4)));
            typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
            const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(tile + tr_at(kk + tr_k, x + tr_x, W)));
            const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(tile + tr_at(kk + 4 + tr_k, x + tr_x, W)));
            const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
            return u32x4{l2[0], l2[1], h2[0], h2[1]};
        };
        auto read_ops = [&](int buf, int s, u32x4 (&av)[TM], u32x4 (&bv)[TN]) {
            const int kk = h * (BK / 2) + 8 * s;
#pragma unroll
            for (int bi = 0; bi < TM; ++bi) {
                if constexpr (A_TR)
                    av[bi] = read_tr(As[buf], BM, kk, wrow + bi * 32);
                else
                    av[bi] = *reinterpret_cast<const u32x4*>(&As[buf][(wrow + bi * 32 + li) * SK + kk]);
            }
#pragma unroll
            for (int bj = 0; bj < TN; ++bj) {
                if constexpr (B_TR)
                    bv[bj] = read_tr(Bs[buf], BN, kk, wcol + bj * 32);
                else
                    bv[bj] = *reinterpret_cast<const u32x4*>(&Bs[buf][(wcol + bj * 32 + li) * SK + kk]);
            }
        };
        // MFMAs [first, last) of one k-step, blocks in row-major order.
        auto mfmas = [&](const u32x4 (&av)[TM], const u32x4 (&bv)[TN], int first, int last) {
#pragma unroll
            for (int i = 0; i < TM * TN; ++i)
                if (i >= first && i < last) acc[i / TN][i % TN] = mfma<BF16>(av[i / TN], bv[i % TN], acc[i / TN][i % TN]);
        };

        if constexpr (!VEC) {
            // Per-element path: straightforward two-stage loop.
            if (n_st > 0) {
                load_stage(k_lo);
                store_stage(0);
            }
            __syncthreads();
            for (int st = 0; st < n_st; ++st) {
                if (st + 1 < n_st) load_stage(k_lo + (st + 1) * BK);
#pragma unroll
                for (int s = 0; s < STEPS; ++s) {
                    u32x4 av[TM], bv[TN];
                    read_ops(st & 1, s, av, bv);
                    mfmas(av, bv, 0, TM * TN);
                }
                if (st + 1 < n_st) store_stage((st + 1) & 1);
                __syncthreads();
            }
        } else {
            {
                // Software pipeline.  Stage st computes from LDS buffer st&1
                // while registers hold the global data of stage st+1.  The
                // staging entries (A slots, then B slots) are split into STEPS
                // parts; during k-step s, part s of stage st+1 is written to the
                // other LDS buffer and part s of stage st+2 is loaded into the
                // registers it frees, interleaved with that step's MFMAs and the
                // operand reads of step s+1 (the other buffer is free from the
                // barrier of stage st-1 on: every read of it precedes that
                // barrier).  In the last step the barrier (stage st+1 complete
                // and visible) comes before the final TAIL MFMAs, so stage
                // st+1's first operands are read under them.  sched_barrier(0)
                // keeps each phase where it is written.  Past the last stage
                // the loads re-read the final stage and the extra LDS writes land
                // in a buffer nobody reads again.
                static_assert(STEPS % 2 == 0, "operand register sets alternate by step");
                constexpr int NB    = TM * TN;
                constexpr int TAIL  = NB >= 8 ? 4 : NB / 2;  // MFMAs left after the barrier
                constexpr int ENT   = A_PER + B_PER;
                constexpr int PART  = (ENT + STEPS - 1) / STEPS;
                // Upper bound of one part's 16-byte loads (or LDS writes) per
                // tail MFMA.
                constexpr int PER_MFMA = (PART + NB - TAIL - 1) / (NB - TAIL);
                u32x4 opa[2][TM], opb[2][TN];
                auto clamp_k0 = [&](int stage) { return k_lo + min(stage, n_st - 1) * BK; };
                if (n_st > 0) {
                    load_stage(k_lo);
                    store_stage(0);
                    load_stage(clamp_k0(1));
                }
                __syncthreads();
                if (n_st > 0) read_ops(0, 0, opa[0], opb[0]);
                for (int st = 0; st < n_st; ++st) {
                    const int cur = st & 1;
    #pragma unroll
                    for (int s = 0; s < STEPS; ++s) {
                        const int e0 = s * PART, e1 = min(ENT, (s + 1) * PART);
                        if (s + 1 < STEPS) read_ops(cur, s + 1, opa[(s + 1) & 1], opb[(s + 1) & 1]);
                        store_stage(cur ^ 1, e0, e1);
                        load_stage(clamp_k0(st + 2), e0, e1);
                        if (s + 1 < STEPS) {
                            mfmas(opa[s & 1], opb[s & 1], 0, NB);
    #pragma unroll
                            for (int i = 0; i < NB; ++i) {
                                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                                __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
                                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
                            }
                            __builtin_amdgcn_sched_barrier(0);
                        } else {
                            mfmas(opa[s & 1], opb[s & 1], 0, NB - TAIL);
    #pragma unroll
                            for (int i = 0; i < NB - TAIL; ++i) {
                                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                                __builtin_amdgcn_sched_group_barrier(0x200, PER_MFMA, 0);  // DS write
                                __builtin_amdgcn_sched_group_barrier(0x020, PER_MFMA, 0);  // VMEM read
                            }
                            __builtin_amdgcn_sched_barrier(0);
                            __syncthreads();
                            read_ops(cur ^ 1, 0, opa[0], opb[0]);
                            __builtin_amdgcn_sched_barrier(0);
                            mfmas(opa[s & 1], opb[s & 1], NB - TAIL, NB);
                            __builtin_amdgcn_sched_barrier(0);
                        }
                    }
                }
            }
        }
    };

    // A k tail: the whole stages run the unchecked loop and the last, partial one a checked pass of
    // its own (zeros past kend); a vector tile checked throughout ran at about 0.7 of the speed
    // (bf16 grouped weight gradient, 8 experts of ragged token counts, 16384x4096x14336 in total:
    // 2.63 ms against 1.93 with token counts rounded to multiples of 64).
    const int full = (kend - kbeg) / BK;
    if (full == nst) {
        main_loop(std::false_type{}, kbeg, nst);
    } else if constexpr (VEC) {
        if (full > 0) {
            main_loop(std::false_type{}, kbeg, full);
            __syncthreads();  // the checked pass rewrites the LDS buffers the last stage read
        }
        main_loop(std::true_type{}, kbeg + full * BK, 1);
    } else {
        main_loop(std::true_type{}, kbeg, nst);
    }

    // Epilogue: lane li owns column wcol + bj*32 + li of each block; c and d
    // are row-major (row strides ldc, ldd) in fp32 or the input type.
    if constexpr (SPLIT == kPartial) {
#pragma unroll
        for (int bi = 0; bi < TM; ++bi)
#pragma unroll
            for (int bj = 0; bj < TN; ++bj) {
                const int col = n0 + wcol + bj * 32 + li;
                if (col >= N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + wrow + bi * 32 + 8 * (r / 4) + 4 * h + (r % 4);
                    if (row < M) static_cast<float*>(p.d)[(size_t)z * M * N + (size_t)row * N + col] = acc[bi][bj][r];
                }
            }
    } else {
        // c is read one unit of UB blocks ahead of the stores, so its loads
        // are in flight while the previous unit is written.
        const float alpha = p.alpha, beta = p.beta;
        constexpr int UB = TN > 1 ? TN / 2 : 1;  // blocks per unit
        constexpr int UNITS = TM * TN / UB;
        auto run = [&](auto c_tag, auto half_tag) {
            constexpr bool HAS_C = decltype(c_tag)::value;
            constexpr bool HALF  = decltype(half_tag)::value;
            float cv[HAS_C ? 2 : 1][UB][16];
            auto load_c = [&](int u, float (&dst)[UB][16]) {
                const int bi = u / (TN / UB), bj0 = (u % (TN / UB)) * UB;
#pragma unroll
                for (int t = 0; t < UB; ++t) {
                    const int col = n0 + wcol + (bj0 + t) * 32 + li;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row     = m0 + wrow + bi * 32 + 8 * (r / 4) + 4 * h + (r % 4);
                        const size_t ci   = (size_t)row * p.ldc + col;
                        const bool inside = col < N && row < M;
                        if constexpr (HALF)
                            dst[t][r] = inside ? to_float<BF16>(static_cast<const u16*>(p.c)[ci]) : 0.f;
                        else
                            dst[t][r] = inside ? static_cast<const float*>(p.c)[ci] : 0.f;
                    }
                }
            };
            if constexpr (HAS_C) load_c(0, cv[0]);
#pragma unroll
            for (int u = 0; u < UNITS; ++u) {
                if constexpr (HAS_C)
                    if (u + 1 < UNITS) load_c(u + 1, cv[(u + 1) & 1]);
                __builtin_amdgcn_sched_barrier(0);
                const int bi = u / (TN / UB), bj0 = (u % (TN / UB)) * UB;
#pragma unroll
                for (int t = 0; t < UB; ++t) {
                    const int col = n0 + wcol + (bj0 + t) * 32 + li;
                    if (col >= N) continue;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = m0 + wrow + bi * 32 + 8 * (r / 4) + 4 * h + (r % 4);
                        if (row >= M) continue;
                        const size_t di = (size_t)row * p.ldd + col;
                        float out       = alpha * acc[bi][bj0 + t][r];
                        if constexpr (HAS_C) out += beta * cv[HAS_C ? u & 1 : 0][t][r];
                        // d is not read again here: non-temporal stores keep
                        // the burst of a round's outputs from allocating in
                        // L2 (bf16 8192^3: +1.7-2.4%).
                        if constexpr (HALF)
                            __builtin_nontemporal_store(from_float<BF16>(out), static_cast<u16*>(p.d) + di);
                        else
                            __builtin_nontemporal_store(out, static_cast<float*>(p.d) + di);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        if (p.c != nullptr) {
            if (p.cd_half)
                run(std::true_type{}, std::true_type{});
            else
                run(std::true_type{}, std::false_type{});
        } else {
            if (p.cd_half)
                run(std::false_type{}, std::true_type{});
            else
                run(std::false_type{}, std::false_type{});
        }
    }
}

template <bool BF16, int BM, int BN, int BK, int WM, int WN, int MINB, bool VEC, int SPLIT, bool TA, bool TB>
__global__ __launch_bounds__(WM* WN * 64, MINB) void half_gemm(HalfGemmParams p) {
    half_gemm_tile<BF16, BM, BN, BK, WM, WN, MINB, VEC, SPLIT, TA, TB>(p, blockIdx.x, blockIdx.z);
}

// Grouped GEMM over a device table of per-group parameters (see
// grouped_mfma_gemm in mfma_tile.hpp).
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

template <bool BF16, int BM, int BN, int BK, int WM, int WN, int MINB, bool VEC, bool TA, bool TB>
__global__ __launch_bounds__(WM* WN * 64, MINB) void grouped_half_gemm(GroupedHalfArgs g) {
    const int bid = blockIdx.x;
    const int grp = find_group(g.tile_start, g.groups, bid);
    const HalfGemmParams p = g.params[grp];
    // Group starts are multiples of 8, so the group-local id keeps the
    // hardware id's XCD (id mod 8); ids past the group's tiles are padding.
    const int local = bid - g.tile_start[grp];
    if (local >= p.tiles_m * p.tiles_n) return;
    half_gemm_tile<BF16, BM, BN, BK, WM, WN, MINB, VEC, kWhole, TA, TB>(p, local, 0);
}

// The 256x256 tile, every operand orientation: 8 waves of 128x64 (two per
// SIMD), transposed operands stored k-major and read with transposing LDS
// reads (TR), staging spread over the k-steps.  Results are bit-identical to
// the 8x8 in-register transposes this replaced (same MFMA sequence).  Measured bf16, TFLOP/s at
// 8192^3 / 4096^3, TR against the in-register transposes with their best
// wave counts: row-major a with row-major b 1221 / 1128 against 1079 / 955;
// column-major a with row-major b 1216 / 1126 against 974 / 789; both
// column-major 1226 / 1114 against 1146 / 946.  TR with 4 waves of 128x128:
// 1153-1201 / 967-999.  The 128x128 tiles (4 waves of 64x64, two
// workgroups per CU) use TR too: at 2048^3 / 4096^3 row-major a with
// row-major b 571 / 921 against 441 / 736, column-major a with row-major b
// 565 / 875 against 287 / 507, both column-major 577 / 880 against 454 / 735.
struct Wide {
    static constexpr int WN = 4;
};

// The half-precision tiles (index as in kHalfTiles) for one input type and
// one operand orientation.
template <bool BF16, bool TA, bool TB>
const void* halfKernel(int tile) {
    switch (tile) {
        case 0: {
            using W = Wide;
            return reinterpret_cast<const void*>(
                &half_gemm<BF16, 256, 256, 64, 2, W::WN, 1, true, kWhole, TA, TB>);
        }
        case 1: return reinterpret_cast<const void*>(&half_gemm<BF16, 128, 128, 64, 2, 2, 2, true, kWhole, TA, TB>);
        case 2:
            return reinterpret_cast<const void*>(&half_gemm<BF16, 128, 128, 64, 2, 2, 2, true, kPartial, TA, TB>);
        case 3: return reinterpret_cast<const void*>(&half_gemm<BF16, 64, 64, 32, 2, 2, 2, false, kWhole, TA, TB>);
        default: return nullptr;
    }
}

// Grouped variants: 0 = 128x128 (16-byte loads), 1 = 64x64 per-element,
// 2 = 256x256 (16-byte loads, Wide).
template <bool BF16, bool TA, bool TB>
const void* groupedHalfKernel(int which) {
    switch (which) {
        case 0:
            return reinterpret_cast<const void*>(&grouped_half_gemm<BF16, 128, 128, 64, 2, 2, 2, true, TA, TB>);
        case 1: return reinterpret_cast<const void*>(&grouped_half_gemm<BF16, 64, 64, 32, 2, 2, 2, false, TA, TB>);
        case 2: {
            using W = Wide;
            return reinterpret_cast<const void*>(
                &grouped_half_gemm<BF16, 256, 256, 64, 2, W::WN, 1, true, TA, TB>);
        }
        default: return nullptr;
    }
}

}  // namespace ftrain::gemm::hdev
