// FP32 tile kernels (v_mfma_f32_16x16x4_f32) whose operands reach LDS by DMA
// (global_load_lds_dwordx4): 256x256 (4 waves of 128x128, one workgroup per
// CU), 64x256 / 256x64 / 128x128 (4 waves of 64x64, two workgroups per CU),
// 64x128 / 128x64 (waves of 32x64) and 64x64 (waves of 16x64), whole-k or
// split-k.  Row-major a and b on every tile; a column-major b (TB) and a
// column-major a (TA) on the tiles their kernels instantiate.  Device code
// only; kernels_dma32.hip (row-major, plain and grouped),
// kernels_dma32_tb.hip and kernels_dma32_ta.hip instantiate them.
//
// d = alpha * (a @ b) + beta * c (the reference's formula,
// src/primitive/hygon/gemm/fp32_gemm.hip:18-31: the beta term dropped for a
// null c, always evaluated otherwise); the split-k form writes each split's
// raw partial tile to slice z of the workspace (dense m x n) and
// splitk_reduce forms d.  Applicability, checked on the host: k a positive
// multiple of 32, n a multiple of 4, 16-byte aligned a, b, c, d with leading
// dimensions multiples of 4, a's and b's below 2^22 elements and c's and d's
// below 2^21 (32-bit offsets); m and n are free otherwise (edge tiles clamp
// their loads and drop their out-of-matrix stores).
//
// Wave tile: TM x TN blocks of 16x16 outputs:
//   A operand: lane l holds A[row l % 16][k slot g = l / 16]
//   B operand: lane l holds B[k slot g][col l % 16]
//   result   : lane l, register r holds D[row 4 g + r][col l % 16]
// Within a stage of 32 k, lane group g takes k = 8 g + s at k-step s
// (s = 0..7), so a lane's A values for four k-steps are one 128-bit LDS read.
// Column interleave: block bj, MFMA column j is wave-tile column
// (bj / 4) * 64 + 4 j + bj % 4, so one 128-bit read of four adjacent columns
// at one k serves four blocks, and each epilogue store writes four adjacent
// columns.
//
// Stage = 32 k of both operands (BM x 32 and 32 x BN floats); two stages.
// One DMA instruction moves 64 lanes x 16 bytes into 1 KiB of LDS at
// M0 + 16 * lane:
//   A [BM rows][32 k]: a DMA covers 8 rows (whole 128-byte lines); 16-byte
//     chunk c of row r sits at slot c ^ h(r) (a_swz below);
//   B [32 k][BN cols]: a DMA covers 256 / BN k rows; for BN >= 128 chunk c of
//     k row kr sits at slot c ^ (16 * ((kr >> 3) & 1)), separating the two k
//     rows a half-wave reads (a 64-wide row has no second half to swap with).
//
// Pipeline per stage st (buffer X; stage st + 1 in Y), per wave: k-steps
// 0..3 from registers while reading k-steps 4..7 of X; wait for this wave's
// LDS reads and DMAs, barrier (every wave is done with X, stage st + 1 has
// landed in Y); k-steps 4..7 while reading k-steps 0..3 of Y and issuing the
// DMA of stage st + 2 into X.  The DMA is issued from inline assembly with
// M0 set in the same statement; every wait on it is an explicit vmcnt in
// this file, and the compiler has no other use of M0 here (no LDS DMA
// builtins, no indexed register access).
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "ft/gemm_kernels.hpp"

namespace ftrain::gemm::d32 {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kStageK = 32;
// Word 3 of a raw (untyped, stride 0) buffer resource on gfx9 parts: 32-bit data format, the range
// check against num_records on every access.
constexpr int kBufferConfig = 0x00020000;

__device__ __forceinline__ void dma_1k(unsigned voff, const void* sbase, unsigned lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(sbase)
                 : "memory", "m0");
}

// 128-bit buffer store whose data registers stay unwritten for two wait states after it.  A VALU
// write of a store's data VGPRs right after a buffer_store_dwordx4 replaced the first dword of
// some lanes' data on MI355X (measured: the dword took the value the next instruction wrote),
// and the compiler inserts no wait for a buffer store with a register soffset.  The asm keeps
// `v` live past the store (so no write to its registers can come earlier) and waits there.
// CPOL: the store's cache-policy bits (0: write-back through the XCD's L2; 2: non-temporal).
template <int CPOL = 0>
__device__ __forceinline__ void store_b128(floatx4 v, __amdgpu_buffer_rsrc_t res, unsigned voff, int soff) {
    const u32x4 x = __builtin_bit_cast(u32x4, v);
    __builtin_amdgcn_raw_buffer_store_b128(x, res, voff, soff, CPOL);
    asm volatile("s_nop 1" ::"v"(x) : "memory");
}

// Output tile of workgroup `bid`: the 8 XCDs take contiguous runs of tile
// ids (hardware ids are dealt to XCDs in turn), walked in bands of
// `rows_per_band` tile rows.
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn, int rows_per_band = 4) {
    const int tiles = tiles_m * tiles_n;
    const int per   = tiles >> 3;
    int t           = bid;
    if (bid < (per << 3)) t = (bid & 7) * per + (bid >> 3);
    const int kBand = rows_per_band;
    const int band_span = kBand * tiles_n;
    const int band      = t / band_span;
    const int first_m   = band * kBand;
    const int band_rows = min(tiles_m - first_m, kBand);
    const int within    = t - band * band_span;
    tm                  = first_m + within % band_rows;
    tn                  = within / band_rows;
}

// Chunk swizzle of A: row bits 2, 1, 3 to chunk bits 0, 1, 2.  Reads run 16 lanes (16 consecutive
// rows, one chunk) at a time over 64 banks: rows of one parity get 8 distinct chunks; the 32
// lanes of a half-wave (two chunks two apart) also cover 128 banks.
__device__ __forceinline__ int a_swz(int row) {
    return ((row >> 2) & 1) | (((row >> 1) & 1) << 1) | (((row >> 3) & 1) << 2);
}

// Output tile `bid`, k split z of p; the whole workgroup calls it.
// TB: b column-major (element (k, j) at b[j * ldb + k]); its stage is staged per column (below).
// TA: a column-major (element (i, k) at a[k * lda + i]); its stage is [32 k][BM] like a row-major
// b's, and its rows interleave like b's columns (below).
// Cache policy of the split-k partial stores: non-temporal (the reduction kernel reads them once,
// after this launch; measured on MI355X, 64x4096x4096 on the 64x128 tile: about 0.5 us less per call).
constexpr int kPartialPolicy = 2;

// What the DMA pipeline reads when k holds no whole stage (its data is discarded): with the
// leading dimensions taken as 0, every lane's offset stays within 1 KiB of it.
static __device__ __attribute__((aligned(256))) float dma32_dummy[512];

template <int BM, int BN, int WM, int WN, bool SPLIT, bool TB = false, bool TA = false>
__device__ __forceinline__ void fp32_gemm_dma_tile(const GemmParams& p, int bid, int z, int band = 4) {
    static_assert(WM * WN == 4, "4 waves");
    constexpr int WTM = BM / WM, WTN = BN / WN, TM = WTM / 16, TN = WTN / 16, NC = TN / 4;
    static_assert(TN % 4 == 0 && TM >= 1, "column runs of four blocks");
    static_assert(!TA || TM % 4 == 0, "row runs of four blocks");
    constexpr int RA = 256 / BM;       // k rows per A DMA (column-major a)
    constexpr int CPA = BM / 4;        // 16-byte chunks per A k row (column-major a)
    constexpr bool ASWZ = CPA >= 32;
    constexpr int DA = BM / 32;        // A DMAs per wave per stage (8-row blocks)
    constexpr int RB = 256 / BN;       // k rows per B DMA (row-major b)
    constexpr int DB = BN / 32;        // B DMAs per wave per stage (8 k rows or 8 columns of b each)
    constexpr int ND = DA + DB;        // DMAs per wave per stage
    constexpr int CPR = BN / 4;        // 16-byte chunks per B k row
    constexpr bool BSWZ = CPR >= 32;   // B k rows have a second half to swap
    constexpr int NR = TM + 4 * NC;    // LDS reads per wave per half stage
    constexpr int SLOTS = 4 * TM;      // groups of TN MFMAs per half stage
    constexpr int A_FLOATS = BM * kStageK, B_FLOATS = kStageK * BN;

    __shared__ __attribute__((aligned(1024))) float As0[A_FLOATS];
    __shared__ __attribute__((aligned(1024))) float Bs0[B_FLOATS];
    __shared__ __attribute__((aligned(1024))) float As1[A_FLOATS];
    __shared__ __attribute__((aligned(1024))) float Bs1[B_FLOATS];
    const int tid = threadIdx.x, lane = tid & 63, j16 = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wrow = (wave / WN) * WTM, wcol = (wave % WN) * WTN;
    int tm, tn;
    tile_of(bid, p.tiles_m, p.tiles_n, tm, tn, band);
    const int m0 = tm * BM, n0 = tn * BN;
    const int M = p.m, N = p.n;
    const int kbeg = SPLIT ? z * p.k_chunk : 0;
    const int kend = SPLIT ? min(p.k, kbeg + p.k_chunk) : p.k;
    // Whole stages go through the DMA pipeline; a partial last one (k_tail) is staged afterwards.
    // With no whole stage the pipeline runs on the dummy (none).
    const int nst     = (kend - kbeg) / kStageK;
    const int k_tail  = (kend - kbeg) - nst * kStageK;
    const int last_st = nst > 0 ? nst - 1 : 0;
    const bool none   = nst == 0;
    const int64_t lda_r = p.lda, ldb_r = p.ldb;
    const int64_t lda = none ? 0 : lda_r, ldb = none ? 0 : ldb_r;
    const char* const dummy = reinterpret_cast<const char*>(dma32_dummy);

    // DMA sources.  A block q = wave + 4 j: rows 8q .. 8q + 7 (lane: row 8q + lane / 8), slot
    // lane % 8 holds chunk (lane % 8) ^ h(row); h does not depend on j (32 j leaves bits 1-3).
    // Rows past the matrix are clamped onto its last row (they feed only outputs that are not
    // stored); 255 rows of lda < 2^22 keep the lane offset below 2^32.
    const unsigned ar     = 8 * wave + (lane >> 3);
    const unsigned achunk = 16 * ((lane & 7) ^ a_swz(ar));
    const unsigned alast  = static_cast<unsigned>(min(M - 1 - m0, BM - 1));
    const unsigned lda4   = static_cast<unsigned>(4 * lda);
    const char* abase_r   = reinterpret_cast<const char*>(p.a + (size_t)m0 * lda_r + kbeg);
    const char* abase     = none ? dummy : abase_r;
    // B block q = wave + 4 j: k rows RB q .. RB q + RB - 1 (lane: row RB q + lane / CPR), slot
    // lane % CPR holds chunk (lane % CPR) ^ swizzle; a chunk past n is clamped onto the last whole
    // one (n % 4 == 0).  x = the swizzle bit of the block's k rows.
    const char* bbase_r = reinterpret_cast<const char*>(p.b + (size_t)kbeg * ldb_r + n0);
    const char* bbase   = none ? dummy : bbase_r;
    auto boff = [&](int x, int64_t ld) {
        const int kr = lane / CPR, chunk = (lane % CPR) ^ (x ? 16 : 0);
        return static_cast<unsigned>((kr * ld + (min(n0 + 4 * chunk, N - 4) - n0)) * 4);
    };
    const unsigned boff0 = boff(0, ldb), boff1 = BSWZ ? boff(1, ldb) : boff0;
    // Column-major a: block q = wave + 4 j holds k rows RA q .. RA q + RA - 1 of the stage (lane: k
    // row RA q + lane / CPA, slot lane % CPA holds chunk (lane % CPA) ^ swizzle, four rows of a);
    // a chunk past m is clamped onto the last whole one (m % 4 == 0).
    const char* atbase_r = reinterpret_cast<const char*>(p.a + (size_t)kbeg * lda_r + m0);
    const char* atbase   = none ? dummy : atbase_r;
    auto aoff = [&](int x, int64_t ld) {
        const int kr = lane / CPA, chunk = (lane % CPA) ^ (x ? 16 : 0);
        return static_cast<unsigned>((kr * ld + (min(m0 + 4 * chunk, M - 4) - m0)) * 4);
    };
    const unsigned aoff0 = TA ? aoff(0, lda) : 0u, aoff1 = TA && ASWZ ? aoff(1, lda) : aoff0;
    auto dma_a = [&](int st, int j, unsigned lds) {
        if constexpr (TA) {
            const int q = wave + 4 * j, kr0 = RA * q;
            dma_1k(ASWZ && ((kr0 >> 3) & 1) ? aoff1 : aoff0, atbase + ((size_t)st * kStageK + kr0) * lda * 4,
                   lds + q * 1024);
        } else {
            const unsigned row = min(ar + 32u * j, alast);
            dma_1k(row * lda4 + achunk, abase + (size_t)st * kStageK * 4, lds + (wave + 4 * j) * 1024);
        }
    };
    // Column-major b: block q = wave + 4 j holds columns 8q .. 8q + 7, each a whole 128-byte line of
    // 32 k.  Slot L of the block holds column 8q + cb, chunk ch with
    //   L = 32 b1(cb) + 16 b1(ch) + 8 b2(cb) + ((q & 7) ^ (4 b2(ch) + 2 b0(ch) + b0(cb)))
    // (bn(x) = bit n of x).  A half-wave read takes columns 4j + c (j = 0..15, c fixed) at chunks
    // 2g + hf of two adjacent g: those 32 sit in 32 distinct 16-byte slots modulo 512 bytes, the
    // width of the LDS banks (no bank conflict).  Columns past n are clamped onto the last one;
    // 255 columns of ldb < 2^22 keep the lane offset below 2^32.
    const char* btbase_r = reinterpret_cast<const char*>(p.b + (size_t)n0 * ldb_r + kbeg);
    const char* btbase   = none ? dummy : btbase_r;
    const unsigned blast = static_cast<unsigned>(min(N - 1 - n0, BN - 1));
    auto dma_bt = [&](int st, int j, unsigned lds) {
        const int q = wave + 4 * j, t = (lane & 7) ^ (q & 7);
        const int cb = 4 * ((lane >> 3) & 1) + 2 * (lane >> 5) + (t & 1), ch = 4 * (t >> 2) + 2 * ((lane >> 4) & 1) + ((t >> 1) & 1);
        const unsigned col = min(static_cast<unsigned>(8 * q + cb), blast);
        dma_1k(col * static_cast<unsigned>(4 * ldb) + 16 * ch, btbase + (size_t)st * kStageK * 4, lds + q * 1024);
    };
    auto dma_b = [&](int st, int j, unsigned lds) {
        if constexpr (TB) {
            dma_bt(st, j, lds);
        } else {
            const int q = wave + 4 * j, kr0 = RB * q;
            dma_1k(BSWZ && ((kr0 >> 3) & 1) ? boff1 : boff0, bbase + ((size_t)st * kStageK + kr0) * ldb * 4,
                   lds + q * 1024);
        }
    };
    // DMA d (0 .. ND - 1) of a stage: A and B alternate while both have some left.
    auto dma_one = [&](int st, int d, unsigned la, unsigned lb) {
        constexpr int PAIRS = DA < DB ? DA : DB;
        if (d < 2 * PAIRS) {
            if (d & 1)
                dma_b(st, d >> 1, lb);
            else
                dma_a(st, d >> 1, la);
        } else if (DA > DB) {
            dma_a(st, d - PAIRS, la);
        } else {
            dma_b(st, d - PAIRS, lb);
        }
    };
    const unsigned la0 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) float*)As0;
    const unsigned lb0 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) float*)Bs0;
    const unsigned la1 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) float*)As1;
    const unsigned lb1 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) float*)Bs1;

    // A operands of half hf (k-steps 4 hf .. 4 hf + 3) for block row bi: A[row][8 g + 4 hf .. + 3].
    // Column-major a: operands of k-step s for row run rr (blocks 4 rr .. 4 rr + 3): A[4 rows][8 g + s]
    // (block bi, MFMA row j is wave-tile row (bi / 4) * 64 + 4 j + bi % 4).
    auto rd_at = [&](const float* T, int s, int rr) {
        const int kr = 8 * g + s, c = (wrow >> 2) + 16 * rr + j16;
        return *reinterpret_cast<const floatx4*>(T + kr * BM + 4 * (ASWZ ? c ^ (16 * ((kr >> 3) & 1)) : c));
    };
    auto rd_a = [&](const float* T, int bi, int hf) {
        const int row = wrow + 16 * bi + j16, c = 2 * g + hf;
        return *reinterpret_cast<const floatx4*>(T + row * kStageK + 4 * (c ^ a_swz(row)));
    };
    // B operands of k-step s for column run cc (blocks 4 cc .. 4 cc + 3): B[8 g + s][4 cols].
    // Column-major b: block bj's operands of half hf (k-steps 4 hf .. 4 hf + 3) for column
    // wcol + (bj / 4) * 64 + 4 j16 + bj % 4 (the column interleave above).
    auto rd_bt = [&](const float* T, int hf, int bj) {
        const int col = wcol + (bj >> 2) * 64 + 4 * j16 + (bj & 3), q = col >> 3, cb = col & 7;
        const int ch = 2 * g + hf;
        const int slot = 64 * q + 32 * ((cb >> 1) & 1) + 16 * ((ch >> 1) & 1) + 8 * (cb >> 2) +
                         ((q & 7) ^ (4 * (ch >> 2) + 2 * (ch & 1) + (cb & 1)));
        return *reinterpret_cast<const floatx4*>(T + 4 * slot);
    };
    auto rd_b = [&](const float* T, int s, int cc) {
        const int kr = 8 * g + s, c = (wcol >> 2) + 16 * cc + j16;
        return *reinterpret_cast<const floatx4*>(T + kr * BN + 4 * (BSWZ ? c ^ (16 * ((kr >> 3) & 1)) : c));
    };

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Operands of one half stage: fa[bi] (4 k-steps), fb[s][cc] (4 columns); column-major b:
    // fb[bj & 3][bj >> 2] holds block bj's 4 k-steps.
    floatx4 fa0[TM], fb0[4][NC], fa1[TM], fb1[4][NC];
    // Read r (0 .. NR - 1) of half hf: TM A reads, then the B reads (k-step major).
    auto read_one = [&](floatx4 (&ga)[TM], floatx4 (&gb)[4][NC], const float* As, const float* Bs, int hf, int r) {
        if (r < TM)
            ga[r] = TA ? rd_at(As, 4 * hf + r / (TM / 4), r % (TM / 4)) : rd_a(As, r, hf);
        else if constexpr (TB)
            gb[(r - TM) & 3][(r - TM) >> 2] = rd_bt(Bs, hf, r - TM);
        else
            gb[(r - TM) / NC][(r - TM) % NC] = rd_b(Bs, 4 * hf + (r - TM) / NC, (r - TM) % NC);
    };
    // The MFMAs of one half stage on (fa, fb), k-step major, in SLOTS groups of TN (one block row
    // at one k-step); the NR reads into (ga, gb) spread over the slots, and with a true with_dma
    // the ND DMAs of stage dma_st too.  The scheduling groups pin that order (left to itself the
    // scheduler bunched the reads at the end of the half: 0.929-0.937 of peak at 8192^3 on the
    // 256x256 tile against 0.962-0.964).
    auto run_half = [&](floatx4 (&fa)[TM], floatx4 (&fb)[4][NC], floatx4 (&ga)[TM], floatx4 (&gb)[4][NC],
                        const float* As, const float* Bs, int hf, auto with_dma, int dma_st, unsigned la,
                        unsigned lb) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
            for (int bi = 0; bi < TM; ++bi) {
#pragma unroll
                for (int bj = 0; bj < TN; ++bj)
                    acc[bi][bj] = __builtin_amdgcn_mfma_f32_16x16x4f32(TA ? fa[s * (TM / 4) + (bi >> 2)][bi & 3]
                                                                                   : fa[bi][s],
                                                                      TB ? fb[bj & 3][bj >> 2][s]
                                                                                   : fb[s][bj >> 2][bj & 3],
                                                                      acc[bi][bj],
                                                                      0, 0, 0);
                const int u = TM * s + bi;
                bool read = false;
#pragma unroll
                for (int r = 0; r < NR; ++r)
                    if ((r * SLOTS) / NR == u) {
                        read_one(ga, gb, As, Bs, hf, r);
                        read = true;
                    }
                // Keep each slot's MFMAs, then its read, in that order.
                __builtin_amdgcn_sched_group_barrier(0x008, TN, 0);
                if (read) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                if constexpr (decltype(with_dma)::value) {
#pragma unroll
                    for (int d = 0; d < ND; ++d)
                        if (((2 * d + 1) * SLOTS) / (2 * ND) == u) dma_one(dma_st, d, la, lb);
                }
            }
        }
    };
    auto read_half = [&](floatx4 (&ga)[TM], floatx4 (&gb)[4][NC], const float* As, const float* Bs, int hf) {
#pragma unroll
        for (int r = 0; r < NR; ++r) read_one(ga, gb, As, Bs, hf, r);
    };

    // The pipeline always runs (on the dummy when k holds no whole stage).
    {
#pragma unroll
        for (int d = 0; d < ND; ++d) dma_one(0, d, la0, lb0);
        const int st1 = min(1, last_st);
#pragma unroll
        for (int d = 0; d < ND; ++d) dma_one(st1, d, la1, lb1);
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(ND) : "memory");
        read_half(fa0, fb0, As0, Bs0, 0);

        // Stages past the last reload the last one (nothing reads them).  The operand sets rotate
        // by copying (f1 -> f0 after each half); the allocator coalesces the copies, where
        // alternating the two sets by reference kept both live in separate registers and spilled.
        auto rotate = [&] {
#pragma unroll
            for (int i = 0; i < TM; ++i) fa0[i] = fa1[i];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int c = 0; c < NC; ++c) fb0[i][c] = fb1[i][c];
        };
#define FT_DMA32_PHASE(XA, XB, YA, YB, LXA, LXB, ST)                                              \
    run_half(fa0, fb0, fa1, fb1, XA, XB, 1, std::false_type{}, 0, 0u, 0u);                        \
    rotate();                                                                                     \
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");         \
    run_half(fa0, fb0, fa1, fb1, YA, YB, 0, std::true_type{}, min((ST) + 2, last_st), LXA, LXB);  \
    rotate();
        int st = 0;
        for (; st + 1 < nst; st += 2) {
            FT_DMA32_PHASE(As0, Bs0, As1, Bs1, la0, lb0, st)
            FT_DMA32_PHASE(As1, Bs1, As0, Bs0, la1, lb1, st + 1)
        }
        if (st < nst) {
            FT_DMA32_PHASE(As0, Bs0, As1, Bs1, la0, lb0, st)
        }
#undef FT_DMA32_PHASE
        // The workgroup's LDS must not be released with a DMA still writing it.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

        // k tail: the partial last stage is staged into buffer 0 by ordinary loads at the addresses
        // the DMAs would use (the real operands), lanes whose k lies past kend storing zeros and
        // loading nothing, once every wave has finished reading the buffers; then it is multiplied
        // like a whole stage.
        if (k_tail > 0) {
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            auto put = [&](float* stage, int q, bool ok, const char* src) {
                floatx4 v = floatx4{0.f, 0.f, 0.f, 0.f};
                if (ok) v = *reinterpret_cast<const floatx4*>(src);
                *reinterpret_cast<floatx4*>(reinterpret_cast<char*>(stage) + q * 1024 + 16 * lane) = v;
            };
            const size_t st_k = (size_t)nst * kStageK;
#pragma unroll
            for (int j = 0; j < DA; ++j) {
                const int q = wave + 4 * j;
                if constexpr (TA) {
                    const int kr0 = RA * q;
                    const unsigned off = aoff(ASWZ && ((kr0 >> 3) & 1), lda_r);
                    put(As0, q, kr0 + lane / CPA < k_tail, atbase_r + (st_k + kr0) * lda_r * 4 + off);
                } else {
                    const unsigned row = min(ar + 32u * j, alast);
                    put(As0, q, int(achunk / 4) < k_tail,
                        abase_r + st_k * 4 + (size_t)row * lda_r * 4 + achunk);
                }
            }
#pragma unroll
            for (int j = 0; j < DB; ++j) {
                const int q = wave + 4 * j;
                if constexpr (TB) {
                    const int t = (lane & 7) ^ (q & 7);
                    const int cb = 4 * ((lane >> 3) & 1) + 2 * (lane >> 5) + (t & 1);
                    const int ch = 4 * (t >> 2) + 2 * ((lane >> 4) & 1) + ((t >> 1) & 1);
                    const unsigned col = min(static_cast<unsigned>(8 * q + cb), blast);
                    put(Bs0, q, 4 * ch < k_tail, btbase_r + st_k * 4 + (size_t)col * ldb_r * 4 + 16 * ch);
                } else {
                    const int kr0 = RB * q;
                    const unsigned off = boff(BSWZ && ((kr0 >> 3) & 1), ldb_r);
                    put(Bs0, q, kr0 + lane / CPR < k_tail, bbase_r + (st_k + kr0) * ldb_r * 4 + off);
                }
            }
            __syncthreads();
            read_half(fa0, fb0, As0, Bs0, 0);
            run_half(fa0, fb0, fa1, fb1, As0, Bs0, 1, std::false_type{}, 0, 0u, 0u);
            rotate();
            run_half(fa0, fb0, fa1, fb1, As0, Bs0, 0, std::false_type{}, 0, 0u, 0u);
        }
    }

    // Epilogue, one row block at a time: block (bi, bj) register r is D[row 16 bi + 4 g + r][col
    // (bj / 4) * 64 + 4 j16 + bj % 4], four adjacent columns per 128-bit access; c of row block
    // bi + 1 is loaded while bi is written.  Buffer accesses relative to the tile's corner: the
    // lane part of the offset (4 g rows, 4 j16 columns) in the VGPR offset, the block part in the
    // scalar offset.  An element outside the matrix gets the lane offset 2^31, past the buffer's
    // size (at most 2^31 - 1 bytes), so its c load returns 0 and its store is dropped; ldc and
    // ldd below 2^21 keep every sum below 2^32.  Split-k: the raw sums go to slice z (dense
    // m x n, row stride n).
    const float alpha = p.alpha, beta = p.beta;
    const int rows_left = M - m0, cols_left = N - n0;
    auto span = [&](uint64_t ld) {
        const uint64_t b = ((uint64_t)(rows_left - 1) * ld + (uint64_t)cols_left) * 4;
        return static_cast<int>(b < 0x7FFFFFFFull ? b : 0x7FFFFFFFull);
    };
    const uint64_t ldd64 = SPLIT ? (uint64_t)N : (uint64_t)p.ldd;
    float* const dcorner = SPLIT ? p.d + (size_t)z * M * N + (size_t)m0 * N + n0 : p.d + (size_t)m0 * p.ldd + n0;
    const __amdgpu_buffer_rsrc_t dres = __builtin_amdgcn_make_buffer_rsrc(dcorner, 0, span(ldd64), kBufferConfig);
    const unsigned ldd = static_cast<unsigned>(ldd64), ldc = static_cast<unsigned>(p.ldc);
    constexpr unsigned kOut = 0x80000000u;
    // Lane group g's first row: 4 g, or with column-major a (rows interleaved) 16 g.
    constexpr int GROW = TA ? 16 : 4;
    const unsigned lane_d = (GROW * g * ldd + 4 * j16) * 4, lane_c = (GROW * g * ldc + 4 * j16) * 4;
    // Row of lane group 0 for block row bi, register r.
    auto row_of = [&](int bi, int r) { return TA ? wrow + (bi >> 2) * 64 + 4 * r + (bi & 3) : wrow + 16 * bi + r; };
    auto run = [&](auto c_tag) {
        constexpr bool HAS_C = decltype(c_tag)::value;
        __amdgpu_buffer_rsrc_t cres = dres;
        if constexpr (HAS_C)
            cres = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.c) + (size_t)m0 * p.ldc + n0, 0,
                                                     span(p.ldc), kBufferConfig);
        floatx4 cv[HAS_C ? 2 : 1][4][NC];
        auto load_c = [&](int bi, floatx4 (&dst)[4][NC]) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row0 = row_of(bi, r);
#pragma unroll
                for (int q = 0; q < NC; ++q) {
                    const int c0  = wcol + 64 * q;
                    const bool ok = GROW * g < rows_left - row0 && c0 + 4 * j16 < cols_left;
                    dst[r][q]     = __builtin_bit_cast(
                        floatx4, __builtin_amdgcn_raw_buffer_load_b128(cres, ok ? lane_c : kOut,
                                                                       static_cast<int>((row0 * ldc + c0) * 4), 0));
                }
            }
        };
        if constexpr (HAS_C) load_c(0, cv[0]);
#pragma unroll
        for (int bi = 0; bi < TM; ++bi) {
            if constexpr (HAS_C)
                if (bi + 1 < TM) load_c(bi + 1, cv[(bi + 1) & 1]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row0 = row_of(bi, r);
#pragma unroll
                for (int q = 0; q < NC; ++q) {
                    const int c0  = wcol + 64 * q;
                    const bool ok = GROW * g < rows_left - row0 && c0 + 4 * j16 < cols_left;
                    floatx4 out;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        if constexpr (SPLIT) {
                            out[t] = acc[bi][4 * q + t][r];
                        } else {
                            out[t] = alpha * acc[bi][4 * q + t][r];
                            if constexpr (HAS_C) out[t] += beta * cv[HAS_C ? bi & 1 : 0][r][q][t];
                        }
                    }
                    store_b128<SPLIT ? kPartialPolicy : 0>(out, dres, ok ? lane_d : kOut,
                                                           static_cast<int>((row0 * ldd + c0) * 4));
                }
            }
        }
    };
    if (!SPLIT && p.c != nullptr)
        run(std::true_type{});
    else
        run(std::false_type{});
}

template <int BM, int BN, int WM, int WN, int MINB, bool SPLIT, bool TB = false, bool TA = false>
__global__ __launch_bounds__(256, MINB) void fp32_gemm_dma(GemmParams p) {
    int bid = blockIdx.x, z = blockIdx.z;
    if constexpr (SPLIT) {
        // Workgroups are dealt to the 8 XCDs in grid order (x fastest); renumber so each XCD runs
        // whole k splits and every tile of a split reuses the split's operand slices from one L2.
        const int tiles = gridDim.x, total = tiles * gridDim.z;
        if ((total & 7) == 0) {
            const int lin = blockIdx.x + tiles * blockIdx.z;
            const int w   = (lin & 7) * (total >> 3) + (lin >> 3);
            z             = w / tiles;
            const int t   = w - z * tiles, per = tiles >> 3;
            bid           = t < (per << 3) ? ((t % per) << 3) + t / per : t;
        }
    }
    fp32_gemm_dma_tile<BM, BN, WM, WN, SPLIT, TB, TA>(p, bid, z);
}

// Grouped GEMM over a device table of per-group parameters (whole-k tiles): the workgroup's
// group is the last one whose first tile id is at most its own.  Group starts are multiples of
// 8, so the group-local id keeps the hardware id's XCD; ids past the group's tiles are padding and
// exit at once (the whole workgroup, before any barrier).
template <int BM, int BN, int WM, int WN, int MINB, bool TB, bool TA>
__global__ __launch_bounds__(256, MINB) void grouped_fp32_gemm_dma(GroupedGemmArgs g) {
    const int bid = blockIdx.x;
    int lo = 0, hi = g.groups - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (g.tile_start[mid] <= bid)
            lo = mid;
        else
            hi = mid - 1;
    }
    const GemmParams p = g.params[lo];
    const int local    = bid - g.tile_start[lo];
    if (local >= p.tiles_m * p.tiles_n) return;
    // One band per group of at most 16 tile rows: each group has a b of its own, which bands of 4
    // rows fetched once per band.
    fp32_gemm_dma_tile<BM, BN, WM, WN, false, TB, TA>(p, local, 0, p.tiles_m <= 16 ? p.tiles_m : 4);
}

}  // namespace ftrain::gemm::d32
