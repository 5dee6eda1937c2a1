// BF16 / FP16 tile kernels whose operands reach LDS by DMA
// (global_load_lds_dwordx4) instead of through registers: 256x256 (plain and
// grouped) and 128x128 (plain whole-k and split-k, grouped).
// Device code only; the per-type translation units kernels_half_dma_*.hip
// instantiate it.
//
// d = alpha * (a @ b) + beta * c, the same contract as the register-staged
// tiles of half_tile.hpp (fp32 accumulation; c and d in fp32 or the input
// type; with a null c the beta term is dropped).  Applicability, checked on
// the host: k a multiple of 64 (no k tail: a DMA cannot zero-fill), a and b
// 16-byte aligned with leading dimensions multiples of 8 elements and below
// 2^23, c and d leading dimensions below 2^21 (32-bit offsets), contiguous
// extents multiples of 8; m and n are free (edge tiles clamp their loads and
// drop their out-of-matrix stores).
//
// Workgroup: 4 waves (one per SIMD), each a T/2 x T/2 block of the tile, as
// (T/64) x (T/64) v_mfma_f32_32x32x16 blocks (4x4 at T = 256, 2x2 at 128):
//   A operand: lane l holds A[row l % 32][8 consecutive k]
//   B operand: lane l holds B[the same 8 k][col l % 32]
//   result   : lane l, register r holds D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32]
// In k-step s (16 k) lane half h = l / 32 takes k 16 s + 8 h .. 16 s + 8 h + 7.
//
// Stage = 64 k of both operands, T x 64 x 2 bytes each; two LDS stages (128
// KiB at T = 256, 64 KiB at 128).  One DMA instruction moves 64 lanes x 16
// bytes into 1 KiB of LDS at M0 + 16 * lane, each lane from its own global
// address, so a stage takes T/8 instructions per operand, T/32 per wave.
// Each covers whole 128-byte lines:
//   k-contiguous operand (row-major a, column-major b): 8 rows x 64 k, LDS
//     [T rows][64 k], 16-byte chunk c of row r at slot c ^ ((r >> 1) & 7);
//     read with ds_read_b128 (one per operand);
//   transposed operand (column-major a, row-major b): 512 / T k rows x T,
//     LDS [64 k][T], chunk c of k row kr at slot c ^ (4 (kr & 3)); read with
//     ds_read_b64_tr_b16 (two per operand).
// Both swizzles keep the reads free of bank conflicts (SQ_LDS_BANK_CONFLICT
// reads 0 on MI355X).
//
// Pipeline of stage st in buffer X (stage st + 1 in Y), per wave:
//   half 1: MFMAs on k 0..31 (registers) while reading k 32..63 of X;
//   wait for this wave's LDS reads and DMAs, barrier: every wave is done
//     with X, and stage st + 1 has landed in Y;
//   half 2: MFMAs on k 32..63 while reading k 0..31 of Y and issuing the
//     DMA of stage st + 2 into X.
// A DMA has one stage of MFMAs (2048 MFMA cycles per wave at T = 256) to land.  The
// DMA is issued from inline assembly with M0 set in the same statement, so
// the compiler's wait-count bookkeeping never sees it: every wait on it is
// the explicit vmcnt in this file.  The compiler does not otherwise use M0
// in this kernel (no LDS DMA builtins, no indexed register access: every
// loop is unrolled).
//
// Measured on MI355X, same box and session, against the register-staged
// 256x256 tile: bf16 8192^3 row-major a and b 848 against 991 us (every
// orientation within 1%); MLP fwd 16384x14336x4096 1467 against 1748 us;
// 4096^3 with c 125 against 158 us; MFMA busy 80-82%.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "ft/gemm_kernels.hpp"

namespace ftrain::gemm::ddev {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
using u16 = unsigned short;

constexpr int kStageK = 64;
// Most tile rows a grouped launch walks as one band (tile_of).
constexpr int kGroupBand = 16;
// Word 3 of a raw (untyped, stride 0) buffer resource on gfx9 parts: 32-bit data format, the range
// check against num_records on every access.
constexpr int kBufferConfig = 0x00020000;

template <bool BF16>
__device__ __forceinline__ floatx16 mfma(u32x4 a, u32x4 b, floatx16 acc) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       acc, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(halfx8, a), __builtin_bit_cast(halfx8, b),
                                                      acc, 0, 0, 0);
}

template <bool BF16>
__device__ __forceinline__ float to_float(u16 v) {
    if constexpr (BF16)
        return __builtin_bit_cast(float, static_cast<unsigned int>(v) << 16);
    else
        return static_cast<float>(__builtin_bit_cast(_Float16, v));
}

template <bool BF16>
__device__ __forceinline__ u16 from_float(float v) {
    if constexpr (BF16)
        return __builtin_bit_cast(u16, static_cast<__bf16>(v));
    else
        return __builtin_bit_cast(u16, static_cast<_Float16>(v));
}

// 1 KiB DMA: lane l copies 16 bytes from sbase + voff(l) to LDS byte address lds + 16 l.
__device__ __forceinline__ void dma_1k(unsigned voff, const void* sbase, unsigned lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(sbase)
                 : "memory", "m0");
}

// Output tile of workgroup `bid`: consecutive ids go to the 8 XCDs in turn,
// so each XCD gets a contiguous run of tile ids, walked in bands of
// `rows_per_band` tile rows (a band's a panels stay in that XCD's L2 while its b panels
// stream; every band fetches the whole of b once).
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn, int rows_per_band = 8) {
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

// One operand's staging: where each DMA reads.  TR: the operand is
// transposed in memory (k rows, its m or n extent contiguous).  Rows (or
// columns) past the matrix edge are clamped onto its last row (column
// group): they read valid memory and feed only outputs the epilogue does not
// store.
template <bool TR, int T>
struct Operand {
    static constexpr int kCpr = T / 8;        // TR: 16-byte chunks per k row
    static constexpr int kRpd = 64 / kCpr;    // TR: k rows per DMA block
    const char* base;  // tile origin (element 0 of its first row / k row)
    int64_t ld;        // leading dimension, elements
    unsigned voff;     // TR: this lane's byte offset inside every DMA block
    unsigned r8;       // k-contiguous: this lane's row inside DMA block 0
    unsigned chunk16;  // k-contiguous: byte offset of this lane's 16-byte k chunk
    unsigned last;     // k-contiguous: last row of the tile inside the matrix
    unsigned ld2;      // k-contiguous: row stride in bytes (below 2^24)

    // origin: the tile's first row (column); extent: rows (columns) in the matrix.
    __device__ __forceinline__ void init(const u16* m, int64_t ld_, int origin, int extent, int wave, int lane) {
        ld = ld_;
        if constexpr (TR) {
            // Block q = wave + 4 j holds k rows R q .. R q + R - 1, R = 64 / (T / 8) (lane: row
            // R q + lane / (T / 8)); slot lane % (T / 8) holds 8-element chunk (lane % (T / 8)) ^
            // (4 (kr & 3)).  kr & 3 does not depend on j (4 R j is a multiple of 4).  The extent is a
            // multiple of 8, so a clamped chunk is a whole one.
            const int kr = kRpd * wave + lane / kCpr, chunk = (lane % kCpr) ^ (4 * (kr & 3));
            const int col = min(origin + 8 * chunk, extent - 8) - origin;
            base          = reinterpret_cast<const char*>(m + origin);
            voff          = static_cast<unsigned>((kr * ld + col) * 2);
        } else {
            // Block q = wave + 4 j holds rows 8q .. 8q + 7 (lane: row 8q + lane / 8); slot lane % 8
            // holds k chunk (lane % 8) ^ ((row >> 1) & 7), which does not depend on j.
            r8      = 8 * wave + (lane >> 3);
            chunk16 = 16 * ((lane & 7) ^ ((r8 >> 1) & 7));
            last    = static_cast<unsigned>(min(extent - 1 - origin, T - 1));
            ld2     = static_cast<unsigned>(2 * ld);
            base    = reinterpret_cast<const char*>(m + (size_t)origin * ld);
        }
    }
    // DMA j (0 .. T / 32 - 1) of this wave for stage st into the stage buffer at LDS byte address lds.
    __device__ __forceinline__ void dma(int st, int j, unsigned lds, int wave) const {
        if constexpr (TR) {
            dma_1k(voff, base + ((size_t)st * kStageK + 4 * kRpd * j) * ld * 2, lds + (wave + 4 * j) * 1024);
        } else {
            // Row 32 j + r8 of the tile, clamped to the matrix (255 * ld2 < 2^32).
            const unsigned row = min(r8 + 32u * j, last);
            dma_1k(row * ld2 + chunk16, base + (size_t)st * kStageK * 2, lds + (wave + 4 * j) * 1024);
        }
    }
    // What DMA j of stage st would write to the stage buffer `stage`, by an ordinary load and LDS
    // store, with zeros for the lanes whose k (within the stage) is k_left or more: the partial last
    // stage of a k tail.  Those lanes load nothing (their address may lie past the matrix).
    __device__ __forceinline__ void fill(int st, int j, u16* stage, int wave, int lane, int k_left) const {
        const char* src;
        bool ok;
        if constexpr (TR) {
            ok  = kRpd * (wave + 4 * j) + lane / kCpr < k_left;
            src = base + ((size_t)st * kStageK + 4 * kRpd * j) * ld * 2 + voff;
        } else {
            ok  = int(chunk16 / 2) < k_left;  // the chunk's first k; k is a multiple of 8
            src = base + (size_t)st * kStageK * 2 + min(r8 + 32u * j, last) * ld2 + chunk16;
        }
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (ok) v = *reinterpret_cast<const u32x4*>(src);
        *reinterpret_cast<u32x4*>(reinterpret_cast<char*>(stage) + (wave + 4 * j) * 1024 + 16 * lane) = v;
    }
};

// What the DMA pipeline reads when k holds no whole stage (its data is discarded): operands
// initialised on it with a leading dimension of 0 keep every lane's offset within 512 bytes.
static __device__ __attribute__((aligned(256))) u16 dma_dummy[512];

// Output tile `bid` of p (tile_of order), k split z when SPLIT; the whole workgroup calls it.
// T: tile size (256: waves of 128x128, one workgroup per CU; 128: waves of 64x64, two per CU).
// SPLIT: the workgroup reduces k range [z k_chunk, (z + 1) k_chunk) and stores its raw fp32 sums
// to slice z of p.d (dense m x n); the reduction kernel forms d.
// BM: tile rows (T by default; 64 with T = 128 for m of at most 64, row-major a only).
// PF: stages of b to prefetch into L2 ahead of the stage being staged (0: none), for a b larger
// than the MALL, whose stages otherwise arrive from HBM later than the DMA lead covers.
// NB: stage buffers (2, or 3 for a ring in which each stage's DMAs run two stages ahead of its use).
template <bool BF16, bool TA, bool TB, int T = 256, bool SPLIT = false, int BM = T, int PF = 0, int NB = 2>
// band: tile rows per band of the tile order (tile_of).
__device__ __forceinline__ void half_gemm_dma_tile(const HalfGemmParams& p, int bid, int z = 0, int band = 8) {
    constexpr bool A_TR = TA, B_TR = !TB;
    static_assert(BM == T || (BM == 64 && !TA), "64-row tiles take row-major a");
    constexpr int NBM = BM / 64, NBN = T / 64;  // 32x32 blocks per wave row / column
    constexpr int NDA = BM / 32, NDB = T / 32;  // DMAs per wave per stage: A, B
    constexpr int kStageA = BM * kStageK, kStageB = T * kStageK;  // one operand, one stage
    __shared__ __attribute__((aligned(1024))) u16 As0[kStageA];
    __shared__ __attribute__((aligned(1024))) u16 Bs0[kStageB];
    __shared__ __attribute__((aligned(1024))) u16 As1[kStageA];
    __shared__ __attribute__((aligned(1024))) u16 Bs1[kStageB];
    static_assert(NB == 2 || (NB == 3 && PF == 0), "a three-buffer ring takes no prefetch");
    __shared__ __attribute__((aligned(1024))) u16 As2[NB > 2 ? kStageA : 8];
    __shared__ __attribute__((aligned(1024))) u16 Bs2[NB > 2 ? kStageB : 8];
    const int tid = threadIdx.x, lane = tid & 63, li = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wrow = (wave >> 1) * (BM / 2), wcol = (wave & 1) * (T / 2);
    int tm, tn;
    tile_of(bid, p.tiles_m, p.tiles_n, tm, tn, band);
    const int m0 = tm * BM, n0 = tn * T;
    const int M = p.m, N = p.n;
    const int kbeg = SPLIT ? z * p.k_chunk : 0;
    const int kend = SPLIT ? min(p.k, kbeg + p.k_chunk) : p.k;
    // Whole stages go through the DMA pipeline; a partial last one (k_tail) is staged afterwards.
    const int nst    = (kend - kbeg) / kStageK;
    const int k_tail = (kend - kbeg) - nst * kStageK;

    // A split's operands start at k = kbeg: a k-contiguous operand's rows advance by kbeg
    // elements, a transposed one's by kbeg rows.
    const u16* const pa = static_cast<const u16*>(p.a) + (A_TR ? (size_t)kbeg * p.lda : (size_t)kbeg);
    const u16* const pb = static_cast<const u16*>(p.b) + (B_TR ? (size_t)kbeg * p.ldb : (size_t)kbeg);
    Operand<A_TR, BM> opa;
    Operand<B_TR, T> opb;
    opa.init(pa, p.lda, m0, M, wave, lane);
    opb.init(pb, p.ldb, n0, N, wave, lane);
    // Last stage index the DMAs clamp to; with no whole stage the pipeline runs on the dummy.
    const int last_st = nst > 0 ? nst - 1 : 0;
    if (nst == 0) {
        opa.init(dma_dummy, 0, 0, BM, wave, lane);
        opb.init(dma_dummy, 0, 0, T, wave, lane);
    }
    // L2 prefetch of b: one DMA per wave per stage, each lane touching one 128-byte line of the
    // stage's b tile (256 lines at T = 256), into a 1 KiB sink per wave that nothing reads.  Lines
    // past the matrix are clamped onto its last column (row-major b) or column (column-major b).
    __shared__ __attribute__((aligned(1024))) u16 pf_sink[PF ? 4 * 512 : 8];
    const unsigned lsink = (unsigned)(uintptr_t)(__attribute__((address_space(3))) u16*)pf_sink + wave * 1024;
    unsigned pf_voff    = 0;
    const char* pf_base = nullptr;
    if constexpr (PF > 0) {
        static_assert(T == 256, "prefetch lines cover a 256-column stage");
        const int L = wave * 64 + lane;
        if constexpr (B_TR) {  // row-major b: 64 k rows x T columns, T / 64 lines per row
            constexpr int LPR = T / 64;
            const int krow = L / LPR, line = L % LPR;
            pf_voff = static_cast<unsigned>((krow * p.ldb + (min(n0 + 64 * line, N - 8) - n0)) * 2);
            pf_base = reinterpret_cast<const char*>(pb + n0);
        } else {  // column-major b: T columns of 64 k, one line each
            pf_voff = static_cast<unsigned>((min(n0 + L, N - 1) - n0) * p.ldb * 2);
            pf_base = reinterpret_cast<const char*>(pb + (size_t)n0 * p.ldb);
        }
        if (nst == 0) {  // every prefetch then reads stage 0 of the dummy
            pf_voff = 0;
            pf_base = reinterpret_cast<const char*>(dma_dummy);
        }
    }
    auto prefetch = [&](int st) {
        if constexpr (PF > 0) {
            const size_t step = B_TR ? (size_t)kStageK * p.ldb * 2 : (size_t)kStageK * 2;
            dma_1k(pf_voff, pf_base + (size_t)st * step, lsink);
        }
    };
    const unsigned la0 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) u16*)As0;
    const unsigned lb0 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) u16*)Bs0;
    const unsigned la1 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) u16*)As1;
    const unsigned lb1 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) u16*)Bs1;
    const unsigned la2 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) u16*)As2;
    const unsigned lb2 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) u16*)Bs2;

    // Operand of k-step ks (0..3 in the stage) for rows (or columns) x .. x + 31.
    const int tr_k = (lane & 15) >> 2, tr_x = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    auto rd_k = [&](const u16* S, int x, int ks) {  // k-contiguous
        const int row = x + li, pos = (2 * ks + h) ^ ((row >> 1) & 7);
        return *reinterpret_cast<const u32x4*>(S + row * kStageK + 8 * pos);
    };
    // Transposed: within each 16 lanes, lane 4j + e reads elements x + tr_x .. + 3 of k row kk + j;
    // lane 4e + i receives element i of lanes e, 4 + e, 8 + e, 12 + e, i.e. 4 consecutive k of
    // column x + lane % 32.  Part `part` covers k 16 ks + 8 h + 4 part .. + 3.
    // W: the stage's row length (the operand's tile extent).
    auto rd_t = [&](const u16* S, int x, int ks, int part, auto w_tag) {
        constexpr int W = decltype(w_tag)::value;
        const int k = 16 * ks + 8 * h + 4 * part + tr_k, n = x + tr_x;
        const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_v4i16*)(S + k * W + 8 * ((n >> 3) ^ (4 * (k & 3))) + (n & 7)));
        return __builtin_bit_cast(u32x2, v);
    };

    floatx16 acc[NBM][NBN];
#pragma unroll
    for (int i = 0; i < NBM; ++i)
#pragma unroll
        for (int j = 0; j < NBN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // Operands of one half stage (32 k): [k-step][block].
    u32x4 fa0[2][NBM], fb0[2][NBN], fa1[2][NBM], fb1[2][NBN];
    constexpr int NRA = (A_TR ? 4 : 2) * NBM, NRB = (B_TR ? 4 : 2) * NBN, NR = NRA + NRB;
    constexpr int NM = 2 * NBM * NBN;  // MFMAs per half stage
    constexpr int ND = NDA + NDB;      // DMAs per wave per stage
    // DMA d (0 .. ND - 1) of a stage: A and B alternate while both have some left.
    auto dma_one = [&](int st, int d, unsigned la, unsigned lb) {
        constexpr int PAIRS = NDA < NDB ? NDA : NDB;
        if (d < 2 * PAIRS) {
            if (d & 1)
                opb.dma(st, d >> 1, lb, wave);
            else
                opa.dma(st, d >> 1, la, wave);
        } else if (NDA > NDB) {
            opa.dma(st, d - PAIRS, la, wave);
        } else {
            opb.dma(st, d - PAIRS, lb, wave);
        }
    };
    // LDS read r (0 .. NR-1) of half `hf`, ordered k-step major (A then B within a k-step), into (ga, gb).
    auto read_one = [&](u32x4 (&ga)[2][NBM], u32x4 (&gb)[2][NBN], const u16* As, const u16* Bs, int hf, int r) {
        const int s = r / (NR / 2), q = r % (NR / 2), ks = 2 * hf + s;
        if (q < NRA / 2) {
            if constexpr (A_TR) {
                const u32x2 v = rd_t(As, wrow + 32 * (q >> 1), ks, q & 1, std::integral_constant<int, BM>{});
                ga[s][q >> 1][2 * (q & 1)]     = v[0];
                ga[s][q >> 1][2 * (q & 1) + 1] = v[1];
            } else {
                ga[s][q] = rd_k(As, wrow + 32 * q, ks);
            }
        } else {
            const int u = q - NRA / 2;
            if constexpr (B_TR) {
                const u32x2 v = rd_t(Bs, wcol + 32 * (u >> 1), ks, u & 1, std::integral_constant<int, T>{});
                gb[s][u >> 1][2 * (u & 1)]     = v[0];
                gb[s][u >> 1][2 * (u & 1) + 1] = v[1];
            } else {
                gb[s][u] = rd_k(Bs, wcol + 32 * u, ks);
            }
        }
    };
    // NM MFMAs on (fa, fb) (k-step major, then block row, block column); the NR reads of half hf
    // of (As, Bs) into (ga, gb) and, with a true with_dma, the ND DMAs of stage dma_st into (la,
    // lb) (A and B alternating) are spread between them in a fixed order.
    auto run_half = [&](u32x4 (&fa)[2][NBM], u32x4 (&fb)[2][NBN], u32x4 (&ga)[2][NBM], u32x4 (&gb)[2][NBN],
                        const u16* As, const u16* Bs, int hf, auto with_dma, int dma_st, unsigned la, unsigned lb) {
#pragma unroll
        for (int t = 0; t < NM; ++t) {
            const int s = t / (NBM * NBN), bi = (t / NBN) % NBM, bj = t % NBN;
            acc[bi][bj] = mfma<BF16>(fa[s][bi], fb[s][bj], acc[bi][bj]);
#pragma unroll
            for (int r = 0; r < NR; ++r)
                if ((r * NM) / NR == t) read_one(ga, gb, As, Bs, hf, r);
            if constexpr (decltype(with_dma)::value) {
#pragma unroll
                for (int d = 0; d < ND; ++d)
                    if (((2 * d + 1) * NM) / (2 * ND) == t) dma_one(dma_st, d, la, lb);
                // After the stage's last DMA: the prefetch is always the latest memory instruction.
                if (PF > 0 && t == NM - 1) prefetch(min(dma_st + PF, last_st));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto read_half = [&](u32x4 (&ga)[2][NBM], u32x4 (&gb)[2][NBN], const u16* As, const u16* Bs, int hf) {
#pragma unroll
        for (int r = 0; r < NR; ++r) read_one(ga, gb, As, Bs, hf, r);
    };

    // Prologue: stages 0 and 1 in flight (ND DMAs per wave each), with prefetch stages 2 .. PF + 1
    // too; wait for stage 0.  Each wait below then leaves exactly one instruction pending, the
    // latest prefetch (memory instructions complete in issue order for the counter).  With no whole
    // stage it reads the dummy.
#pragma unroll
    for (int d = 0; d < ND; ++d) dma_one(0, d, la0, lb0);
#pragma unroll
    for (int i = 2; i <= PF; ++i) prefetch(min(i, last_st));
    const int st1 = min(1, last_st);
#pragma unroll
    for (int d = 0; d < ND; ++d) dma_one(st1, d, la1, lb1);
    prefetch(min(1 + PF, last_st));
    if constexpr (NB == 3) {
        const int st2 = min(2, last_st);
#pragma unroll
        for (int d = 0; d < ND; ++d) dma_one(st2, d, la2, lb2);
    }
    static_assert((NB - 1) * ND + PF <= 63, "the wait count field holds 63");
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NB - 1) * ND + PF) : "memory");
    read_half(fa0, fb0, As0, Bs0, 0);

    // Stages past the last reload the last one (harmless: nothing reads them).
#define FT_DMA_PHASE(XA, XB, YA, YB, LXA, LXB, ST)                               \
    run_half(fa0, fb0, fa1, fb1, XA, XB, 1, std::false_type{}, 0, 0u, 0u);                          \
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(PF > 0 ? 1 : 0) : "memory"); \
    run_half(fa1, fb1, fa0, fb0, YA, YB, 0, std::true_type{}, min((ST) + 2, last_st), LXA, LXB);
    // Ring: the wait for the next stage leaves the one after it in flight, and the freed buffer
    // takes the stage three ahead.
#define FT_RING_PHASE(XA, XB, YA, YB, LXA, LXB, ST)                                                  \
    run_half(fa0, fb0, fa1, fb1, XA, XB, 1, std::false_type{}, 0, 0u, 0u);                          \
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(ND) : "memory");   \
    run_half(fa1, fb1, fa0, fb0, YA, YB, 0, std::true_type{}, min((ST) + 3, last_st), LXA, LXB);
    int st = 0;
    if constexpr (NB == 2) {
        for (; st + 1 < nst; st += 2) {
            FT_DMA_PHASE(As0, Bs0, As1, Bs1, la0, lb0, st)
            FT_DMA_PHASE(As1, Bs1, As0, Bs0, la1, lb1, st + 1)
        }
        // An odd stage count ends with one more stage in buffer 0 (a separate copy: leaving the
        // loop between its two phases costs the register allocator the fragment double buffer).
        if (st < nst) {
            FT_DMA_PHASE(As0, Bs0, As1, Bs1, la0, lb0, st)
        }
    } else {
        for (; st + 2 < nst; st += 3) {
            FT_RING_PHASE(As0, Bs0, As1, Bs1, la0, lb0, st)
            FT_RING_PHASE(As1, Bs1, As2, Bs2, la1, lb1, st + 1)
            FT_RING_PHASE(As2, Bs2, As0, Bs0, la2, lb2, st + 2)
        }
        if (st < nst) {
            FT_RING_PHASE(As0, Bs0, As1, Bs1, la0, lb0, st)
        }
        if (st + 1 < nst) {
            FT_RING_PHASE(As1, Bs1, As2, Bs2, la1, lb1, st + 1)
        }
    }
#undef FT_RING_PHASE
#undef FT_DMA_PHASE
    // The workgroup's LDS must not be released with a DMA still writing it.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // k tail: the partial last stage is staged into buffer 0 by ordinary loads (zeros past kend),
    // once every wave has finished reading the buffers, then multiplied like a whole stage.
    if (k_tail > 0) {
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        opa.init(pa, p.lda, m0, M, wave, lane);
        opb.init(pb, p.ldb, n0, N, wave, lane);
#pragma unroll
        for (int j = 0; j < NDA; ++j) opa.fill(nst, j, As0, wave, lane, k_tail);
#pragma unroll
        for (int j = 0; j < NDB; ++j) opb.fill(nst, j, Bs0, wave, lane, k_tail);
        __syncthreads();
        read_half(fa0, fb0, As0, Bs0, 0);
        run_half(fa0, fb0, fa1, fb1, As0, Bs0, 1, std::false_type{}, 0, 0u, 0u);
        run_half(fa1, fb1, fa0, fb0, As0, Bs0, 0, std::false_type{}, 0, 0u, 0u);
    }

    // Epilogue through buffer loads and stores relative to the tile's corner.  The byte offset of
    // an element splits into a per-lane part (4 h rows and lane column li) in the VGPR offset and
    // a wave-uniform part (block, register) in the scalar offset.  An element outside the matrix
    // (edge tiles: a grouped GEMM's last rows, any m or n not a multiple of 256) gets the lane
    // offset 2^31, past the buffer's size (at most 2^31 - 1 bytes), so its c load returns 0 and
    // its store is dropped by the hardware range check: no branches, one copy for whole and edge
    // tiles.  ldc, ldd below 2^21 (checked on the host) keep every sum below 2^32.
    const float alpha = p.alpha, beta = p.beta;
    auto epilogue = [&](auto c_tag, auto half_tag) {
        constexpr bool HAS_C = decltype(c_tag)::value;
        constexpr bool HALF  = decltype(half_tag)::value;
        constexpr unsigned ES = HALF ? 2 : 4;
        // Split-k: raw fp32 sums to slice z of the workspace (dense m x n).
        const uint64_t ldd64 = SPLIT ? (uint64_t)N : (uint64_t)p.ldd;
        char* const dcorner = SPLIT ? reinterpret_cast<char*>(static_cast<float*>(p.d) + (size_t)z * M * N +
                                                              (size_t)m0 * N + n0)
                                    : static_cast<char*>(p.d) + ((size_t)m0 * p.ldd + n0) * ES;
        const unsigned ldd = static_cast<unsigned>(ldd64), ldc = static_cast<unsigned>(p.ldc);
        const int rows_left = M - m0, cols_left = N - n0;
        auto span = [&](uint64_t ld) {  // bytes from the tile's corner to the matrix's last element
            const uint64_t b = ((uint64_t)(rows_left - 1) * ld + (uint64_t)cols_left) * ES;
            return static_cast<int>(b < 0x7FFFFFFFull ? b : 0x7FFFFFFFull);
        };
        const __amdgpu_buffer_rsrc_t dres = __builtin_amdgcn_make_buffer_rsrc(dcorner, 0, span(ldd64), kBufferConfig);
        __amdgpu_buffer_rsrc_t cres = dres;
        if constexpr (HAS_C)
            cres = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<char*>(static_cast<const char*>(p.c)) + ((size_t)m0 * p.ldc + n0) * ES, 0, span(p.ldc),
                kBufferConfig);
        const unsigned lane_d = (4 * h * ldd + li) * ES, lane_c = (4 * h * ldc + li) * ES;
        constexpr unsigned kOut = 0x80000000u;
#pragma unroll
        for (int bi = 0; bi < NBM; ++bi)
#pragma unroll
            for (int bj = 0; bj < NBN; ++bj) {
                const int col    = wcol + 32 * bj;  // wave-uniform block column
                const bool colok = col + li < cols_left;
                float cv[16];
                if constexpr (HAS_C) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row0 = wrow + 32 * bi + 8 * (r / 4) + (r % 4);  // row of lane half 0
                        const bool ok  = colok && 4 * h < rows_left - row0;
                        const int so   = static_cast<int>((row0 * ldc + col) * ES);
                        if constexpr (HALF)
                            cv[r] = to_float<BF16>(
                                static_cast<u16>(__builtin_amdgcn_raw_buffer_load_b16(cres, ok ? lane_c : kOut, so, 0)));
                        else
                            cv[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(cres, ok ? lane_c : kOut, so, 0));
                    }
                }
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row0 = wrow + 32 * bi + 8 * (r / 4) + (r % 4);
                    const bool ok  = colok && 4 * h < rows_left - row0;
                    const int so   = static_cast<int>((row0 * ldd + col) * ES);
                    float out      = SPLIT ? acc[bi][bj][r] : alpha * acc[bi][bj][r];
                    if constexpr (HAS_C) out += beta * cv[r];
                    // Non-temporal (aux 2): d is not read again here.
                    if constexpr (HALF)
                        __builtin_amdgcn_raw_buffer_store_b16(from_float<BF16>(out), dres, ok ? lane_d : kOut, so, 2);
                    else
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, out), dres, ok ? lane_d : kOut,
                                                              so, 2);
                }
            }
    };
    if constexpr (SPLIT) {
        epilogue(std::false_type{}, std::false_type{});
    } else if (p.c != nullptr) {
        if (p.cd_half)
            epilogue(std::true_type{}, std::true_type{});
        else
            epilogue(std::true_type{}, std::false_type{});
    } else {
        if (p.cd_half)
            epilogue(std::false_type{}, std::true_type{});
        else
            epilogue(std::false_type{}, std::false_type{});
    }
}

template <bool BF16, bool TA, bool TB, int PF = 0>
__global__ __launch_bounds__(256, 1) void half_gemm_dma(HalfGemmParams p) {
    half_gemm_dma_tile<BF16, TA, TB, 256, false, 256, PF>(p, blockIdx.x);
}

// 128x128 tiles, two workgroups per CU, whole-k or split-k.  Split-k workgroups are renumbered so
// each XCD runs whole k splits (hardware ids go to the XCDs in turn, x fastest).
template <bool BF16, bool TA, bool TB, bool SPLIT>
__global__ __launch_bounds__(256, 2) void half_gemm_dma128(HalfGemmParams p) {
    int bid = blockIdx.x, z = blockIdx.z;
    if constexpr (SPLIT) {
        const int tiles = gridDim.x, total = tiles * gridDim.z;
        if ((total & 7) == 0) {
            const int lin = blockIdx.x + tiles * blockIdx.z;
            const int w   = (lin & 7) * (total >> 3) + (lin >> 3);
            z             = w / tiles;
            const int t   = w - z * tiles, per = tiles >> 3;
            bid           = t < (per << 3) ? ((t % per) << 3) + t / per : t;
        }
    }
    half_gemm_dma_tile<BF16, TA, TB, 128, SPLIT>(p, bid, z);
}

// 64x128 split-k tiles for m of at most 64 (a 128-row tile would stage and multiply 64 rows of
// clamped copies): waves of 32x64, row-major a.  Measured on MI355X, 64x4096x4096 bf16 at 8
// splits: 6.7 us for the GEMM kernel against 8.0 us on the 128x128 split tile.  Three stage
// buffers (72 KiB, still two workgroups per CU), each stage's DMAs issued two stages ahead:
// 12.2 / 11.6 us per step with row- / column-major b against 12.8 / 12.3 with two.
template <bool BF16, bool TB>
__global__ __launch_bounds__(256, 2) void half_gemm_dma64x128(HalfGemmParams p) {
    int bid = blockIdx.x, z = blockIdx.z;
    const int tiles = gridDim.x, total = tiles * gridDim.z;
    if ((total & 7) == 0) {
        const int lin = blockIdx.x + tiles * blockIdx.z;
        const int w   = (lin & 7) * (total >> 3) + (lin >> 3);
        z             = w / tiles;
        const int t   = w - z * tiles, per = tiles >> 3;
        bid           = t < (per << 3) ? ((t % per) << 3) + t / per : t;
    }
    half_gemm_dma_tile<BF16, false, TB, 128, true, 64, 0, 3>(p, bid, z);
}

// Grouped GEMM over a device table of per-group parameters: the workgroup's
// group is the last one whose first tile id is at most its own.  Group starts
// are multiples of 8, so the group-local id keeps the hardware id's XCD;
// ids past the group's tiles are padding and exit at once (before any
// barrier, the whole workgroup).
template <bool BF16, bool TA, bool TB, int T = 256, int PF = 0>
__global__ __launch_bounds__(256, 256 / T) void grouped_half_gemm_dma(GroupedHalfArgs g) {
    const int bid = blockIdx.x;
    int lo = 0, hi = g.groups - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (g.tile_start[mid] <= bid)
            lo = mid;
        else
            hi = mid - 1;
    }
    const HalfGemmParams p = g.params[lo];
    const int local        = bid - g.tile_start[lo];
    if (local >= p.tiles_m * p.tiles_n) return;
    // One band per group when the group has at most kGroupBand tile rows: each group has a b of its
    // own, which bands of 8 rows fetched once per band (8 MoE experts of 4 to 13 tile rows: 1.5x
    // the b bytes of one band per expert).  With the L2 prefetch of b those re-reads are cheap and
    // bands of 8 rows, which re-read less of a, are faster (8 experts, 940 MB of weights: 1.638
    // against 1.662 ms).
    const int band = PF > 0 ? 8 : p.tiles_m <= kGroupBand ? p.tiles_m : 8;
    half_gemm_dma_tile<BF16, TA, TB, T, false, T, PF>(p, local, 0, band);
}

// Kernel for one input type, tile size and operand orientation (ta: column-major a, tb:
// column-major b).
template <bool BF16, int T = 256, int PF = 0>
const void* groupedDmaKernel(bool ta, bool tb) {
    if (ta) return tb ? reinterpret_cast<const void*>(&grouped_half_gemm_dma<BF16, true, true, T, PF>)
                      : reinterpret_cast<const void*>(&grouped_half_gemm_dma<BF16, true, false, T, PF>);
    return tb ? reinterpret_cast<const void*>(&grouped_half_gemm_dma<BF16, false, true, T, PF>)
              : reinterpret_cast<const void*>(&grouped_half_gemm_dma<BF16, false, false, T, PF>);
}
template <bool BF16, bool SPLIT>
const void* dma128Kernel(bool ta, bool tb) {
    if (ta) return tb ? reinterpret_cast<const void*>(&half_gemm_dma128<BF16, true, true, SPLIT>)
                      : reinterpret_cast<const void*>(&half_gemm_dma128<BF16, true, false, SPLIT>);
    return tb ? reinterpret_cast<const void*>(&half_gemm_dma128<BF16, false, true, SPLIT>)
              : reinterpret_cast<const void*>(&half_gemm_dma128<BF16, false, false, SPLIT>);
}
template <bool BF16>
const void* dma64x128Kernel(bool ta, bool tb) {
    if (ta) return nullptr;
    return tb ? reinterpret_cast<const void*>(&half_gemm_dma64x128<BF16, true>)
              : reinterpret_cast<const void*>(&half_gemm_dma64x128<BF16, false>);
}
// Stages of b a large-b launch prefetches ahead (measured: 2048x114688x4096 bf16 1508-1512 us at 4,
// 1517-1530 at 2, 1620-1633 without).
constexpr int kLargeBPrefetch = 4;
template <bool BF16, int PF = 0>
const void* dmaKernelFor(bool ta, bool tb) {
    if (ta) return tb ? reinterpret_cast<const void*>(&half_gemm_dma<BF16, true, true, PF>)
                      : reinterpret_cast<const void*>(&half_gemm_dma<BF16, true, false, PF>);
    return tb ? reinterpret_cast<const void*>(&half_gemm_dma<BF16, false, true, PF>)
              : reinterpret_cast<const void*>(&half_gemm_dma<BF16, false, false, PF>);
}
template <bool BF16>
const void* dmaKernel(bool ta, bool tb, bool prefetch_b) {
    return prefetch_b ? dmaKernelFor<BF16, kLargeBPrefetch>(ta, tb) : dmaKernelFor<BF16>(ta, tb);
}

}  // namespace ftrain::gemm::ddev
