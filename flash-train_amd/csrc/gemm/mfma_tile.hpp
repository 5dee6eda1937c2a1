// The FP32 MFMA tile kernel template, shared by the per-layout HIP
// translation units (kernels.hip instantiates the row-major a and b case,
// kernels_layout_*.hip the transposed ones).  Device code only.
//
// Replaces the reference's single SIMT kernel
// (src/primitive/hygon/gemm/fp32_gemm.hip:18-31) for the MFMA variants.
//
// MFMA operand/result layout used below (v_mfma_f32_32x32x2_f32, one block):
//   A operand: lane l holds A[row = l % 32][kk = l / 32]
//   B operand: lane l holds B[kk = l / 32][col = l % 32]
//   result   : lane l, register r holds D[row = 8*(r/4) + 4*(l/32) + r%4][col = l % 32]
// The two reduction slots kk = 0, 1 may carry any two k indices as long as
// A and B agree; here lane half h = l/32 walks k = h*BK/2 + s for step s.
// With a row-major (k-contiguous) A tile in LDS each lane then fetches its A
// values for four steps with one 128-bit LDS read.
//
// Column interleave: inside a wave tile made of TN 32-column MFMA blocks,
// block bj / MFMA column j maps to tile column j*TN + bj.  A lane then owns TN
// adjacent output columns per row, so the epilogue's c loads and d stores
// are TN-wide vectors.
//
// Operand layouts (template flags TA, TB):
//   TA = false: a[r][k] at a[r*lda + k]  (row-major, k contiguous)
//   TA = true : a[r][k] at a[k*lda + r]  (column-major, r contiguous)
//   TB = false: b[k][c] at b[k*ldb + c]  (row-major, c contiguous)
//   TB = true : b[k][c] at b[c*ldb + k]  (column-major, k contiguous)
// Each layout is staged in LDS with its contiguous dimension innermost, so
// the 128-bit global loads become 128-bit LDS writes:
//   A tile: TA ? [BK][BM + 4] : [BM][BK + 4]
//   B tile: TB ? [BN][BK + 4] : [BK][BN + 4]
// The operand reads then differ: an [BM][BK+4] A tile gives four steps per
// 128-bit read, a [BK][BM+4] one a 32-bit read per step (consecutive lanes,
// consecutive rows: conflict free); a [BK][BN+4] B tile gives the TN
// adjacent columns of one step per read, a [BN][BK+4] one four steps of one
// column per 128-bit read.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "ft/gemm_kernels.hpp"

namespace ftrain::gemm::dev {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

template <int N>
struct VecOf;
template <>
struct VecOf<1> {
    using type = float;
};
template <>
struct VecOf<2> {
    using type = floatx2;
};
template <>
struct VecOf<4> {
    using type = floatx4;
};

__device__ __forceinline__ float lane_of(float v, int) { return v; }
__device__ __forceinline__ float lane_of(floatx2 v, int i) { return v[i]; }
__device__ __forceinline__ float lane_of(floatx4 v, int i) { return v[i]; }
__device__ __forceinline__ void set_lane(float& v, int, float x) { v = x; }
template <typename V>
__device__ __forceinline__ void set_lane(V& v, int i, float x) {
    v[i] = x;
}

// Maps a linear workgroup id to an output tile.  Workgroups are dispatched
// round-robin over the 8 XCDs (each with its own L2), so consecutive ids
// land on different XCDs; the first step regroups ids so that each XCD
// receives a contiguous range of logical tiles.  The second step walks those
// tiles in column sweeps over bands of 8 tile rows, so the tiles resident on
// one XCD share A row-panels and B column-panels in its L2.
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int tiles = tiles_m * tiles_n;
    const int per   = tiles >> 3;
    int t           = bid;
    if (bid < (per << 3)) t = (bid & 7) * per + (bid >> 3);
    constexpr int kBand  = 8;
    const int band_span  = kBand * tiles_n;
    const int band       = t / band_span;
    const int first_m    = band * kBand;
    const int band_rows  = min(tiles_m - first_m, kBand);
    const int within     = t - band * band_span;
    tm                   = first_m + within % band_rows;
    tn                   = within / band_rows;
}

enum SplitMode : int { kWhole = 0, kPartial = 2 };

// ----------------------------------------------------------------------------
// MFMA tile kernel.
//   BM x BN output tile per workgroup, BK reduction depth per stage, WM x WN
//   waves, each wave owning a (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA
//   blocks; MINB workgroups per CU bound the register budget.  VEC: 128-bit
//   global loads/stores along each matrix's contiguous dimension (the caller
//   guarantees 16-byte aligned bases, leading dimensions and contiguous
//   extents that are multiples of 4, and n % 4 == 0).  SPLIT selects the
//   epilogue:
//     kWhole   - this workgroup owns the whole reduction: d = alpha*acc + beta*c;
//     kPartial - it reduces [z*k_chunk, z*k_chunk + k_chunk) and stores the raw
//                partial tile to slice z of the workspace p.d (z*m*n floats,
//                dense m x n); splitk_reduce
//                then forms d = alpha * sum_z(partial_z) + beta*c in fixed z
//                order.
//
// Pipeline (NBUF LDS buffers, stage s in buffer s % NBUF).  With three
// buffers, iteration s:
//   1. read the operands of stage s+1 from LDS into the spare register set
//      (its data became visible at the previous barrier);
//   2. first half of stage s's MFMAs (operands already in registers);
//   3. write stage s+2 (global loads issued one iteration earlier) to LDS;
//   4. issue the global loads of stage s+3;
//   5. second half of the MFMAs;
//   6. one barrier.
// The MFMA stream therefore never waits on an LDS read issued in the same
// stage, and a buffer is rewritten only after the barrier that follows its
// last read.  Interior tiles (no m/n edge, whole stages) take a copy of the
// loop without bounds checks.
// ----------------------------------------------------------------------------
// The tile body: output tile number `bid` of p's tile grid, split `z` of
// the reduction (0 when not split).  Wrapped below by the plain kernel (one
// problem: the workgroup's x and z grid indices) and the grouped kernel
// (many problems in one launch).
template <int BM, int BN, int BK, int WM, int WN, int NBUF, int MINB, bool VEC, int SPLIT, bool TA, bool TB>
__device__ __forceinline__ void mfma_gemm_tile(const GemmParams& p, int bid, int z) {
    constexpr int NT  = WM * WN * 64;
    constexpr int WTM = BM / WM;
    constexpr int WTN = BN / WN;
    constexpr int TM  = WTM / 32;
    constexpr int TN  = WTN / 32;
    constexpr int HK  = BK / 2;  // k steps per stage
    // LDS row strides (floats); the +4 spreads rows over banks and keeps
    // every row 16-byte aligned.
    constexpr int SA      = TA ? BM + 4 : BK + 4;
    constexpr int SB      = TB ? BK + 4 : BN + 4;
    constexpr int A_ELEMS = TA ? BK * SA : BM * SA;
    constexpr int B_ELEMS = TB ? BN * SB : BK * SB;
    static_assert(TM >= 1 && TN >= 1 && (TN == 1 || TN == 2 || TN == 4), "wave tile");
    static_assert(BK % 8 == 0, "BK");
    static_assert(NBUF == 2 || NBUF == 3, "two or three LDS stages");
    using BVec = typename VecOf<TN>::type;

    __shared__ __attribute__((aligned(16))) float As[NBUF][A_ELEMS];
    __shared__ __attribute__((aligned(16))) float Bs[NBUF][B_ELEMS];

    const int tid  = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int li   = lane & 31;
    const int h    = lane >> 5;
    const int wrow = (wave / WN) * WTM;
    const int wcol = (wave % WN) * WTN;

    int tm, tn;
    tile_of(bid, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    const int M = p.m, N = p.n, K = p.k;
    const int kbeg = SPLIT != kWhole ? z * p.k_chunk : 0;
    const int kend = SPLIT != kWhole ? min(K, kbeg + p.k_chunk) : K;
    const int nst  = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

    const float* __restrict__ A = p.a;
    const float* __restrict__ B = p.b;
    const size_t lda = p.lda, ldb = p.ldb;

    // Global -> register staging for one stage.
    constexpr int A_LD = VEC ? BM * BK / 4 / NT : BM * BK / NT;
    constexpr int B_LD = VEC ? BK * BN / 4 / NT : BK * BN / NT;
    static_assert(A_LD >= 1 && B_LD >= 1, "tile too small for the workgroup");
    floatx4 ra4[VEC ? A_LD : 1];
    floatx4 rb4[VEC ? B_LD : 1];
    float ra1[VEC ? 1 : A_LD];
    float rb1[VEC ? 1 : B_LD];

    // Element coordinates (tile-local) of staging slot j of this thread.
    // Consecutive threads walk the matrix's contiguous dimension.
    //   A row-major: (r, k) = (idx / (BK/V), V * (idx % (BK/V)))
    //   A col-major: (r, k) = (V * (idx % (BM/V)), idx / (BM/V))
    //   B row-major: (k, c) = (idx / (BN/V), V * (idx % (BN/V)))
    //   B col-major: (k, c) = (V * (idx % (BK/V)), idx / (BK/V))
    constexpr int V = VEC ? 4 : 1;
    auto a_coord = [&](int j, int& r, int& k) {
        const int idx = tid + j * NT;
        if constexpr (TA) {
            r = V * (idx % (BM / V));
            k = idx / (BM / V);
        } else {
            r = idx / (BK / V);
            k = V * (idx % (BK / V));
        }
    };
    auto b_coord = [&](int j, int& k, int& c) {
        const int idx = tid + j * NT;
        if constexpr (TB) {
            k = V * (idx % (BK / V));
            c = idx / (BK / V);
        } else {
            k = idx / (BN / V);
            c = V * (idx % (BN / V));
        }
    };
    // LDS offset of tile element (r, k) of A / (k, c) of B.
    auto a_lds = [&](int r, int k) { return TA ? k * SA + r : r * SA + k; };
    auto b_lds = [&](int k, int c) { return TB ? c * SB + k : k * SB + c; };

    // One wave's operands for one stage: A for HK steps of TM blocks, B for
    // HK steps (TN adjacent columns per lane).
    struct Operands {
        floatx4 a[TM][HK / 4];
        BVec b[HK];
    };

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    auto store_stage = [&](int buf) {
#pragma unroll
        for (int j = 0; j < A_LD; ++j) {
            int r, k;
            a_coord(j, r, k);
            if constexpr (VEC)
                *reinterpret_cast<floatx4*>(&As[buf][a_lds(r, k)]) = ra4[j];
            else
                As[buf][a_lds(r, k)] = ra1[j];
        }
#pragma unroll
        for (int j = 0; j < B_LD; ++j) {
            int k, c;
            b_coord(j, k, c);
            if constexpr (VEC)
                *reinterpret_cast<floatx4*>(&Bs[buf][b_lds(k, c)]) = rb4[j];
            else
                Bs[buf][b_lds(k, c)] = rb1[j];
        }
    };

    auto read_operands = [&](int buf, Operands& o) {
#pragma unroll
        for (int bi = 0; bi < TM; ++bi) {
            const int r = wrow + bi * 32 + li;
#pragma unroll
            for (int q = 0; q < HK / 4; ++q) {
                if constexpr (TA) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) o.a[bi][q][t] = As[buf][(h * HK + 4 * q + t) * SA + r];
                } else {
                    o.a[bi][q] = *reinterpret_cast<const floatx4*>(&As[buf][r * SA + h * HK + 4 * q]);
                }
            }
        }
        if constexpr (TB) {
#pragma unroll
            for (int bj = 0; bj < TN; ++bj)
#pragma unroll
                for (int q = 0; q < HK / 4; ++q) {
                    const floatx4 v =
                        *reinterpret_cast<const floatx4*>(&Bs[buf][(wcol + li * TN + bj) * SB + h * HK + 4 * q]);
#pragma unroll
                    for (int t = 0; t < 4; ++t) set_lane(o.b[4 * q + t], bj, v[t]);
                }
        } else {
#pragma unroll
            for (int s = 0; s < HK; ++s)
                o.b[s] = *reinterpret_cast<const BVec*>(&Bs[buf][(h * HK + s) * SB + wcol + li * TN]);
        }
    };

    auto mfma_steps = [&](const Operands& o, auto first, auto last) {
#pragma unroll
        for (int s = decltype(first)::value; s < decltype(last)::value; ++s)
#pragma unroll
            for (int bi = 0; bi < TM; ++bi)
#pragma unroll
                for (int bj = 0; bj < TN; ++bj)
                    acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x2f32(o.a[bi][s / 4][s % 4], lane_of(o.b[s], bj),
                                                                       acc[bi][bj], 0, 0, 0);
    };

    auto main_loop = [&](auto checked_tag) {
        constexpr bool CHECKED = decltype(checked_tag)::value;
        // m / n index of a load.  The unchecked loop clamps it into the matrix
        // (a vector of `run` elements stays inside): an edge tile then reads
        // valid memory for rows and columns past the edge, whose products
        // land only in outputs the epilogue does not store.  Only a k tail
        // needs the zero-filling checked loop.
        auto row_at = [](int i, int extent, int run) { return CHECKED ? i : min(i, extent - run); };

        // Global address of A(gm, gk) / B(gk, gn).
        auto a_at = [&](int gm, int gk) { return A + (TA ? (size_t)gk * lda + gm : (size_t)gm * lda + gk); };
        auto b_at = [&](int gk, int gn) { return B + (TB ? (size_t)gn * ldb + gk : (size_t)gk * ldb + gn); };

        auto load_stage = [&](int k0) {
#pragma unroll
            for (int j = 0; j < A_LD; ++j) {
                int r, k;
                a_coord(j, r, k);
                const int gm = row_at(m0 + r, M, VEC && TA ? 4 : 1), gk = k0 + k;
                // A vector never straddles an edge: its contiguous extent
                // (k, or m when TA) is a multiple of 4.
                const bool ok = !CHECKED || (gm < M && gk < kend);
                if constexpr (VEC) {
                    ra4[j] = floatx4{0.f, 0.f, 0.f, 0.f};
                    if (ok) ra4[j] = *reinterpret_cast<const floatx4*>(a_at(gm, gk));
                } else {
                    ra1[j] = ok ? *a_at(gm, gk) : 0.f;
                }
            }
#pragma unroll
            for (int j = 0; j < B_LD; ++j) {
                int k, c;
                b_coord(j, k, c);
                const int gk = k0 + k, gn = row_at(n0 + c, N, VEC && !TB ? 4 : 1);
                const bool ok = !CHECKED || (gk < kend && gn < N);
                if constexpr (VEC) {
                    rb4[j] = floatx4{0.f, 0.f, 0.f, 0.f};
                    if (ok) rb4[j] = *reinterpret_cast<const floatx4*>(b_at(gk, gn));
                } else {
                    rb1[j] = ok ? *b_at(gk, gn) : 0.f;
                }
            }
        };

        using Zero = std::integral_constant<int, 0>;
        using Half = std::integral_constant<int, HK / 2>;
        using Full = std::integral_constant<int, HK>;

        if constexpr (NBUF == 3) {
            // Prologue: stages 0 and 1 in LDS, stage 2 in flight.
            if (nst > 0) {
                load_stage(kbeg);
                store_stage(0);
            }
            if (nst > 1) {
                load_stage(kbeg + BK);
                store_stage(1);
            }
            if (nst > 2) load_stage(kbeg + 2 * BK);
            __syncthreads();

            Operands x, y;
            if (nst > 0) read_operands(0, x);

            auto iteration = [&](int st, Operands& cur, Operands& nxt) {
                if (st + 1 < nst) read_operands((st + 1) % NBUF, nxt);
                mfma_steps(cur, Zero{}, Half{});
                if (st + 2 < nst) store_stage((st + 2) % NBUF);
                if (st + 3 < nst) load_stage(kbeg + (st + 3) * BK);
                mfma_steps(cur, Half{}, Full{});
                __syncthreads();
            };

            int st = 0;
            for (; st + 1 < nst; st += 2) {
                iteration(st, x, y);
                iteration(st + 1, y, x);
            }
            if (st < nst) iteration(st, x, y);
        } else {
            // Two LDS stages, one operand set: the stage's operands are read
            // at the top of the iteration (co-resident workgroups cover the
            // read latency), stage s+1 is written mid-stream, stage s+2 loads
            // are issued, one barrier.
            if (nst > 0) {
                load_stage(kbeg);
                store_stage(0);
            }
            if (nst > 1) load_stage(kbeg + BK);
            __syncthreads();
            Operands x;
            for (int st = 0; st < nst; ++st) {
                read_operands(st & 1, x);
                mfma_steps(x, Zero{}, Half{});
                if (st + 1 < nst) store_stage((st + 1) & 1);
                if (st + 2 < nst) load_stage(kbeg + (st + 2) * BK);
                mfma_steps(x, Half{}, Full{});
                __syncthreads();
            }
        }
    };

    if ((kend - kbeg) % BK == 0)
        main_loop(std::false_type{});
    else
        main_loop(std::true_type{});

    // Epilogue.  c and d are row-major with row strides ldc and ldd; the
    // split-k partial slices are dense m x n.
    const float alpha = p.alpha;
    const float beta  = p.beta;
    const float* __restrict__ C = p.c;
    float* __restrict__ D       = p.d;
    const size_t ldc = p.ldc, ldd = p.ldd;
    const int col = n0 + wcol + li * TN;
#pragma unroll
    for (int bi = 0; bi < TM; ++bi) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + wrow + bi * 32 + 8 * (r / 4) + 4 * h + (r % 4);
            if (row >= M) continue;
            const size_t dbase = (size_t)row * ldd + col;
            const size_t cbase = (size_t)row * ldc + col;
            if constexpr (SPLIT == kPartial) {
                float* W           = D + (size_t)z * M * N;
                const size_t pbase = (size_t)row * N + col;
                if constexpr (VEC && TN > 1) {
                    if (col >= N) continue;
                    BVec out;
#pragma unroll
                    for (int bj = 0; bj < TN; ++bj) out[bj] = acc[bi][bj][r];
                    *reinterpret_cast<BVec*>(W + pbase) = out;
                } else {
#pragma unroll
                    for (int bj = 0; bj < TN; ++bj)
                        if (col + bj < N) W[pbase + bj] = acc[bi][bj][r];
                }
            } else if constexpr (VEC) {
                if (col >= N) continue;
                BVec out;
                if constexpr (TN == 1) {
                    out = alpha * acc[bi][0][r] + (C != nullptr ? beta * C[cbase] : 0.f);
                } else {
                    BVec cv;
#pragma unroll
                    for (int bj = 0; bj < TN; ++bj) cv[bj] = 0.f;
                    if (C != nullptr) cv = *reinterpret_cast<const BVec*>(C + cbase);
#pragma unroll
                    for (int bj = 0; bj < TN; ++bj)
                        out[bj] = alpha * acc[bi][bj][r] + (C != nullptr ? beta * cv[bj] : 0.f);
                }
                *reinterpret_cast<BVec*>(D + dbase) = out;
            } else {
#pragma unroll
                for (int bj = 0; bj < TN; ++bj)
                    if (col + bj < N)
                        D[dbase + bj] = alpha * acc[bi][bj][r] + (C != nullptr ? beta * C[cbase + bj] : 0.f);
            }
        }
    }
}

template <int BM, int BN, int BK, int WM, int WN, int NBUF, int MINB, bool VEC, int SPLIT, bool TA, bool TB>
__global__ __launch_bounds__(WM* WN * 64, MINB) void mfma_gemm(GemmParams p) {
    mfma_gemm_tile<BM, BN, BK, WM, WN, NBUF, MINB, VEC, SPLIT, TA, TB>(p, blockIdx.x, blockIdx.z);
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

// Grouped GEMM: the tiles of every group in one launch.  Workgroup bid runs
// tile bid - start[g] of group g, whose parameters (pointers, shape, leading
// dimensions, tile grid) sit in a device table.
template <int BM, int BN, int BK, int WM, int WN, int NBUF, int MINB, bool VEC, bool TA, bool TB>
__global__ __launch_bounds__(WM* WN * 64, MINB) void grouped_mfma_gemm(GroupedGemmArgs g) {
    const int bid = blockIdx.x;
    const int grp = find_group(g.tile_start, g.groups, bid);
    const GemmParams p = g.params[grp];
    // Group starts are multiples of 8, so the group-local id keeps the
    // hardware id's XCD (id mod 8); ids past the group's tiles are padding.
    const int local = bid - g.tile_start[grp];
    if (local >= p.tiles_m * p.tiles_n) return;
    mfma_gemm_tile<BM, BN, BK, WM, WN, NBUF, MINB, VEC, kWhole, TA, TB>(p, local, 0);
}

// The variants with all four operand layouts instantiated, keyed by the
// Variant they implement.  Used by each layout translation unit.
template <bool TA, bool TB>
const void* layoutKernel(Variant v) {
    switch (v) {
        case Variant::kMfma128x128: return reinterpret_cast<const void*>(&mfma_gemm<128, 128, 16, 2, 2, 2, 3, true, kWhole, TA, TB>);
        case Variant::kMfma128x128S: return reinterpret_cast<const void*>(&mfma_gemm<128, 128, 16, 2, 2, 2, 3, true, kPartial, TA, TB>);
        case Variant::kMfma64x64: return reinterpret_cast<const void*>(&mfma_gemm<64, 64, 16, 2, 2, 3, 1, true, kWhole, TA, TB>);
        case Variant::kMfma64x64S: return reinterpret_cast<const void*>(&mfma_gemm<64, 64, 16, 2, 2, 3, 1, true, kPartial, TA, TB>);
        case Variant::kMfma128x128U: return reinterpret_cast<const void*>(&mfma_gemm<128, 128, 16, 2, 2, 3, 1, false, kWhole, TA, TB>);
        case Variant::kMfma128x128US: return reinterpret_cast<const void*>(&mfma_gemm<128, 128, 16, 2, 2, 3, 1, false, kPartial, TA, TB>);
        case Variant::kMfma64x64U: return reinterpret_cast<const void*>(&mfma_gemm<64, 64, 16, 2, 2, 3, 1, false, kWhole, TA, TB>);
        default: return nullptr;
    }
}

// Grouped variants for one orientation: 0 = 128x128 (128-bit loads),
// 1 = 64x64 per-element.
template <bool TA, bool TB>
const void* groupedLayoutKernel(int which) {
    switch (which) {
        case 0: return reinterpret_cast<const void*>(&grouped_mfma_gemm<128, 128, 16, 2, 2, 2, 3, true, TA, TB>);
        case 1: return reinterpret_cast<const void*>(&grouped_mfma_gemm<64, 64, 16, 2, 2, 3, 1, false, TA, TB>);
        default: return nullptr;
    }
}

}  // namespace ftrain::gemm::dev
