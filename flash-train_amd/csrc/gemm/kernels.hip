// FP32 GEMM kernels for MI355X (gfx950 / CDNA4).
//
// Replaces the reference's single SIMT kernel
// (src/primitive/hygon/gemm/fp32_gemm.hip:18-51) with:
//   * MFMA tile kernels built on v_mfma_f32_32x32x2_f32 (a 32x32 fp32 output
//     block per wave-instruction, k = 2 per instruction, 16 accumulator
//     registers per lane), LDS double buffering, 128-bit global loads, an
//     XCD-aware tile order, and a fused alpha/beta epilogue with optional
//     c read; optionally split over k with atomic accumulation;
//   * a streaming split-k kernel for skinny m (GEMV-like, HBM bound);
//   * a general SIMT kernel with 64-bit indexing for shapes the others
//     cannot take;
//   * the elementwise prologue d = beta*c (or 0) used by the split-k paths.
//
// MFMA operand/result layout used below (v_mfma_f32_32x32x2_f32, one block):
//   A operand: lane l holds A[row = l % 32][kk = l / 32]
//   B operand: lane l holds B[kk = l / 32][col = l % 32]
//   result   : lane l, register r holds D[row = 8*(r/4) + 4*(l/32) + r%4][col = l % 32]
// The two reduction slots kk = 0, 1 may carry any two k indices as long as
// A and B agree; here lane half h = l/32 walks k = h*BK/2 + s for step s,
// which lets each lane fetch its A values for four steps with one 128-bit
// LDS read from a row-major (k-contiguous) A tile.
//
// Column interleave: inside a wave tile made of TN 32-column MFMA blocks,
// block bj / MFMA column j maps to tile column j*TN + bj.  A lane then owns TN
// adjacent output columns per row, so B operands come from one TN-wide LDS
// read and the epilogue stores and c loads are TN-wide vectors.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "ft/gemm_kernels.hpp"

namespace ftrain::gemm {
namespace {

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

enum SplitMode : int { kWhole = 0, kAtomic = 1, kPartial = 2 };

// ----------------------------------------------------------------------------
// MFMA tile kernel.
//   BM x BN output tile per workgroup, BK reduction depth per stage, WM x WN
//   waves, each wave owning a (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA
//   blocks; MINB workgroups per CU bound the register budget.  VEC: 128-bit global loads/stores (caller guarantees alignment and
//   k % 4 == n % 4 == 0).  SPLIT selects the epilogue:
//     kWhole   - this workgroup owns the whole reduction: d = alpha*acc + beta*c;
//     kAtomic  - it reduces [z*k_chunk, z*k_chunk + k_chunk) and atomically
//                adds alpha*partial into d, which the prologue kernel set to
//                beta*c (or 0);
//     kPartial - same k range, but the raw partial tile is stored to slice z
//                of the workspace p.d (z*m*n floats); splitk_reduce then forms
//                d = alpha * sum_z(partial_z) + beta*c in fixed z order.
//
// Pipeline (three LDS buffers, stage s in buffer s % 3).  Iteration s:
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
template <int BM, int BN, int BK, int WM, int WN, int NBUF, int MINB, bool VEC, int SPLIT>
__global__ __launch_bounds__(WM* WN * 64, MINB) void mfma_gemm(GemmParams p) {
    constexpr int NT  = WM * WN * 64;
    constexpr int WTM = BM / WM;
    constexpr int WTN = BN / WN;
    constexpr int TM  = WTM / 32;
    constexpr int TN  = WTN / 32;
    constexpr int SA  = BK + 4;  // A tile row stride in LDS (floats); +4 spreads rows over banks
    constexpr int SB  = BN + 4;  // B tile row stride in LDS (floats)
    constexpr int HK  = BK / 2;  // k steps per stage
    static_assert(TM >= 1 && TN >= 1 && (TN == 1 || TN == 2 || TN == 4), "wave tile");
    static_assert(BK % 8 == 0, "BK");
    static_assert(NBUF == 2 || NBUF == 3, "two or three LDS stages");
    using BVec = typename VecOf<TN>::type;

    __shared__ __attribute__((aligned(16))) float As[NBUF][BM * SA];
    __shared__ __attribute__((aligned(16))) float Bs[NBUF][BK * SB];

    const int tid  = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int li   = lane & 31;
    const int h    = lane >> 5;
    const int wrow = (wave / WN) * WTM;
    const int wcol = (wave % WN) * WTN;

    int tm, tn;
    tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    const int M = p.m, N = p.n, K = p.k;
    const int kbeg = SPLIT != kWhole ? blockIdx.z * p.k_chunk : 0;
    const int kend = SPLIT != kWhole ? min(K, kbeg + p.k_chunk) : K;
    const int nst  = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

    const float* __restrict__ A = p.a;
    const float* __restrict__ B = p.b;

    // Global -> register staging for one stage.
    constexpr int A_LD = VEC ? BM * BK / 4 / NT : BM * BK / NT;
    constexpr int B_LD = VEC ? BK * BN / 4 / NT : BK * BN / NT;
    static_assert(A_LD >= 1 && B_LD >= 1, "tile too small for the workgroup");
    floatx4 ra4[VEC ? A_LD : 1];
    floatx4 rb4[VEC ? B_LD : 1];
    float ra1[VEC ? 1 : A_LD];
    float rb1[VEC ? 1 : B_LD];

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
        if constexpr (VEC) {
#pragma unroll
            for (int j = 0; j < A_LD; ++j) {
                const int idx = tid + j * NT;
                *reinterpret_cast<floatx4*>(&As[buf][(idx / (BK / 4)) * SA + 4 * (idx % (BK / 4))]) = ra4[j];
            }
#pragma unroll
            for (int j = 0; j < B_LD; ++j) {
                const int idx = tid + j * NT;
                *reinterpret_cast<floatx4*>(&Bs[buf][(idx / (BN / 4)) * SB + 4 * (idx % (BN / 4))]) = rb4[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < A_LD; ++j) {
                const int idx                       = tid + j * NT;
                As[buf][(idx / BK) * SA + idx % BK] = ra1[j];
            }
#pragma unroll
            for (int j = 0; j < B_LD; ++j) {
                const int idx                       = tid + j * NT;
                Bs[buf][(idx / BN) * SB + idx % BN] = rb1[j];
            }
        }
    };

    auto read_operands = [&](int buf, Operands& o) {
#pragma unroll
        for (int bi = 0; bi < TM; ++bi)
#pragma unroll
            for (int q = 0; q < HK / 4; ++q)
                o.a[bi][q] = *reinterpret_cast<const floatx4*>(&As[buf][(wrow + bi * 32 + li) * SA + h * HK + 4 * q]);
#pragma unroll
        for (int s = 0; s < HK; ++s)
            o.b[s] = *reinterpret_cast<const BVec*>(&Bs[buf][(h * HK + s) * SB + wcol + li * TN]);
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

        auto load_stage = [&](int k0) {
            if constexpr (VEC) {
#pragma unroll
                for (int j = 0; j < A_LD; ++j) {
                    const int idx = tid + j * NT;
                    const int gm = m0 + idx / (BK / 4), gk = k0 + 4 * (idx % (BK / 4));
                    if (CHECKED) {
                        ra4[j] = floatx4{0.f, 0.f, 0.f, 0.f};
                        if (gm < M && gk < kend) ra4[j] = *reinterpret_cast<const floatx4*>(A + (size_t)gm * K + gk);
                    } else {
                        ra4[j] = *reinterpret_cast<const floatx4*>(A + (size_t)gm * K + gk);
                    }
                }
#pragma unroll
                for (int j = 0; j < B_LD; ++j) {
                    const int idx = tid + j * NT;
                    const int gk = k0 + idx / (BN / 4), gn = n0 + 4 * (idx % (BN / 4));
                    if (CHECKED) {
                        rb4[j] = floatx4{0.f, 0.f, 0.f, 0.f};
                        if (gk < kend && gn < N) rb4[j] = *reinterpret_cast<const floatx4*>(B + (size_t)gk * N + gn);
                    } else {
                        rb4[j] = *reinterpret_cast<const floatx4*>(B + (size_t)gk * N + gn);
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < A_LD; ++j) {
                    const int idx = tid + j * NT;
                    const int gm = m0 + idx / BK, gk = k0 + idx % BK;
                    ra1[j]        = (!CHECKED || (gm < M && gk < kend)) ? A[(size_t)gm * K + gk] : 0.f;
                }
#pragma unroll
                for (int j = 0; j < B_LD; ++j) {
                    const int idx = tid + j * NT;
                    const int gk = k0 + idx / BN, gn = n0 + idx % BN;
                    rb1[j]        = (!CHECKED || (gk < kend && gn < N)) ? B[(size_t)gk * N + gn] : 0.f;
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

    const bool interior = m0 + BM <= M && n0 + BN <= N && (kend - kbeg) % BK == 0;
    if (interior)
        main_loop(std::false_type{});
    else
        main_loop(std::true_type{});

    // Epilogue.
    const float alpha = p.alpha;
    const float beta  = p.beta;
    const float* __restrict__ C = p.c;
    float* __restrict__ D       = p.d;
    const int col = n0 + wcol + li * TN;
#pragma unroll
    for (int bi = 0; bi < TM; ++bi) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + wrow + bi * 32 + 8 * (r / 4) + 4 * h + (r % 4);
            if (row >= M) continue;
            const size_t base = (size_t)row * N + col;
            if constexpr (SPLIT == kAtomic) {
#pragma unroll
                for (int bj = 0; bj < TN; ++bj)
                    if (col + bj < N) unsafeAtomicAdd(D + base + bj, alpha * acc[bi][bj][r]);
            } else if constexpr (SPLIT == kPartial) {
                float* W = D + (size_t)blockIdx.z * M * N;
                if constexpr (VEC && TN > 1) {
                    if (col >= N) continue;
                    BVec out;
#pragma unroll
                    for (int bj = 0; bj < TN; ++bj) out[bj] = acc[bi][bj][r];
                    *reinterpret_cast<BVec*>(W + base) = out;
                } else {
#pragma unroll
                    for (int bj = 0; bj < TN; ++bj)
                        if (col + bj < N) W[base + bj] = acc[bi][bj][r];
                }
            } else if constexpr (VEC) {
                if (col >= N) continue;
                BVec out;
                if constexpr (TN == 1) {
                    out = alpha * acc[bi][0][r] + (C != nullptr ? beta * C[base] : 0.f);
                } else {
                    BVec cv;
#pragma unroll
                    for (int bj = 0; bj < TN; ++bj) cv[bj] = 0.f;
                    if (C != nullptr) cv = *reinterpret_cast<const BVec*>(C + base);
#pragma unroll
                    for (int bj = 0; bj < TN; ++bj)
                        out[bj] = alpha * acc[bi][bj][r] + (C != nullptr ? beta * cv[bj] : 0.f);
                }
                *reinterpret_cast<BVec*>(D + base) = out;
            } else {
#pragma unroll
                for (int bj = 0; bj < TN; ++bj)
                    if (col + bj < N)
                        D[base + bj] = alpha * acc[bi][bj][r] + (C != nullptr ? beta * C[base + bj] : 0.f);
            }
        }
    }
}

// ----------------------------------------------------------------------------
// Skinny-m streaming kernel (m <= 8).  Each workgroup covers 256 columns and
// one k range; its 4 waves interleave over the k rows of that range, each
// lane streaming 4 adjacent columns of b.  The waves' partial sums meet in
// LDS; alpha*sum is then added atomically into d (initialised by the
// prologue) or, with PARTIAL, stored raw to slice z of the workspace for
// splitk_reduce.  Bound by the one pass over b.
// ----------------------------------------------------------------------------

template <bool VEC, bool PARTIAL>
__global__ __launch_bounds__(256) void gemv_splitk(GemmParams p) {
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
        const float* brow = B + (size_t)k * N;
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
                const float av = A[(size_t)i * K + k];
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
            if constexpr (PARTIAL)
                p.d[(size_t)blockIdx.z * M * N + (size_t)i * N + col] = s;
            else
                unsafeAtomicAdd(p.d + (size_t)i * N + col, p.alpha * s);
        }
    }
}

// ----------------------------------------------------------------------------
// d = c ? beta * c : 0 (grid-stride, 64-bit).  Initialises the accumulation
// target of the split-k kernels; safe in place (c == d).
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prologue(WideParams p) {
    const uint64_t total  = p.m * p.n;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride)
        p.d[i] = p.c != nullptr ? p.beta * p.c[i] : 0.f;
}

// ----------------------------------------------------------------------------
// Split-k reduction: d = alpha * sum_{z < splits} W[z] + (c ? beta*c : 0),
// summing the partial slices in increasing z (deterministic).  VEC: four
// adjacent elements per thread (m*n % 4 == 0 and 16-byte aligned c, d, W).
// ----------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(256) void splitk_reduce(ReduceParams p) {
    const uint64_t total  = p.count;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    if constexpr (VEC) {
        const floatx4* __restrict__ W = reinterpret_cast<const floatx4*>(p.partials);
        const uint64_t vecs           = total / 4;
        for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < vecs; i += stride) {
            floatx4 s = W[i];
            for (int z = 1; z < p.splits; ++z) s += W[(uint64_t)z * vecs + i];
            floatx4 out = p.alpha * s;
            if (p.c != nullptr) {
                const floatx4 cv = reinterpret_cast<const floatx4*>(p.c)[i];
#pragma unroll
                for (int j = 0; j < 4; ++j) out[j] = p.alpha * s[j] + p.beta * cv[j];
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) out[j] = p.alpha * s[j] + 0.f;
            }
            reinterpret_cast<floatx4*>(p.d)[i] = out;
        }
    } else {
        for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
            float s = p.partials[i];
            for (int z = 1; z < p.splits; ++z) s += p.partials[(uint64_t)z * total + i];
            p.d[i] = p.alpha * s + (p.c != nullptr ? p.beta * p.c[i] : 0.f);
        }
    }
}

// ----------------------------------------------------------------------------
// General SIMT kernel: 64x64 tiles, 4x4 outputs per thread, 64-bit indices,
// grid-stride over tiles.  Any shape, 4-byte alignment.
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
                As[kk][r] = (gm < M && gk < K) ? p.a[gm * K + gk] : 0.f;
                const int rb = idx / T, cb = idx % T;
                const uint64_t bk = k0 + rb, bn = n0 + cb;
                Bs[rb][cb] = (bk < K && bn < N) ? p.b[bk * N + bn] : 0.f;
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
                const uint64_t idx = row * N + c;
                p.d[idx]           = p.alpha * acc[i][j] + (p.c != nullptr ? p.beta * p.c[idx] : 0.f);
            }
        }
    }
}


}  // namespace

const void* kernelFor(Variant v) {
    switch (v) {
        case Variant::kMfma256x256: return reinterpret_cast<const void*>(&mfma_gemm<256, 256, 16, 2, 2, 3, 1, true, kWhole>);
        case Variant::kMfma256x256S: return reinterpret_cast<const void*>(&mfma_gemm<256, 256, 16, 2, 2, 3, 1, true, kPartial>);
        case Variant::kMfma256x128: return reinterpret_cast<const void*>(&mfma_gemm<256, 128, 16, 2, 2, 2, 2, true, kWhole>);
        case Variant::kMfma128x128: return reinterpret_cast<const void*>(&mfma_gemm<128, 128, 16, 2, 2, 2, 3, true, kWhole>);
        case Variant::kMfma128x128S: return reinterpret_cast<const void*>(&mfma_gemm<128, 128, 16, 2, 2, 2, 3, true, kPartial>);
        case Variant::kMfma64x256: return reinterpret_cast<const void*>(&mfma_gemm<64, 256, 16, 1, 4, 3, 1, true, kWhole>);
        case Variant::kMfma64x256S: return reinterpret_cast<const void*>(&mfma_gemm<64, 256, 16, 1, 4, 3, 1, true, kPartial>);
        case Variant::kMfma256x64: return reinterpret_cast<const void*>(&mfma_gemm<256, 64, 16, 4, 1, 3, 1, true, kWhole>);
        case Variant::kMfma256x64S: return reinterpret_cast<const void*>(&mfma_gemm<256, 64, 16, 4, 1, 3, 1, true, kPartial>);
        case Variant::kMfma64x64: return reinterpret_cast<const void*>(&mfma_gemm<64, 64, 16, 2, 2, 3, 1, true, kWhole>);
        case Variant::kMfma64x64S: return reinterpret_cast<const void*>(&mfma_gemm<64, 64, 16, 2, 2, 3, 1, true, kPartial>);
        case Variant::kMfma128x128U: return reinterpret_cast<const void*>(&mfma_gemm<128, 128, 16, 2, 2, 3, 1, false, kWhole>);
        case Variant::kMfma128x128US: return reinterpret_cast<const void*>(&mfma_gemm<128, 128, 16, 2, 2, 3, 1, false, kPartial>);
        case Variant::kMfma64x64U: return reinterpret_cast<const void*>(&mfma_gemm<64, 64, 16, 2, 2, 3, 1, false, kWhole>);
        case Variant::kGemvS: return reinterpret_cast<const void*>(&gemv_splitk<true, false>);
        case Variant::kGemvUS: return reinterpret_cast<const void*>(&gemv_splitk<false, false>);
        case Variant::kSimt: return reinterpret_cast<const void*>(&simt_gemm);
        default: return nullptr;
    }
}

const void* prologueKernel() { return reinterpret_cast<const void*>(&prologue); }

const void* reduceKernel(bool vec) {
    return vec ? reinterpret_cast<const void*>(&splitk_reduce<true>) : reinterpret_cast<const void*>(&splitk_reduce<false>);
}

}  // namespace ftrain::gemm
