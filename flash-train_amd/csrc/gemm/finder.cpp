// ShapeCost Finder: ranks the kernel catalog by a roofline cost model.
//
// The reference ships only a placeholder Finder that expresses no preference
// (src/include/flash_train/family/gemm/finder.hpp:21-26); selection then falls
// back to registration order.  This Finder estimates each variant's time on
// the problem's shape and returns the variants best-first; the engine drops
// the ones whose applicability check fails (alignment, size limits) and
// caches the surviving order per problem key.
//
// Model, per variant (microseconds):
//   compute: workgroups = tiles * splits; each CU runs ceil(wgs / CUs) of
//            them back to back at the variant's sustained fraction of its
//            MFMA FLOP/clk/CU at 2.4 GHz (interpolated down to the variant's
//            single-workgroup fraction while fewer than its resident count
//            are available), plus a fixed cost per round of resident
//            workgroups.
//   memory : algorithmic bytes (a, b, d, optional c) at 80% of 8 TB/s, plus
//            the partial tiles (written and read once) for split-k; scaled
//            by the share of CUs the launch's workgroups occupy when there
//            are fewer workgroups than CUs.
//   time   = max(compute, memory) + the reduction's pass over the partial
//            tiles (split-k) + launch latency (one more for split-k).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <limits>
#include <numeric>

#include <hip/hip_runtime_api.h>

#include "ft/gemm.hpp"

namespace ftrain {
namespace gemm {

namespace {
constexpr double kClockPerMicro = 2.4e3;  // peak engine clock (MHz)
constexpr double kHbmBytesPerMicro = 8.0e6 * 0.8;  // sustained HBM bytes per microsecond
constexpr double kLaunchMicros = 1.23;
constexpr double kPoolMicros      = 3.48;  // dependency gap before the reduction kernel (fitted)
// The reduction kernel's pass over the partial tiles, relative to HBM time (fitted).
constexpr double kReduceFactor    = 1.206;
// The deep-k kernel (SplitKind::kFused): ramp of its single round, and the
// tile's last workgroup storing, counting and gathering the partial tiles
// (measured on MI355X: 3.7 us at 4 splits, 11-12 us at 16; the per-split
// figure is set so that the kernel loses to the split-k tiles at 16 splits,
// as measured: 64x1024x16384 33.9 against 31.1 us, 256x256x65536 89.8
// against 80.0).
constexpr double kFusedRampMicros     = 1.5;
constexpr double kFusedGatherMicros   = 2.2;
constexpr double kFusedPerSplitMicros = 0.9;
constexpr double kFusedStoreMicros    = 2.0;  // per round: a split workgroup's partial store and count
// Fixed cost per round of resident workgroups (operand prologue, epilogue
// stores, the ramp of the first stages); fitted with the catalog efficiencies.
constexpr double kRoundMicros     = 3.35;
constexpr double kTieWeight       = 1e-3;
constexpr double kCuBytesPerMicro = 6.4e4;  // one CU's sustained load rate (about 27 bytes per clock)
// A DMA tile stages a partial last stage (k not a multiple of its stage) by ordinary loads once its
// pipeline has drained: per tile, the drain, the loads' latency and a barrier.  Fitted to the bf16
// grouped weight gradient (16384 ragged tokens, 4096x14336 weights, ms, DMA against register-staged
// 256x256 tile): 8 experts 1.80 / 2.01, 16 2.25 / 2.42, 32 3.28 / 3.23, 64 5.28 / 4.86, 128 9.15 /
// 8.22; the DMA tile is ranked first at 8 experts only (7% lost at 16).
constexpr double kDmaTailMicros = 3.0;
constexpr uint64_t kMinSplitDepth = 256;  // reduction depth worth one split-k workgroup
constexpr uint64_t kMinGemvDepth  = 64;

uint64_t ceilDiv(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

// Whether variant vi runs a k tail through the separate pass of the DMA tiles (stages of 32 k for
// fp32, 64 for 16-bit inputs).
bool dmaTail(const VariantInfo& vi, uint64_t k) {
    return std::strstr(vi.name, "_Dma") != nullptr && k % (vi.input == FTRAIN_NUMERIC_TYPE_FP32 ? 32 : 64) != 0;
}
}  // namespace

int computeUnits(FTrainDeviceId device) {
    static std::atomic<int> cached[64] = {};
    const int slot = device >= 0 && device < 64 ? device : -1;
    if (slot >= 0) {
        const int v = cached[slot].load(std::memory_order_relaxed);
        if (v > 0) return v;
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        n = 256;
    }
    if (slot >= 0) cached[slot].store(n, std::memory_order_relaxed);
    return n;
}

namespace {

// Sustained fraction of the MFMA rate when a CU holds `per_cu` of the
// launch's workgroups: interpolated between one resident workgroup and the
// variant's full occupancy.
double residentEfficiency(const VariantInfo& vi, uint64_t per_cu) {
    if (vi.occupancy <= 1) return vi.efficiency;
    const double resident = double(std::min<uint64_t>(std::max<uint64_t>(per_cu, 1), uint64_t(vi.occupancy)));
    return vi.solo_efficiency + (vi.efficiency - vi.solo_efficiency) * (resident - 1.0) / double(vi.occupancy - 1);
}

// Modelled time of variant `v` with a given split count (1 = no split).
double modelMicros(const VariantInfo& vi, const GemmShape& s, bool has_c, int cus, uint64_t splits) {
    const double m = double(s.m), n = double(s.n), k = double(s.k);
    // a and b in the variant's input type; c and d counted at the same size.
    const double eb   = vi.input == FTRAIN_NUMERIC_TYPE_FP32 ? 4.0 : 2.0;
    double bytes      = eb * (m * k + k * n + m * n * (has_c ? 2.0 : 1.0));
    double launch     = kLaunchMicros;
    double serial_us  = 0.0;  // work in a second kernel that cannot overlap the first
    if (vi.split == SplitKind::kPartial) {
        // The GEMM kernel writes splits partial tiles instead of d; the
        // reduction kernel then reads them (and c) and writes d.
        bytes += 4.0 * m * n * (double(splits) - 1.0 - (has_c ? 1.0 : 0.0));
        serial_us = kReduceFactor * 4.0 * m * n * (double(splits) + (has_c ? 2.0 : 1.0)) / kHbmBytesPerMicro;
        launch += kLaunchMicros + kPoolMicros;
    }
    if (vi.split == SplitKind::kFused && splits > 1) {
        // Partial tiles written and read once, plus the last workgroup's
        // store / count / gather, after the tile's other workgroups.
        const double tiles = double(ceilDiv(s.m, vi.bm) * ceilDiv(s.n, vi.bn));
        bytes += 2.0 * 4.0 * tiles * vi.bm * vi.bn * double(splits);
        serial_us = kFusedGatherMicros + kFusedPerSplitMicros * (double(splits) - 1.0);
    }
    if (vi.gemv) {
        // Too few waves cannot reach the HBM peak; about four per CU do
        // (measured with the one-pass kernel: 1024 waves over 256 CUs stream
        // 5.4-6.3 TB/s, 256 waves lose to split-k).
        // A CU also loads at a bounded rate, so a launch of few workgroups is bound by the bytes each
        // one reads (bf16 1x4096x4096, 64 workgroups of 512 KiB: 9.0 us).
        const int threads = vi.split == SplitKind::kNone ? gemvPassThreads(int(std::max<uint64_t>(s.m, 1))) : vi.threads;
        const double wgs  = double(ceilDiv(std::max<uint64_t>(s.n, 1), uint64_t(vi.bn)) * splits);
        const double fill = std::min(1.0, wgs * (threads / 64) / (double(cus) * 4.0));
        const double per_cu = std::ceil(wgs / double(cus)) * bytes / wgs;
        const double t      = std::max(bytes / (kHbmBytesPerMicro * fill), per_cu / kCuBytesPerMicro) + serial_us + launch;
        // The split-k skinny kernel keeps few loads in flight per wave and runs well below the
        // streaming model, more so with more rows of a (measured on MI355X, us, model in brackets:
        // 1x1024x4096 11.9 [8.7], 4x1024x4096 16.5 [8.9], 8x1024x8192 40.1 [12.0], 1x4096x4096 28.4
        // [16.5], 8x4096x4096 68.3 [17.2]); it lost to the one-pass kernel or a DMA split-k tile on
        // every shape measured (1x1024x4096 one-pass 6.7, 8x1024x8192 64x128 DMA split-k 13.4).
        return vi.split == SplitKind::kPartial ? t * (1.5 + double(std::min<uint64_t>(s.m, 8)) / 4.0) : t;
    }
    // Work per workgroup includes the tile padding at the m/n edges.  The
    // dispatcher refills a CU as soon as one of its workgroups retires, so a
    // CU's load is its share of workgroups, ceil(wgs / CUs), each at the
    // CU's sustained rate; below `occupancy` resident workgroups a CU runs
    // correspondingly below that rate.
    const uint64_t chunk   = splits == 1 ? s.k : ceilDiv(ceilDiv(s.k, splits), vi.bk) * vi.bk;
    const uint64_t used    = chunk == 0 ? 1 : ceilDiv(s.k, chunk);
    const uint64_t tiles   = ceilDiv(s.m, vi.bm) * ceilDiv(s.n, vi.bn);
    const uint64_t wgs     = tiles * used;
    const uint64_t per_cu  = ceilDiv(wgs, cus);
    const double depth     = double(std::max<uint64_t>(chunk, vi.bk));
    // SIMT FMAs run at half the matrix rate without packed FP32.
    const double cu_rate   = vi.flop_per_clk * kClockPerMicro * residentEfficiency(vi, per_cu) * (vi.simt ? 0.5 : 1.0);
    const double rounds    = double(ceilDiv(per_cu, uint64_t(vi.occupancy)));
    // The deep-k kernel runs one workgroup per CU: each round pays the ramp
    // and, when split, its workgroups' partial-tile stores and arrival.
    const double per_round = vi.split != SplitKind::kFused ? kRoundMicros
                             : kFusedRampMicros + (splits > 1 ? kFusedStoreMicros : 0.0);
    // The tail pass: every tile's when whole-k, the last split's tiles when split.
    const double tails     = !dmaTail(vi, s.k) ? 0.0 : used == 1 ? rounds
                                                   : double(ceilDiv(ceilDiv(tiles, cus), uint64_t(vi.occupancy)));
    const double compute   = double(per_cu) * 2.0 * vi.bm * vi.bn * depth / cu_rate + rounds * per_round +
                           tails * kDmaTailMicros;
    // A launch with fewer workgroups than CUs streams memory through only that many of them (a CU
    // moves a bounded number of bytes per clock): 64x4096x14336 bf16 on the 64x128 split tile took
    // 36.3 us at 4 splits (128 workgroups) against 23.8 us at 8.  On the 16-bit 64x128 split tile
    // (m of at most 64) 85% of the CUs already stream at the full rate: 32x14336x4096 22.5 us at 2
    // splits (224 workgroups) against 24.1 at 4, and 5-10% the same way at 4 to 64 rows of n 13824
    // and 14336; the 128x128 split tile at such counts lost 4-15%, so it keeps the plain fraction.
    const bool half_64x128 = vi.input != FTRAIN_NUMERIC_TYPE_FP32 && vi.bm == 64 && vi.bn == 128 &&
                             vi.split == SplitKind::kPartial;
    const double fill = std::min(1.0, double(wgs) / (double(cus) * (half_64x128 ? 0.85 : 1.0)));
    double memory     = bytes / (kHbmBytesPerMicro * fill);
    // A whole-k launch of at most half as many workgroups as CUs is bound by what each workgroup
    // loads at one CU's rate, not by a fraction of HBM: bf16 128x4096x1024 on the 128x128 DMA
    // tile (32 workgroups of 0.5 MiB) 9.3 us against 13.2 for the split tile the fraction picked,
    // 128x256x512 6.5 against 10.7 for the 64x64 unaligned tile.  At 224 workgroups (4x28672x4096)
    // the fraction still ranks right.
    if (vi.split == SplitKind::kNone && !vi.simt && 2 * wgs <= uint64_t(cus)) {
        const double wg_bytes = eb * double(vi.bm + vi.bn) * double(s.k) + 4.0 * vi.bm * vi.bn;
        memory = std::max(bytes / kHbmBytesPerMicro, wg_bytes / kCuBytesPerMicro);
    }
    // When memory bounds several variants alike, the one with the least compute overlaps it best
    // (64x14336x4096 bf16 at 4 splits: the 64x128 DMA split tile 25.9 us, the 128x128 one 27.6,
    // the register-staged 128x128 30.2): a thousandth of the compute time breaks such ties.
    return std::max(compute, memory) + serial_us + launch + kTieWeight * compute;
}

}  // namespace

namespace {
std::atomic<uint32_t> g_forced_splits{0};
}

void forceSplits(uint32_t s) { g_forced_splits.store(s, std::memory_order_relaxed); }

uint32_t chooseSplits(Variant v, const GemmShape& s, int cus) {
    const VariantInfo& vi = info(v);
    if (vi.split == SplitKind::kNone) return 1;
    if (const uint32_t forced = g_forced_splits.load(std::memory_order_relaxed); forced > 0 && !vi.gemv) {
        // Clamped to whole reduction steps per split, the workspace cap, and
        // (deep-k) one arrival counter per tile.
        const uint64_t tiles = std::max<uint64_t>(ceilDiv(s.m, vi.bm) * ceilDiv(s.n, vi.bn), 1);
        const uint64_t unit  = vi.split == SplitKind::kPartial ? s.m * s.n * sizeof(float)
                                                               : tiles * vi.bm * vi.bn * sizeof(float);
        const uint64_t most =
            std::min<uint64_t>(s.k / vi.bk, (kMaxPartialBytes - kCounterBytes) / std::max<uint64_t>(unit, 1));
        const uint64_t got = std::min<uint64_t>(forced, most);
        return static_cast<uint32_t>(got >= 2 ? got : vi.split == SplitKind::kPartial ? 0 : 1);
    }
    const uint64_t min_depth = vi.gemv ? kMinGemvDepth : kMinSplitDepth;
    uint64_t most            = std::min<uint64_t>(1024, s.k / min_depth);
    if (vi.split == SplitKind::kPartial && s.m * s.n > 0)
        most = std::min<uint64_t>(most, (kMaxPartialBytes - kCounterBytes) / (s.m * s.n * sizeof(float)));
    if (vi.split == SplitKind::kFused) {
        // One split is a plain whole-k launch; more only while the partial
        // tiles fit the cap.
        const uint64_t tile_bytes = ceilDiv(s.m, vi.bm) * ceilDiv(s.n, vi.bn) * vi.bm * vi.bn * sizeof(float);
        most = std::min<uint64_t>(most, (kMaxPartialBytes - kCounterBytes) / std::max<uint64_t>(tile_bytes, 1));
        uint64_t best = 1;
        double best_t = modelMicros(vi, s, false, cus, 1);
        for (uint64_t sp = 2; sp <= most; sp *= 2) {
            const double t = modelMicros(vi, s, false, cus, sp);
            if (t < best_t * 0.999) {
                best_t = t;
                best   = sp;
            }
        }
        return static_cast<uint32_t>(best);
    }
    if (vi.gemv && most < 2) return 1;  // the skinny kernel also runs unsplit
    if (most < 2 || s.m == 0 || s.n == 0) return 0;
    // Smallest modelled time over powers of two in [2, most] (ties: fewer splits).
    uint64_t best = 0;
    double best_t = std::numeric_limits<double>::infinity();
    for (uint64_t sp = 2; sp <= most; sp *= 2) {
        const double t = modelMicros(vi, s, false, cus, sp);
        if (t < best_t * 0.999) {
            best_t = t;
            best   = sp;
        }
    }
    return static_cast<uint32_t>(best);
}

double estimateMicros(Variant v, const GemmShape& s, bool has_c, int cus) {
    const VariantInfo& vi = info(v);
    if (vi.gemv && s.m > uint64_t(vi.bm)) return std::numeric_limits<double>::infinity();
    const uint32_t splits = vi.split != SplitKind::kNone ? chooseSplits(v, s, cus) : 1;
    if (splits == 0) return std::numeric_limits<double>::infinity();
    return modelMicros(vi, s, has_c, cus, splits);
}

double groupedMicros(Variant v, const std::vector<GemmShape>& shapes, bool has_c, int cus) {
    // The groups' tiles share one grid: a CU's load is its share of all
    // tiles, each costing its own group's depth; bytes add over the groups.
    const VariantInfo& vi = info(v);
    const double eb = vi.input == FTRAIN_NUMERIC_TYPE_FP32 ? 4.0 : 2.0;
    double flops = 0.0, bytes = 0.0;
    uint64_t tiles = 0, tail_tiles = 0;
    for (const GemmShape& s : shapes) {
        const uint64_t t = ceilDiv(s.m, vi.bm) * ceilDiv(s.n, vi.bn);
        tiles += t;
        if (dmaTail(vi, s.k)) tail_tiles += t;
        flops += double(t) * 2.0 * vi.bm * vi.bn * double(std::max<uint64_t>(s.k, vi.bk));
        bytes += eb * (double(s.m) * s.k + double(s.k) * s.n + double(s.m) * s.n * (has_c ? 2.0 : 1.0));
    }
    if (tiles == 0) return kLaunchMicros;
    const uint64_t per_cu = ceilDiv(tiles, cus);
    const double cu_rate  = vi.flop_per_clk * kClockPerMicro * residentEfficiency(vi, per_cu);
    const double rounds   = double(ceilDiv(per_cu, uint64_t(vi.occupancy)));
    const double tails    = double(ceilDiv(ceilDiv(tail_tiles, cus), uint64_t(vi.occupancy)));
    const double compute  = double(per_cu) * (flops / double(tiles)) / cu_rate + rounds * kRoundMicros +
                           tails * kDmaTailMicros;
    return std::max(compute, bytes / kHbmBytesPerMicro) + kLaunchMicros;
}

}  // namespace gemm

std::vector<std::string> ShapeCostFinder::candidates(const GemmProblem& problem, const Constraints& constraints) {
    // Rank on the shape the kernels run: a column-major d swaps m and n.
    GemmLaunch g;
    const GemmShape s = problem.launch(g) == nullptr ? g.shape : problem.shape();
    const int cus     = gemm::computeUnits(constraints.device());
    const bool has_c  = problem.c().memory() != nullptr;
    std::vector<std::pair<double, int>> ranked;
    for (int i = 0; i < static_cast<int>(gemm::Variant::kCount); ++i) {
        // Only variants for a's element type compete.
        if (gemm::info(static_cast<gemm::Variant>(i)).input != problem.a().numericType()) continue;
        const double t = gemm::estimateMicros(static_cast<gemm::Variant>(i), s, has_c, cus);
        if (std::isfinite(t)) ranked.emplace_back(t, i);
    }
    std::stable_sort(ranked.begin(), ranked.end(),
                     [](const auto& x, const auto& y) { return x.first < y.first; });
    std::vector<std::string> names;
    names.reserve(ranked.size());
    for (const auto& r : ranked) names.emplace_back(gemm::info(static_cast<gemm::Variant>(r.second)).name);
    return names;
}

}  // namespace ftrain
