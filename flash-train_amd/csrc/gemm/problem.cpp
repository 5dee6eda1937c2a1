// GemmProblem validation and selection key; GemmFamily pattern and Args
// extraction.  Validation follows src/family/gemm/problem.cpp:13-56.
#include <algorithm>
#include <limits>

#include "ft/gemm.hpp"
#include "ft/grouped.hpp"

namespace ftrain {

GemmProblem::GemmProblem(Tensor a, Tensor b, Tensor c, Tensor d, Tensor alpha, Tensor beta,
                         FTrainNumericType compute_type)
    : a_(std::move(a)), b_(std::move(b)), c_(std::move(c)), d_(std::move(d)), alpha_(std::move(alpha)),
      beta_(std::move(beta)), compute_type_(compute_type) {
    if (a_.view.rank() != 2 || b_.view.rank() != 2 || c_.view.rank() != 2 || d_.view.rank() != 2)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Gemm requires rank-two a, b, c, and d Tensors");
    if (alpha_.view.rank() != 0 || beta_.view.rank() != 0)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Gemm requires scalar alpha and beta Tensors");
    if (a_.view.isHost() || b_.view.isHost() || c_.view.isHost() || d_.view.isHost())
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Gemm requires a, b, c, and d in device memory");
    if (!alpha_.view.isHost() || !beta_.view.isHost())
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Gemm requires alpha and beta in host memory");
    if (a_.view.dims()[1] != b_.view.dims()[0])
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Gemm a column count %lld does not match b row count %lld",
                        static_cast<long long>(a_.view.dims()[1]), static_cast<long long>(b_.view.dims()[0]));
    const GemmShape s = shape();
    const std::vector<int64_t> mn{static_cast<int64_t>(s.m), static_cast<int64_t>(s.n)};
    if (c_.view.dims() != mn || d_.view.dims() != mn)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Gemm c and d shapes must both be m-by-n");
    // Each matrix's byte size must fit in uint64.
    const uint64_t max_elems = std::numeric_limits<uint64_t>::max() / sizeof(float);
    const auto over          = [max_elems](uint64_t x, uint64_t y) { return y != 0 && x > max_elems / y; };
    if (over(s.m, s.k) || over(s.k, s.n) || over(s.m, s.n))
        raise(FTRAIN_STATUS_OVERFLOW, "Gemm matrix byte size overflows uint64_t");
}

const char* matrixLayout(const StorageView& v, MatrixLayout& out) {
    const int64_t r = v.dims()[0], c = v.dims()[1];
    if (v.indexType() == FTRAIN_INDEX_TYPE_CONTINUOUS) {
        out = MatrixLayout{false, std::max<int64_t>(c, 1)};
        return nullptr;
    }
    if (v.indexType() != FTRAIN_INDEX_TYPE_INVALID) return "an operand is not continuously indexed";
    const int64_t s0 = v.strides()[0], s1 = v.strides()[1];
    if (s0 < 0 || s1 < 0) return "a matrix stride is negative";
    const bool unit_cols = c <= 1 || s1 == 1;  // consecutive columns adjacent
    const bool unit_rows = r <= 1 || s0 == 1;  // consecutive rows adjacent
    if (unit_cols && (r <= 1 || s0 == c))
        return "explicit strides restate the continuous layout (use FTRAIN_INDEX_TYPE_CONTINUOUS)";
    // Largest element offset must stay addressable.
    const int64_t max_off = std::numeric_limits<int64_t>::max() / int64_t(sizeof(double));
    const auto span       = [max_off](int64_t n, int64_t s) { return n <= 1 ? 0 : (s > max_off / (n - 1) ? max_off : (n - 1) * s); };
    if (span(r, s0) >= max_off || span(c, s1) >= max_off || span(r, s0) + span(c, s1) >= max_off)
        return "a matrix extent overflows the address range";
    if (unit_cols && s0 >= c) {
        out = MatrixLayout{false, r <= 1 ? std::max<int64_t>(c, 1) : s0};
        return nullptr;
    }
    if (unit_rows && (c <= 1 || s1 >= r)) {
        out = MatrixLayout{true, c <= 1 ? std::max<int64_t>(r, 1) : s1};
        return nullptr;
    }
    return "matrix strides need a unit stride in one dimension and a non-overlapping leading dimension";
}

const char* GemmProblem::launch(GemmLaunch& out) const {
    MatrixLayout la, lb, lc, ld;
    if (const char* why = matrixLayout(a_.view, la)) return why;
    if (const char* why = matrixLayout(b_.view, lb)) return why;
    if (const char* why = matrixLayout(c_.view, lc)) return why;
    if (const char* why = matrixLayout(d_.view, ld)) return why;
    const GemmShape s = shape();
    const bool has_c  = c_.view.memory() != nullptr;
    // A 1-row or 1-column matrix fits either orientation; take d's.
    if (has_c && lc.col_major != ld.col_major) {
        if (s.m <= 1 || s.n <= 1)
            lc = MatrixLayout{ld.col_major, ld.col_major ? std::max<int64_t>(int64_t(s.m), 1) : std::max<int64_t>(int64_t(s.n), 1)};
        else
            return "c and d must share one orientation";
    }
    if (!ld.col_major) {
        out = GemmLaunch{s, a_.view.memory(), b_.view.memory(), c_.view.memory(), d_.view.memory(),
                         la.col_major, lb.col_major, la.ld, lb.ld, lc.ld, ld.ld};
    } else {
        // d^T (n x m, row-major with row stride ld) = b^T a^T + c^T.
        out = GemmLaunch{GemmShape{s.n, s.m, s.k}, b_.view.memory(), a_.view.memory(), c_.view.memory(),
                         d_.view.memory(), !lb.col_major, !la.col_major, lb.ld, la.ld, lc.ld, ld.ld};
    }
    if (!has_c) out.ldc = out.ldd;
    return nullptr;
}

const StorageView& GemmProblem::port(int i) const noexcept {
    switch (i) {
        case 0: return a_.view;
        case 1: return b_.view;
        case 2: return c_.view;
        case 3: return d_.view;
        case 4: return alpha_.view;
        default: return beta_.view;
    }
}

std::vector<uint64_t> GemmProblem::key() const {
    std::vector<uint64_t> k;
    k.reserve(96);
    uint64_t field = 0;
    for (int i = 0; i < 6; ++i) {
        const StorageView& v = port(i);
        const auto addr      = reinterpret_cast<uintptr_t>(v.memory());
        k.insert(k.end(), {++field, v.numericType(), ++field, v.indexType(), ++field, uint64_t(v.memory() != nullptr),
                           ++field, uint64_t(addr % 16), ++field, uint64_t(v.rank())});
        for (int64_t x : v.dims()) k.push_back(static_cast<uint64_t>(x));
        k.insert(k.end(), {++field, uint64_t(v.strides().size())});
        for (int64_t x : v.strides()) k.push_back(static_cast<uint64_t>(x));
    }
    k.insert(k.end(), {++field, compute_type_, ++field, uint64_t(inPlace())});
    return k;
}

const GemmFamily::Roles& GemmFamily::roles() {
    static const Roles r = [] {
        PatternBuilder pb;
        const uint64_t a     = pb.addOperand(OperandKind::kTensor);
        const uint64_t b     = pb.addOperand(OperandKind::kTensor);
        const uint64_t c     = pb.addOperand(OperandKind::kTensor);
        const uint64_t alpha = pb.addOperand(OperandKind::kTensor);
        const uint64_t beta  = pb.addOperand(OperandKind::kTensor);
        const uint64_t d     = pb.addOperand(OperandKind::kTensor);
        const uint64_t op    = pb.addOperation(OpNode{OperationKind::kGemm, {a, b, c, alpha, beta}, {d}});
        return Roles{pb.build(), a, b, c, d, alpha, beta, op};
    }();
    return r;
}

GemmProblem GemmFamily::makeProblem(const Args& args) {
    const Roles& r = roles();
    auto tensor    = [&](uint64_t id) { return std::get<Tensor>(*args.operand(id)); };
    return GemmProblem(tensor(r.a), tensor(r.b), tensor(r.c), tensor(r.d), tensor(r.alpha), tensor(r.beta),
                       args.operation(r.gemm)->compute_type);
}

std::vector<std::shared_ptr<OpsEngineBase>> builtinEngines() {
    std::vector<std::shared_ptr<OpsEngineBase>> engines{std::make_shared<GemmEngine>()};
    for (auto& e : groupedEngines()) engines.push_back(std::move(e));
    return engines;
}

}  // namespace ftrain
