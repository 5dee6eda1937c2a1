// flash_train.torch.gemm: PyTorch-ROCm binding over the ftrainGemm C API.
//
// Checks and defaults follow the reference binding
// (python/flash_train/torch/csrc/flash_train_torch.cpp:34-75).  The stream is
// torch's current HIP stream read natively (c10::hip::getCurrentHIPStreamMasqueradingAsCUDA),
// not through a Python call as the reference does (:28-32), and the whole
// binding is one translation unit.
#include <torch/extension.h>

#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <flash_train/flash_train.h>

namespace {

void checkMatrix(const at::Tensor& t, const char* name) {
    TORCH_CHECK(t.is_cuda(), name, " must be a device tensor");
    TORCH_CHECK(t.scalar_type() == at::kFloat, name, " must be FP32");
    TORCH_CHECK(t.dim() == 2, name, " must be rank two");
    TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

FTrainStorageView deviceMatrix(const void* p, const int64_t* dims) {
    return FTrainStorageView{const_cast<void*>(p), dims, nullptr, 2, FTRAIN_NUMERIC_TYPE_FP32,
                             FTRAIN_INDEX_TYPE_CONTINUOUS, false};
}

FTrainStorageView hostScalar(float* p) {
    return FTrainStorageView{p, nullptr, nullptr, 0, FTRAIN_NUMERIC_TYPE_FP32, FTRAIN_INDEX_TYPE_CONTINUOUS, true};
}

at::Tensor gemm(const at::Tensor& a, const at::Tensor& b, const c10::optional<at::Tensor>& c, double alpha,
                double beta) {
    checkMatrix(a, "a");
    checkMatrix(b, "b");
    TORCH_CHECK(a.size(1) == b.size(0), "a's reduction depth must equal b's rows");
    if (c.has_value()) {
        checkMatrix(*c, "c");
        TORCH_CHECK(c->size(0) == a.size(0) && c->size(1) == b.size(1), "c must be shaped m-by-n");
    }
    TORCH_CHECK(b.device() == a.device() && (!c.has_value() || c->device() == a.device()),
                "a, b and c must be on one device");

    c10::hip::HIPGuardMasqueradingAsCUDA guard(a.device());
    at::Tensor d = torch::empty({a.size(0), b.size(1)}, a.options());
    const int64_t a_dims[2] = {a.size(0), a.size(1)};
    const int64_t b_dims[2] = {b.size(0), b.size(1)};
    const int64_t d_dims[2] = {a.size(0), b.size(1)};
    float alpha_value       = static_cast<float>(alpha);
    float beta_value        = static_cast<float>(beta);
    const hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(a.device().index()).stream();

    const FTrainStatus status =
        ftrainGemm(deviceMatrix(a.data_ptr(), a_dims), deviceMatrix(b.data_ptr(), b_dims),
                   deviceMatrix(c.has_value() ? c->data_ptr() : nullptr, d_dims), deviceMatrix(d.data_ptr(), d_dims),
                   hostScalar(&alpha_value), hostScalar(&beta_value), FTRAIN_NUMERIC_TYPE_FP32, nullptr, 0, stream);
    TORCH_CHECK(status == FTRAIN_STATUS_SUCCESS, "ftrainGemm failed with status ", static_cast<unsigned>(status), ": ",
                ftrainGetLastMessage());
    return d;
}

}  // namespace

PYBIND11_MODULE(_flash_train_torch, m) {
    m.doc() = "flash-train for MI355X PyTorch binding";
    m.def("gemm", &gemm, "d = alpha * (a @ b) + beta * c on the current stream", py::arg("a"), py::arg("b"),
          py::arg("c") = py::none(), py::arg("alpha") = 1.0, py::arg("beta") = 0.0);
}
