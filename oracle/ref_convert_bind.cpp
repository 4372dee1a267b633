// Python binding for the reference's own CPU converter, compiled from
// /root/reference/core/wrapper/convert_wrapper.cpp where it lies (see
// oracle/build_ref.py).  Test infrastructure: used only to pin the oracle's
// CSR->BCSR restatement and as the "reference" CPU baseline of the build.
// The declaration below repeats the signature of convert_wrapper.cpp:27-33.
#include <torch/extension.h>
#include <tuple>

std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> csr_to_bcsr_cpu(
    long long num_rows, const torch::Tensor& row_ptr, const torch::Tensor& col_idx,
    const torch::Tensor& values, long long tile_rows, long long tile_cols);

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("csr_to_bcsr_cpu", &csr_to_bcsr_cpu, "reference CSR->BCSR (OpenMP)");
}
