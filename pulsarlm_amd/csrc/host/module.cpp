// Python bindings of the C++ host layer (pulsarlm_ops.hpp, linear.hpp), so the tests
// can exercise the drop-in C++ operators exactly as a C++ caller would.
#include <torch/extension.h>

#include "linear.hpp"
#include "pulsarlm_ops.hpp"

PYBIND11_MODULE(_host, m) {
    m.doc() = "pulsarlm_amd C++ host layer: pulsarlm-core quant-linear operators over the gfx950 C ABI";
    m.def("repack_int4_marlin_cuda", &pulsarlm::repack_int4_marlin_cuda);
    m.def("repack_fp8_marlin_cuda", &pulsarlm::repack_fp8_marlin_cuda);
    m.def("gemm_int4_marlin_cuda", &pulsarlm::gemm_int4_marlin_cuda);
    m.def("gemm_fp8_marlin_cuda", &pulsarlm::gemm_fp8_marlin_cuda);
    m.def("gemm_fp8_w8a8_cuda", &pulsarlm::gemm_fp8_w8a8_cuda);
    m.def("quantize_rows_e4m3_cuda", &pulsarlm::quantize_rows_e4m3_cuda);
    m.def("convert_marlin_cuda", &pulsarlm::convert_marlin_cuda);
    m.def("dequant_marlin_cuda", &pulsarlm::dequant_marlin_cuda);
    m.def("repack_int4_experts_cuda", &pulsarlm::repack_int4_experts_cuda);
    m.def("grouped_gemm_int4_cuda", &pulsarlm::grouped_gemm_int4_cuda);
    m.def("routed_experts_int4_cuda", &pulsarlm::routed_experts_int4_cuda);
    m.def("route_top_k_cuda", &pulsarlm::route_top_k_cuda);
    m.def("silu_mul_cuda", &pulsarlm::silu_mul_cuda);
    m.def("gemm_int4_cuda", &pulsarlm::gemm_int4_cuda);
    m.def("gemm_int4_split_cuda", &pulsarlm::gemm_int4_split_cuda);
    py::class_<pulsarlm::linear>(m, "linear")
        .def_static("dense", &pulsarlm::linear::dense)
        .def_static("fp8", &pulsarlm::linear::fp8)
        .def_static("fp8_rows", &pulsarlm::linear::fp8_rows)
        .def_static("int4", &pulsarlm::linear::int4)
        .def("apply", &pulsarlm::linear::apply);
}
