// Drop-in pybind11 `matmul_module` for the quantized entry points of the reference
// (src/python_bindings/bindings.cpp:100-322, m.def at :653-728): same function names,
// py::arg names, validation, exception types (ValueError / RuntimeError), GIL release and
// process-wide serialisation; compute goes through the C ABI of libqmm_gfx950.so.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>

#include <mutex>
#include <stdexcept>
#include <string>

#include "qmm.h"

namespace py = pybind11;

namespace {

// One lock around every call, as the reference does for its static workspaces
// (bindings.cpp:17-18).
std::mutex g_call_mutex;

constexpr int kQK4_0 = 32, kQ4_0Bytes = 18;
constexpr int kQK8_0 = 32, kQ8_0Bytes = 34;
constexpr int kQK_K = 256, kQ4_KBytes = 144, kQ6_KBytes = 210;

void check_fp16_contiguous(const py::array& arr, const char* name, py::ssize_t min_elems,
                           bool require_writeable = false) {
    if (arr.dtype().kind() != 'f' || arr.itemsize() != 2)
        throw std::invalid_argument(std::string(name) + " must be a 2-byte FP16 (numpy.float16) array.");
    if (!(arr.flags() & py::array::c_style))
        throw std::invalid_argument(std::string(name) + " must be a C-contiguous array.");
    if (require_writeable && !arr.writeable())
        throw std::invalid_argument(std::string(name) + " must be a writeable array.");
    if (arr.size() < min_elems)
        throw std::invalid_argument(std::string(name) + " buffer is smaller than expected dimensions.");
}

void check_buffer_contiguous(const py::buffer_info& info, const char* name) {
    if (info.ndim <= 0) return;
    py::ssize_t expected = info.itemsize;
    for (py::ssize_t d = info.ndim - 1; d >= 0; --d) {
        if (info.shape[d] > 1 && info.strides[d] != expected)
            throw std::invalid_argument(std::string(name) + " buffer must be C-contiguous.");
        expected *= info.shape[d];
    }
}

void raise_status(int rc) {
    if (rc == QMM_OK) return;
    const std::string msg = qmm_last_error();
    if (rc == QMM_ERR_INVALID_ARGUMENT) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

using DequantFn = int (*)(const void*, void*, int);
using MatmulFn = int (*)(const void*, const void*, void*, int, int, int);

void dequantize_impl(const py::buffer& qbuf, py::array& out_fp16, int num_elements, int qk, int bb,
                     const char* buf_name, const char* type_name, DequantFn fn) {
    if (num_elements <= 0 || num_elements % qk != 0)
        throw std::invalid_argument("num_elements must be a positive multiple of " + std::to_string(qk) + ".");
    py::buffer_info info = qbuf.request();
    check_buffer_contiguous(info, buf_name);
    const size_t expected = static_cast<size_t>(num_elements / qk) * bb;
    const size_t actual = static_cast<size_t>(info.size) * info.itemsize;
    if (actual < expected)
        throw std::invalid_argument(std::string(type_name) + " buffer is smaller than required (num_elements / " +
                                    std::to_string(qk) + " * " + std::to_string(bb) + " bytes).");
    check_fp16_contiguous(out_fp16, "out_fp16", num_elements, true);
    const void* src = info.ptr;
    void* dst = out_fp16.mutable_data();
    int rc;
    {
        py::gil_scoped_release release;
        std::lock_guard<std::mutex> lock(g_call_mutex);
        rc = fn(src, dst, num_elements);
    }
    raise_status(rc);
}

void matmul_impl(const py::array& A, const py::buffer& B, py::array& C, int M, int N, int K, int qk, int bb,
                 const char* b_name, const char* type_name, MatmulFn fn) {
    if (K <= 0 || K % qk != 0)
        throw std::invalid_argument("K must be a positive multiple of " + std::to_string(qk) + " for " +
                                    type_name + " matmul.");
    check_fp16_contiguous(A, "A", static_cast<py::ssize_t>(M) * K);
    check_fp16_contiguous(C, "C", static_cast<py::ssize_t>(M) * N, true);
    py::buffer_info info = B.request();
    check_buffer_contiguous(info, b_name);
    const size_t expected = static_cast<size_t>(N) * (K / qk) * bb;
    const size_t actual = static_cast<size_t>(info.size) * info.itemsize;
    if (actual < expected)
        throw std::invalid_argument(std::string(b_name) + " buffer is smaller than required N * (K / " +
                                    std::to_string(qk) + ") * " + std::to_string(bb) + " bytes.");
    const void* a = A.data();
    const void* b = info.ptr;
    void* c = C.mutable_data();
    int rc;
    {
        py::gil_scoped_release release;
        std::lock_guard<std::mutex> lock(g_call_mutex);
        rc = fn(a, b, c, M, N, K);
    }
    raise_status(rc);
}

void dequantize_q4_0(const py::buffer& q4_buf, py::array& out_fp16, int num_elements) {
    dequantize_impl(q4_buf, out_fp16, num_elements, kQK4_0, kQ4_0Bytes, "q4_buf", "Q4_0", qmm_dequantize_q4_0_host);
}
void dequantize_q8_0(const py::buffer& q8_buf, py::array& out_fp16, int num_elements) {
    dequantize_impl(q8_buf, out_fp16, num_elements, kQK8_0, kQ8_0Bytes, "q8_buf", "Q8_0", qmm_dequantize_q8_0_host);
}
void dequantize_q4_k(const py::buffer& q4k_buf, py::array& out_fp16, int num_elements) {
    dequantize_impl(q4k_buf, out_fp16, num_elements, kQK_K, kQ4_KBytes, "q4k_buf", "Q4_K", qmm_dequantize_q4_k_host);
}
void dequantize_q6_k(const py::buffer& q6k_buf, py::array& out_fp16, int num_elements) {
    dequantize_impl(q6k_buf, out_fp16, num_elements, kQK_K, kQ6_KBytes, "q6k_buf", "Q6_K", qmm_dequantize_q6_k_host);
}

void matmul_q4_0(const py::array& A, const py::buffer& B_q4, py::array& C, int M, int N, int K) {
    matmul_impl(A, B_q4, C, M, N, K, kQK4_0, kQ4_0Bytes, "B_q4", "Q4_0", qmm_matmul_q4_0_host);
}
void matmul_q8_0(const py::array& A, const py::buffer& B_q8, py::array& C, int M, int N, int K) {
    matmul_impl(A, B_q8, C, M, N, K, kQK8_0, kQ8_0Bytes, "B_q8", "Q8_0", qmm_matmul_q8_0_host);
}
void matmul_q4_k(const py::array& A, const py::buffer& B_q4k, py::array& C, int M, int N, int K) {
    matmul_impl(A, B_q4k, C, M, N, K, kQK_K, kQ4_KBytes, "B_q4k", "Q4_K", qmm_matmul_q4_k_host);
}
void matmul_q6_k(const py::array& A, const py::buffer& B_q6k, py::array& C, int M, int N, int K) {
    matmul_impl(A, B_q6k, C, M, N, K, kQK_K, kQ6_KBytes, "B_q6k", "Q6_K", qmm_matmul_q6_k_host);
}

}  // namespace

PYBIND11_MODULE(matmul_module, m) {
    m.doc() = "MI355X (gfx950) fused GGUF quantized matmul kernels (Q4_0, Q8_0, Q4_K, Q6_K)";
    m.def("dequantize_q4_0", &dequantize_q4_0,
          "Dequantize GGUF Q4_0 blocks (18B per 32 weights) to FP16 on MI355X (gfx950)",
          py::arg("q4_buf"), py::arg("out_fp16"), py::arg("num_elements"));
    m.def("matmul_q4_0", &matmul_q4_0,
          "Fused FP16 x Q4_0 matrix multiplication C(M,N) = A(M,K) @ B(N,K)^T on MI355X (gfx950)",
          py::arg("A"), py::arg("B_q4"), py::arg("C"), py::arg("M"), py::arg("N"), py::arg("K"));
    m.def("dequantize_q8_0", &dequantize_q8_0,
          "Dequantize GGUF Q8_0 blocks (34B per 32 weights) to FP16 on MI355X (gfx950)",
          py::arg("q8_buf"), py::arg("out_fp16"), py::arg("num_elements"));
    m.def("matmul_q8_0", &matmul_q8_0,
          "Fused FP16 x Q8_0 matrix multiplication C(M,N) = A(M,K) @ B(N,K)^T on MI355X (gfx950)",
          py::arg("A"), py::arg("B_q8"), py::arg("C"), py::arg("M"), py::arg("N"), py::arg("K"));
    m.def("dequantize_q4_k", &dequantize_q4_k,
          "Dequantize GGUF Q4_K super-blocks (144B per 256 weights) to FP16 on MI355X (gfx950)",
          py::arg("q4k_buf"), py::arg("out_fp16"), py::arg("num_elements"));
    m.def("matmul_q4_k", &matmul_q4_k,
          "Fused FP16 x Q4_K (Q4_K_M / Q4_K_S) matrix multiplication C(M,N) = A(M,K) @ B(N,K)^T on MI355X (gfx950)",
          py::arg("A"), py::arg("B_q4k"), py::arg("C"), py::arg("M"), py::arg("N"), py::arg("K"));
    m.def("dequantize_q6_k", &dequantize_q6_k,
          "Dequantize GGUF Q6_K super-blocks (210B per 256 weights) to FP16 on MI355X (gfx950)",
          py::arg("q6k_buf"), py::arg("out_fp16"), py::arg("num_elements"));
    m.def("matmul_q6_k", &matmul_q6_k,
          "Fused FP16 x Q6_K matrix multiplication C(M,N) = A(M,K) @ B(N,K)^T on MI355X (gfx950)",
          py::arg("A"), py::arg("B_q6k"), py::arg("C"), py::arg("M"), py::arg("N"), py::arg("K"));
}
