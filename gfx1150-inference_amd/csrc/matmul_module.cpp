// Drop-in pybind11 `matmul_module` for the reference's entry points
// (src/python_bindings/bindings.cpp:53-627, m.def at :629-859): the quantized dequantize /
// matmul functions, the dense fp16 matmul / matmul_nt, the layer operations, the device KV
// pool and forward_layer_cached.  Same function names, py::arg names and defaults, validation,
// exception types (ValueError / IndexError / RuntimeError), GIL release and process-wide
// serialisation; compute goes through the C ABI of libqmm_gfx950.so.
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
    if (rc == QMM_ERR_OUT_OF_RANGE) throw std::out_of_range(msg);
    throw std::runtime_error(msg);
}

// Runs `fn` (returning a QMM status) without the GIL, under the process-wide lock.
template <class Fn>
void locked_call(Fn fn) {
    int rc;
    {
        py::gil_scoped_release release;
        std::lock_guard<std::mutex> lock(g_call_mutex);
        rc = fn();
    }
    raise_status(rc);
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

// ---- dense fp16 matmuls (bindings.cpp:53-98) -------------------------------------------------
void matmul(const py::array& A, const py::array& B, py::array& C, int M, int N, int K) {
    check_fp16_contiguous(A, "A", static_cast<py::ssize_t>(M) * K);
    check_fp16_contiguous(B, "B", static_cast<py::ssize_t>(K) * N);
    check_fp16_contiguous(C, "C", static_cast<py::ssize_t>(M) * N, true);
    const void* a = A.data();
    const void* b = B.data();
    void* c = C.mutable_data();
    locked_call([&] { return qmm_matmul_fp16_host(a, b, c, M, N, K); });
}

void matmul_nt(const py::array& A, const py::array& B_nt, py::array& C, int M, int N, int K) {
    check_fp16_contiguous(A, "A", static_cast<py::ssize_t>(M) * K);
    check_fp16_contiguous(B_nt, "B_nt", static_cast<py::ssize_t>(N) * K);
    if (B_nt.ndim() != 2 || B_nt.shape(0) != N || B_nt.shape(1) != K)
        throw std::invalid_argument("B_nt must be a 2D array with shape (N, K) for matmul_nt.");
    check_fp16_contiguous(C, "C", static_cast<py::ssize_t>(M) * N, true);
    const void* a = A.data();
    const void* b = B_nt.data();
    void* c = C.mutable_data();
    locked_call([&] { return qmm_matmul_fp16_nt_host(a, b, c, M, N, K); });
}

// ---- layer operations (bindings.cpp:324-514) ---------------------------------------------------
void rmsnorm(const py::array& x, const py::array& weight, py::array& out, int M, int K, float eps) {
    check_fp16_contiguous(x, "x", static_cast<py::ssize_t>(M) * K);
    check_fp16_contiguous(weight, "weight", K);
    check_fp16_contiguous(out, "out", static_cast<py::ssize_t>(M) * K, true);
    const void* px = x.data();
    const void* pw = weight.data();
    void* po = out.mutable_data();
    locked_call([&] { return qmm_rmsnorm_host(px, pw, po, M, K, eps); });
}

void rmsnorm_residual(const py::array& x, const py::array& residual, const py::array& weight, py::array& h_out,
                      py::array& norm_out, int M, int K, float eps) {
    const py::ssize_t total = static_cast<py::ssize_t>(M) * K;
    check_fp16_contiguous(x, "x", total);
    check_fp16_contiguous(residual, "residual", total);
    check_fp16_contiguous(weight, "weight", K);
    check_fp16_contiguous(h_out, "h_out", total, true);
    check_fp16_contiguous(norm_out, "norm_out", total, true);
    const void* px = x.data();
    const void* pr = residual.data();
    const void* pw = weight.data();
    void* ph = h_out.mutable_data();
    void* pn = norm_out.mutable_data();
    locked_call([&] { return qmm_rmsnorm_residual_host(px, pr, pw, ph, pn, M, K, eps); });
}

void residual_add(const py::array& x, const py::array& residual, py::array& out, int num_elements) {
    check_fp16_contiguous(x, "x", num_elements);
    check_fp16_contiguous(residual, "residual", num_elements);
    check_fp16_contiguous(out, "out", num_elements, true);
    const void* px = x.data();
    const void* pr = residual.data();
    void* po = out.mutable_data();
    locked_call([&] { return qmm_residual_add_host(px, pr, po, num_elements); });
}

void rope(const py::array& x_in, py::array& x_out, int seq_len, int num_heads, int head_dim, int pos_offset,
          float freq_base, bool neox_style) {
    const py::ssize_t total = static_cast<py::ssize_t>(seq_len) * num_heads * head_dim;
    check_fp16_contiguous(x_in, "x_in", total);
    check_fp16_contiguous(x_out, "x_out", total, true);
    const void* pi = x_in.data();
    void* po = x_out.mutable_data();
    locked_call([&] {
        return qmm_rope_host(pi, po, seq_len, num_heads, head_dim, pos_offset, freq_base, neox_style ? 1 : 0);
    });
}

void gqa_attention(const py::array& Q, const py::array& K, const py::array& V, py::array& Out, int q_len, int kv_len,
                   int num_heads, int num_kv_heads, int head_dim, int start_pos, float scale, bool causal) {
    const py::ssize_t q_elems = static_cast<py::ssize_t>(q_len) * num_heads * head_dim;
    const py::ssize_t kv_elems = static_cast<py::ssize_t>(kv_len) * num_kv_heads * head_dim;
    check_fp16_contiguous(Q, "Q", q_elems);
    check_fp16_contiguous(K, "K", kv_elems);
    check_fp16_contiguous(V, "V", kv_elems);
    check_fp16_contiguous(Out, "Out", q_elems, true);
    const void* pq = Q.data();
    const void* pk = K.data();
    const void* pv = V.data();
    void* po = Out.mutable_data();
    locked_call([&] {
        return qmm_gqa_attention_host(pq, pk, pv, po, q_len, kv_len, num_heads, num_kv_heads, head_dim, start_pos, scale,
                                      causal ? 1 : 0);
    });
}

void swiglu(const py::array& gate, const py::array& up, py::array& out, int num_elements) {
    check_fp16_contiguous(gate, "gate", num_elements);
    check_fp16_contiguous(up, "up", num_elements);
    check_fp16_contiguous(out, "out", num_elements, true);
    const void* pg = gate.data();
    const void* pu = up.data();
    void* po = out.mutable_data();
    locked_call([&] { return qmm_swiglu_host(pg, pu, po, num_elements); });
}

void kv_cache_init(int num_layers, int max_seq_len, int num_kv_heads, int head_dim) {
    locked_call([&] { return qmm_kv_cache_init(num_layers, max_seq_len, num_kv_heads, head_dim); });
}

void kv_cache_free() {
    locked_call([&] { return qmm_kv_cache_free(); });
}

void gqa_attention_cached(const py::array& Q, const py::array& K_new, const py::array& V_new, py::array& Out,
                          int layer_idx, int q_len, int start_pos, int num_heads, int num_kv_heads, int head_dim,
                          float scale, bool causal) {
    const py::ssize_t q_elems = static_cast<py::ssize_t>(q_len) * num_heads * head_dim;
    const py::ssize_t kv_new_elems = static_cast<py::ssize_t>(q_len) * num_kv_heads * head_dim;
    check_fp16_contiguous(Q, "Q", q_elems);
    check_fp16_contiguous(K_new, "K_new", kv_new_elems);
    check_fp16_contiguous(V_new, "V_new", kv_new_elems);
    check_fp16_contiguous(Out, "Out", q_elems, true);
    const void* pq = Q.data();
    const void* pk = K_new.data();
    const void* pv = V_new.data();
    void* po = Out.mutable_data();
    locked_call([&] {
        return qmm_gqa_attention_cached_host(pq, pk, pv, po, layer_idx, q_len, start_pos, num_heads, num_kv_heads,
                                             head_dim, scale, causal ? 1 : 0);
    });
}

// ---- forward_layer_cached (bindings.cpp:516-627) ------------------------------------------------
const void* check_weight_buffer(const py::buffer& buf, int w_type, int N, int K, const char* name) {
    py::buffer_info info = buf.request();
    check_buffer_contiguous(info, name);
    const size_t actual = static_cast<size_t>(info.size) * info.itemsize;
    size_t expected = 0;
    auto blocks = [&](int qk, int bb, const char* tname) {
        if (K <= 0 || K % qk != 0)
            throw std::invalid_argument(std::string(name) + " K must be divisible by " + std::to_string(qk) + " for " +
                                        tname + ".");
        return static_cast<size_t>(N) * (K / qk) * bb;
    };
    if (w_type == 1) expected = static_cast<size_t>(N) * K * 2;
    else if (w_type == 2) expected = blocks(kQK4_0, kQ4_0Bytes, "Q4_0");
    else if (w_type == 8) expected = blocks(kQK8_0, kQ8_0Bytes, "Q8_0");
    else if (w_type == 12) expected = blocks(kQK_K, kQ4_KBytes, "Q4_K");
    else if (w_type == 14) expected = blocks(kQK_K, kQ6_KBytes, "Q6_K");
    else throw std::invalid_argument(std::string(name) + " has unsupported ggml_type.");
    if (actual < expected) throw std::invalid_argument(std::string(name) + " weight buffer is smaller than required.");
    return info.ptr;
}

void forward_layer_cached(const py::array& x_in, py::array& x_out, const py::array& attn_norm_w, const py::buffer& wq,
                          int wq_type, const py::buffer& wk, int wk_type, const py::buffer& wv, int wv_type,
                          const py::buffer& wo, int wo_type, const py::array& ffn_norm_w, const py::buffer& wgate,
                          int wgate_type, const py::buffer& wup, int wup_type, const py::buffer& wdown, int wdown_type,
                          int layer_idx, int seq_len, int pos_offset, int hidden_size, int intermediate_size,
                          int num_heads, int num_kv_heads, int head_dim, float rms_norm_eps, float rope_freq_base,
                          bool rope_neox, float scale) {
    const py::ssize_t hidden_elems = static_cast<py::ssize_t>(seq_len) * hidden_size;
    check_fp16_contiguous(x_in, "x_in", hidden_elems);
    check_fp16_contiguous(x_out, "x_out", hidden_elems, true);
    check_fp16_contiguous(attn_norm_w, "attn_norm_w", hidden_size);
    check_fp16_contiguous(ffn_norm_w, "ffn_norm_w", hidden_size);
    const int q_dim = num_heads * head_dim, kv_dim = num_kv_heads * head_dim;
    qmm_layer_weights w{};
    w.attn_norm = attn_norm_w.data();
    w.attn_norm_dtype = QMM_DTYPE_F16;
    w.ffn_norm = ffn_norm_w.data();
    w.ffn_norm_dtype = QMM_DTYPE_F16;
    w.wq = check_weight_buffer(wq, wq_type, q_dim, hidden_size, "wq");
    w.wk = check_weight_buffer(wk, wk_type, kv_dim, hidden_size, "wk");
    w.wv = check_weight_buffer(wv, wv_type, kv_dim, hidden_size, "wv");
    w.wo = check_weight_buffer(wo, wo_type, hidden_size, q_dim, "wo");
    w.wgate = check_weight_buffer(wgate, wgate_type, intermediate_size, hidden_size, "wgate");
    w.wup = check_weight_buffer(wup, wup_type, intermediate_size, hidden_size, "wup");
    w.wdown = check_weight_buffer(wdown, wdown_type, hidden_size, intermediate_size, "wdown");
    w.wq_type = wq_type;
    w.wk_type = wk_type;
    w.wv_type = wv_type;
    w.wo_type = wo_type;
    w.wgate_type = wgate_type;
    w.wup_type = wup_type;
    w.wdown_type = wdown_type;
    qmm_layer_config c{};
    c.hidden_size = hidden_size;
    c.intermediate_size = intermediate_size;
    c.num_heads = num_heads;
    c.num_kv_heads = num_kv_heads;
    c.head_dim = head_dim;
    c.rms_norm_eps = rms_norm_eps;
    c.rope_freq_base = rope_freq_base;
    c.rope_neox = rope_neox ? 1 : 0;
    c.scale = scale;
    const void* xi = x_in.data();
    void* xo = x_out.mutable_data();
    locked_call([&] { return qmm_forward_layer_host(&c, &w, xi, xo, layer_idx, seq_len, pos_offset); });
}

}  // namespace

PYBIND11_MODULE(matmul_module, m) {
    m.doc() = "MI355X (gfx950) fused GGUF quantized matmul kernels (Q4_0, Q8_0, Q4_K, Q6_K) and transformer layer kernels";
    m.def("matmul", &matmul, "FP16 matrix multiplication C(M,N) = A(M,K) @ B(K,N) on MI355X (gfx950)", py::arg("A"),
          py::arg("B"), py::arg("C"), py::arg("M"), py::arg("N"), py::arg("K"));
    m.def("matmul_nt", &matmul_nt, "FP16 matrix multiplication C(M,N) = A(M,K) @ B_nt(N,K)^T on MI355X (gfx950)",
          py::arg("A"), py::arg("B_nt"), py::arg("C"), py::arg("M"), py::arg("N"), py::arg("K"));
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
    m.def("rmsnorm", &rmsnorm, "Root Mean Square Layer Normalization on MI355X (gfx950)", py::arg("x"), py::arg("weight"),
          py::arg("out"), py::arg("M"), py::arg("K"), py::arg("eps") = 1e-5f);
    m.def("rmsnorm_residual", &rmsnorm_residual, "Fused Residual Add + RMSNorm on MI355X (gfx950)", py::arg("x"),
          py::arg("residual"), py::arg("weight"), py::arg("h_out"), py::arg("norm_out"), py::arg("M"), py::arg("K"),
          py::arg("eps") = 1e-5f);
    m.def("residual_add", &residual_add, "FP32-accumulated FP16 residual addition on MI355X (gfx950)", py::arg("x"),
          py::arg("residual"), py::arg("out"), py::arg("num_elements"));
    m.def("rope", &rope, "Rotary Positional Embeddings (RoPE) on MI355X (gfx950)", py::arg("x_in"), py::arg("x_out"),
          py::arg("seq_len"), py::arg("num_heads"), py::arg("head_dim"), py::arg("pos_offset") = 0,
          py::arg("freq_base") = 10000.0f, py::arg("neox_style") = false);
    m.def("gqa_attention", &gqa_attention, "Grouped-Query Attention (GQA) with online softmax on MI355X (gfx950)",
          py::arg("Q"), py::arg("K"), py::arg("V"), py::arg("Out"), py::arg("q_len"), py::arg("kv_len"),
          py::arg("num_heads"), py::arg("num_kv_heads"), py::arg("head_dim"), py::arg("start_pos") = 0,
          py::arg("scale") = 0.0f, py::arg("causal") = true);
    m.def("swiglu", &swiglu, "Fused SwiGLU activation out = SiLU(gate) * up on MI355X (gfx950)", py::arg("gate"),
          py::arg("up"), py::arg("out"), py::arg("num_elements"));
    m.def("kv_cache_init", &kv_cache_init, "Allocate GPU-resident GQA KV cache pool for all transformer layers",
          py::arg("num_layers"), py::arg("max_seq_len"), py::arg("num_kv_heads"), py::arg("head_dim"));
    m.def("kv_cache_free", &kv_cache_free, "Free GPU-resident GQA KV cache pool");
    m.def("gqa_attention_cached", &gqa_attention_cached,
          "Update GPU-resident KV cache at start_pos and run GQA online-softmax attention", py::arg("Q"), py::arg("K_new"),
          py::arg("V_new"), py::arg("Out"), py::arg("layer_idx"), py::arg("q_len"), py::arg("start_pos"),
          py::arg("num_heads"), py::arg("num_kv_heads"), py::arg("head_dim"), py::arg("scale") = 0.0f,
          py::arg("causal") = true);
    m.def("forward_layer_cached", &forward_layer_cached,
          "Execute a full transformer layer on-device with GPU-resident KV cache", py::arg("x_in"), py::arg("x_out"),
          py::arg("attn_norm_w"), py::arg("wq"), py::arg("wq_type"), py::arg("wk"), py::arg("wk_type"), py::arg("wv"),
          py::arg("wv_type"), py::arg("wo"), py::arg("wo_type"), py::arg("ffn_norm_w"), py::arg("wgate"),
          py::arg("wgate_type"), py::arg("wup"), py::arg("wup_type"), py::arg("wdown"), py::arg("wdown_type"),
          py::arg("layer_idx"), py::arg("seq_len"), py::arg("pos_offset"), py::arg("hidden_size"),
          py::arg("intermediate_size"), py::arg("num_heads"), py::arg("num_kv_heads"), py::arg("head_dim"),
          py::arg("rms_norm_eps"), py::arg("rope_freq_base"), py::arg("rope_neox"), py::arg("scale"));
}
