// Host-pointer entry points of the dense fp16 matmuls and of the layer operations: the
// reference's synchronous launchers (copy the operands in, run on the device, copy the result
// out), kept for drop-in callers that hold NumPy arrays.  Reference: launch_matmul_fp16 /
// launch_matmul_fp16_nt (src/kernels/matmul.hip:340-395, 441-463), launch_rmsnorm_fp16,
// launch_rmsnorm_residual_fp16, launch_residual_add_fp16 (src/kernels/rmsnorm.h), launch_rope_fp16
// (rope.h), launch_swiglu_fp16 (mlp.h), launch_gqa_attention_fp16 and
// launch_gqa_attention_cached_fp16 (attention.hip:228-374), launch_forward_layer_cached_fp16
// (attention.hip:603-695).
//
// All device work runs on the null stream between synchronous copies.  Operands are staged in
// one grow-only device buffer per device (256-byte aligned pieces), serialised by one lock, as
// the reference's static workspaces are.  Device-pointer callers use the qmm_* entry points
// directly and never pay for these copies.
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "qmm_internal.h"

namespace qmm {
namespace {

constexpr int kTile = 64;

// out[n][k] = in[k][n] for an fp16 [rows = K][cols = N] matrix: 64 x 64 tiles through LDS (one
// padding column against bank conflicts), 256 threads, coalesced reads and writes.
__global__ __launch_bounds__(256) void transpose_f16_kernel(const uint16_t* __restrict__ in, uint16_t* __restrict__ out,
                                                            int rows, int cols) {
    __shared__ uint16_t tile[kTile][kTile + 1];
    const int c0 = blockIdx.x * kTile, r0 = blockIdx.y * kTile;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
    for (int i = ty; i < kTile; i += 4) {
        const int r = r0 + i, c = c0 + tx;
        if (r < rows && c < cols) tile[i][tx] = in[static_cast<size_t>(r) * cols + c];
    }
    __syncthreads();
    for (int i = ty; i < kTile; i += 4) {
        const int c = c0 + i, r = r0 + tx;  // output row c, column r
        if (c < cols && r < rows) out[static_cast<size_t>(c) * rows + r] = tile[tx][i];
    }
}

struct Staging {
    void* buf = nullptr;
    size_t cap = 0;
};
std::mutex g_mutex;
std::unordered_map<int, Staging> g_staging;

size_t round256(size_t b) { return (b + 255) / 256 * 256; }

// Device buffer of at least `bytes` for the current device (grow-only; the caller holds g_mutex).
hipError_t staging(size_t bytes, char** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    Staging& st = g_staging[dev];
    if (st.cap < bytes) {
        if (st.buf) {
            if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
            if ((e = hipFree(st.buf)) != hipSuccess) return e;
            st.buf = nullptr;
            st.cap = 0;
        }
        if ((e = hipMalloc(&st.buf, bytes)) != hipSuccess) return e;
        st.cap = bytes;
    }
    *out = static_cast<char*>(st.buf);
    return hipSuccess;
}

// One host operand of a staged call: `in` operands are copied to the device before the call,
// `out` operands back after it.
struct Operand {
    const void* host_in;
    void* host_out;
    size_t bytes;
    void* dev = nullptr;
};

}  // namespace

hipError_t release_host_staging() {
    std::lock_guard<std::mutex> lock(g_mutex);
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    for (auto& kv : g_staging) {
        if (!kv.second.buf) continue;
        if ((e = hipSetDevice(kv.first)) != hipSuccess) return e;
        if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
        if ((e = hipFree(kv.second.buf)) != hipSuccess) return e;
        kv.second = Staging{};
    }
    g_staging.clear();
    return hipSetDevice(cur);
}

}  // namespace qmm

namespace {

using qmm::Operand;

// Stages `ops` (device addresses assigned in order), runs `body` on the null stream, copies the
// outputs back.  body returns a QMM status; its message is already in qmm_last_error().
template <class Body>
int staged(std::vector<Operand>& ops, Body body) {
    std::lock_guard<std::mutex> lock(qmm::g_mutex);
    size_t total = 0;
    for (const Operand& o : ops) total += qmm::round256(o.bytes);
    char* base = nullptr;
    hipError_t e;
    if (total > 0 && (e = qmm::staging(total, &base)) != hipSuccess)
        return qmm::set_last_error(QMM_ERR_HIP, std::string("hipMalloc (host staging): ") + hipGetErrorString(e));
    size_t off = 0;
    for (Operand& o : ops) {
        o.dev = base + off;
        off += qmm::round256(o.bytes);
        if (o.host_in && o.bytes > 0 && (e = hipMemcpy(o.dev, o.host_in, o.bytes, hipMemcpyHostToDevice)) != hipSuccess)
            return qmm::set_last_error(QMM_ERR_HIP, std::string("hipMemcpy (to device): ") + hipGetErrorString(e));
    }
    const int rc = body();
    if (rc != QMM_OK) return rc;
    if ((e = hipDeviceSynchronize()) != hipSuccess)
        return qmm::set_last_error(QMM_ERR_HIP, std::string("kernel execution: ") + hipGetErrorString(e));
    for (Operand& o : ops) {
        if (o.host_out && o.bytes > 0 && (e = hipMemcpy(o.host_out, o.dev, o.bytes, hipMemcpyDeviceToHost)) != hipSuccess)
            return qmm::set_last_error(QMM_ERR_HIP, std::string("hipMemcpy (to host): ") + hipGetErrorString(e));
    }
    return QMM_OK;
}

int bad(const std::string& msg) { return qmm::set_last_error(QMM_ERR_INVALID_ARGUMENT, msg); }

size_t h2(int64_t n) { return n > 0 ? static_cast<size_t>(n) * 2 : 0; }

}  // namespace

extern "C" {

int qmm_matmul_fp16_nt_device(const void* d_A, const void* d_B_nt, void* d_C, int M, int N, int K, void* stream) {
    return qmm_gemm(QMM_TYPE_F16, d_A, QMM_DTYPE_F16, d_B_nt, d_C, QMM_DTYPE_F16, M, N, K, stream);
}

int qmm_matmul_fp16_nt_host(const void* h_A, const void* h_B_nt, void* h_C, int M, int N, int K) {
    if (M < 0 || N < 0 || K <= 0) return bad("M and N must be non-negative and K positive.");
    if (M == 0 || N == 0) return QMM_OK;
    std::vector<Operand> ops = {{h_A, nullptr, h2(int64_t{M} * K)}, {h_B_nt, nullptr, h2(int64_t{N} * K)},
                                {nullptr, h_C, h2(int64_t{M} * N)}};
    return staged(ops, [&] {
        return qmm_gemm(QMM_TYPE_F16, ops[0].dev, QMM_DTYPE_F16, ops[1].dev, ops[2].dev, QMM_DTYPE_F16, M, N, K, nullptr);
    });
}

int qmm_matmul_fp16_host(const void* h_A, const void* h_B, void* h_C, int M, int N, int K) {
    if (M < 0 || N < 0 || K <= 0) return bad("M and N must be non-negative and K positive.");
    if (M == 0 || N == 0) return QMM_OK;
    // B [K, N] is transposed on the device into B_nt [N, K] (staged after it), then C = A @ B_nt^T.
    std::vector<Operand> ops = {{h_A, nullptr, h2(int64_t{M} * K)}, {h_B, nullptr, h2(int64_t{K} * N)},
                                {nullptr, h_C, h2(int64_t{M} * N)}, {nullptr, nullptr, h2(int64_t{N} * K)}};
    return staged(ops, [&] {
        const dim3 grid((N + qmm::kTile - 1) / qmm::kTile, (K + qmm::kTile - 1) / qmm::kTile);
        hipLaunchKernelGGL(qmm::transpose_f16_kernel, grid, dim3(256), 0, nullptr,
                           static_cast<const uint16_t*>(ops[1].dev), static_cast<uint16_t*>(ops[3].dev), K, N);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess)
            return qmm::set_last_error(QMM_ERR_HIP, std::string("transpose kernel launch: ") + hipGetErrorString(e));
        return qmm_gemm(QMM_TYPE_F16, ops[0].dev, QMM_DTYPE_F16, ops[3].dev, ops[2].dev, QMM_DTYPE_F16, M, N, K, nullptr);
    });
}

int qmm_rmsnorm_host(const void* h_x, const void* h_weight, void* h_out, int M, int K, float eps) {
    if (M < 0 || K < 0) return bad("M and K must be non-negative.");
    std::vector<Operand> ops = {{h_x, nullptr, h2(int64_t{M} * K)}, {h_weight, nullptr, h2(K)},
                                {nullptr, h_out, h2(int64_t{M} * K)}};
    return staged(ops, [&] {
        return qmm_rmsnorm(ops[0].dev, ops[1].dev, QMM_DTYPE_F16, ops[2].dev, M, K, eps, nullptr);
    });
}

int qmm_rmsnorm_residual_host(const void* h_x, const void* h_residual, const void* h_weight, void* h_h_out,
                              void* h_norm_out, int M, int K, float eps) {
    if (M < 0 || K < 0) return bad("M and K must be non-negative.");
    const size_t n = h2(int64_t{M} * K);
    std::vector<Operand> ops = {{h_x, nullptr, n}, {h_residual, nullptr, n}, {h_weight, nullptr, h2(K)},
                                {nullptr, h_h_out, n}, {nullptr, h_norm_out, n}};
    return staged(ops, [&] {
        return qmm_rmsnorm_residual(ops[0].dev, ops[1].dev, ops[2].dev, QMM_DTYPE_F16, ops[3].dev, ops[4].dev, M, K, eps,
                                    nullptr);
    });
}

int qmm_residual_add_host(const void* h_x, const void* h_residual, void* h_out, int64_t num_elements) {
    if (num_elements < 0) return bad("num_elements must be non-negative.");
    const size_t n = h2(num_elements);
    std::vector<Operand> ops = {{h_x, nullptr, n}, {h_residual, nullptr, n}, {nullptr, h_out, n}};
    return staged(ops, [&] { return qmm_residual_add(ops[0].dev, ops[1].dev, ops[2].dev, num_elements, nullptr); });
}

int qmm_swiglu_host(const void* h_gate, const void* h_up, void* h_out, int64_t num_elements) {
    if (num_elements < 0) return bad("num_elements must be non-negative.");
    const size_t n = h2(num_elements);
    std::vector<Operand> ops = {{h_gate, nullptr, n}, {h_up, nullptr, n}, {nullptr, h_out, n}};
    return staged(ops, [&] { return qmm_swiglu(ops[0].dev, ops[1].dev, ops[2].dev, num_elements, nullptr); });
}

int qmm_rope_host(const void* h_in, void* h_out, int seq_len, int num_heads, int head_dim, int pos_offset,
                  float freq_base, int neox) {
    if (seq_len < 0 || num_heads < 0 || head_dim < 0) return bad("seq_len, num_heads and head_dim must be non-negative.");
    const size_t n = h2(int64_t{seq_len} * num_heads * head_dim);
    std::vector<Operand> ops = {{h_in, nullptr, n}, {nullptr, h_out, n}};
    return staged(ops, [&] {
        return qmm_rope(ops[0].dev, ops[1].dev, seq_len, num_heads, head_dim, pos_offset, freq_base, neox, nullptr);
    });
}

int qmm_gqa_attention_host(const void* h_Q, const void* h_K, const void* h_V, void* h_out, int q_len, int kv_len,
                           int num_heads, int num_kv_heads, int head_dim, int start_pos, float scale, int causal) {
    if (q_len < 0 || kv_len < 0 || num_heads < 0 || num_kv_heads < 0 || head_dim < 0)
        return bad("q_len, kv_len, num_heads, num_kv_heads and head_dim must be non-negative.");
    const size_t nq = h2(int64_t{q_len} * num_heads * head_dim), nkv = h2(int64_t{kv_len} * num_kv_heads * head_dim);
    std::vector<Operand> ops = {{h_Q, nullptr, nq}, {h_K, nullptr, nkv}, {h_V, nullptr, nkv}, {nullptr, h_out, nq}};
    return staged(ops, [&] {
        return qmm_gqa_attention(ops[0].dev, ops[1].dev, ops[2].dev, ops[3].dev, q_len, kv_len, num_heads, num_kv_heads,
                                 head_dim, start_pos, scale, causal, nullptr);
    });
}

int qmm_gqa_attention_cached_host(const void* h_Q, const void* h_K_new, const void* h_V_new, void* h_out, int layer_idx,
                                  int q_len, int start_pos, int num_heads, int num_kv_heads, int head_dim, float scale,
                                  int causal) {
    if (q_len < 0 || num_heads < 0 || num_kv_heads < 0 || head_dim < 0)
        return bad("q_len, num_heads, num_kv_heads and head_dim must be non-negative.");
    const size_t nq = h2(int64_t{q_len} * num_heads * head_dim), nkv = h2(int64_t{q_len} * num_kv_heads * head_dim);
    std::vector<Operand> ops = {{h_Q, nullptr, nq}, {h_K_new, nullptr, nkv}, {h_V_new, nullptr, nkv}, {nullptr, h_out, nq}};
    return staged(ops, [&] {
        return qmm_gqa_attention_cached(ops[0].dev, ops[1].dev, ops[2].dev, ops[3].dev, layer_idx, q_len, start_pos,
                                        num_heads, num_kv_heads, head_dim, scale, causal, nullptr);
    });
}

int qmm_forward_layer_host(const qmm_layer_config* cfg, const qmm_layer_weights* w, const void* h_x_in, void* h_x_out,
                           int layer_idx, int seq_len, int pos_offset) {
    if (!cfg || !w) return bad("cfg and w must be non-null.");
    if (seq_len < 0 || cfg->hidden_size <= 0 || cfg->intermediate_size <= 0 || cfg->num_heads <= 0 ||
        cfg->num_kv_heads <= 0 || cfg->head_dim <= 0)
        return bad("seq_len must be non-negative and the layer dimensions positive.");
    const int hidden = cfg->hidden_size, inter = cfg->intermediate_size;
    const int q_dim = cfg->num_heads * cfg->head_dim, kv_dim = cfg->num_kv_heads * cfg->head_dim;
    const void* wp[7] = {w->wq, w->wk, w->wv, w->wo, w->wgate, w->wup, w->wdown};
    const int wt[7] = {w->wq_type, w->wk_type, w->wv_type, w->wo_type, w->wgate_type, w->wup_type, w->wdown_type};
    const int wn[7] = {q_dim, kv_dim, kv_dim, hidden, inter, inter, hidden};
    const int wk[7] = {hidden, hidden, hidden, q_dim, hidden, hidden, inter};
    static const char* const names[7] = {"wq", "wk", "wv", "wo", "wgate", "wup", "wdown"};
    std::vector<Operand> ops;
    ops.push_back({h_x_in, nullptr, h2(int64_t{seq_len} * hidden)});
    ops.push_back({nullptr, h_x_out, h2(int64_t{seq_len} * hidden)});
    const size_t norm_bytes[2] = {static_cast<size_t>(hidden) * (w->attn_norm_dtype == QMM_DTYPE_F32 ? 4 : 2),
                                  static_cast<size_t>(hidden) * (w->ffn_norm_dtype == QMM_DTYPE_F32 ? 4 : 2)};
    ops.push_back({w->attn_norm, nullptr, norm_bytes[0]});
    ops.push_back({w->ffn_norm, nullptr, norm_bytes[1]});
    for (int i = 0; i < 7; ++i) {
        const size_t b = qmm_weight_bytes(wt[i], wn[i], wk[i]);
        if (b == 0)
            return bad(std::string(names[i]) + " has an unsupported ggml_type or a K its blocks do not divide.");
        ops.push_back({wp[i], nullptr, b});
    }
    // optional fp16 biases (host vectors) follow the weights
    const void* bp[4] = {w->bq, w->bk, w->bv, w->bo};
    const int bn[4] = {q_dim, kv_dim, kv_dim, hidden};
    int bias_op[4] = {-1, -1, -1, -1};
    for (int i = 0; i < 4; ++i) {
        if (bp[i] == nullptr) continue;
        bias_op[i] = static_cast<int>(ops.size());
        ops.push_back({bp[i], nullptr, h2(bn[i])});
    }
    return staged(ops, [&] {
        qmm_layer_weights d = *w;
        d.attn_norm = ops[2].dev;
        d.ffn_norm = ops[3].dev;
        const void** dst[7] = {&d.wq, &d.wk, &d.wv, &d.wo, &d.wgate, &d.wup, &d.wdown};
        for (int i = 0; i < 7; ++i) *dst[i] = ops[4 + i].dev;
        const void** bdst[4] = {&d.bq, &d.bk, &d.bv, &d.bo};
        for (int i = 0; i < 4; ++i) *bdst[i] = bias_op[i] >= 0 ? ops[bias_op[i]].dev : nullptr;
        return qmm_forward_layer(cfg, &d, ops[0].dev, ops[1].dev, layer_idx, seq_len, pos_offset, nullptr);
    });
}

}  // extern "C"
