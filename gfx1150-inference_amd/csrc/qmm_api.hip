// C ABI of libqmm_gfx950.so (declared in include/qmm.h): argument validation, kernel dispatch
// and the host-pointer copy-in / compute / copy-out entry points.
//
// Error conventions follow the reference launchers (src/kernels/dequantize.hip:7-15, 734-736,
// 771-773): a shape the block format cannot represent is QMM_ERR_INVALID_ARGUMENT (the
// reference's std::invalid_argument), a HIP failure is QMM_ERR_HIP (std::runtime_error).
#include <atomic>
#include <cmath>
#include <mutex>
#include <string>
#include <unordered_map>

#include "qmm_internal.h"

namespace {

thread_local std::string g_last_error;
std::atomic<int> g_gemv_max_m{qmm::kGemvMaxMDefault};  // qmm_set_gemv_max_m
thread_local int g_thread_gemv_max_m = 0;              // qmm_set_thread_gemv_max_m (0: the process value)
thread_local int g_row_identity = 0;                   // qmm_set_row_identity

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char* where) {
    return fail(QMM_ERR_HIP, std::string("HIP error in ") + where + " - " + hipGetErrorString(e));
}

const char* type_name(int t) {
    switch (t) {
        case QMM_TYPE_Q4_0: return "Q4_0";
        case QMM_TYPE_Q8_0: return "Q8_0";
        case QMM_TYPE_Q4_K: return "Q4_K";
        case QMM_TYPE_Q6_K: return "Q6_K";
        case QMM_TYPE_F16: return "F16";
        default: return "unknown";
    }
}

bool known_type(int t) {
    return t == QMM_TYPE_Q4_0 || t == QMM_TYPE_Q8_0 || t == QMM_TYPE_Q4_K || t == QMM_TYPE_Q6_K;
}

// Weight types of the GEMM entry points: the quantized formats and dense F16 rows (the
// reference's matmul_nt operand, w_type 1 of its layer pipeline).
bool gemm_type(int t) { return known_type(t) || t == QMM_TYPE_F16; }

int check_gemm_args(int t, const void* A, int a_dtype, const void* W, void* C, int c_dtype, int M, int N,
                    int K) {
    if (!gemm_type(t)) return fail(QMM_ERR_INVALID_ARGUMENT, "Unsupported ggml_type " + std::to_string(t) + ".");
    if (a_dtype != QMM_DTYPE_F32 && a_dtype != QMM_DTYPE_F16)
        return fail(QMM_ERR_INVALID_ARGUMENT, "a_dtype must be QMM_DTYPE_F32 or QMM_DTYPE_F16.");
    if (c_dtype != QMM_DTYPE_F32 && c_dtype != QMM_DTYPE_F16)
        return fail(QMM_ERR_INVALID_ARGUMENT, "c_dtype must be QMM_DTYPE_F32 or QMM_DTYPE_F16.");
    const int qk = qmm::block_elems(t);
    if (K <= 0 || K % qk != 0)
        return fail(QMM_ERR_INVALID_ARGUMENT, std::string("K dimension must be a positive multiple of ") +
                                                  std::to_string(qk) + " for " + type_name(t) + " matmul.");
    if (M < 0 || N < 0) return fail(QMM_ERR_INVALID_ARGUMENT, "M and N must be non-negative.");
    if (M > 0 && N > 0 && (A == nullptr || W == nullptr || C == nullptr))
        return fail(QMM_ERR_INVALID_ARGUMENT, "A, W and C must be non-null device pointers.");
    if (M > 0 && N > 0) {
        // every workgroup reads all of A while others write C: an output over the input would race
        const uintptr_t a0 = reinterpret_cast<uintptr_t>(A), c0 = reinterpret_cast<uintptr_t>(C);
        const uintptr_t a1 = a0 + static_cast<size_t>(M) * K * (a_dtype == QMM_DTYPE_F32 ? 4 : 2);
        const uintptr_t c1 = c0 + static_cast<size_t>(M) * N * (c_dtype == QMM_DTYPE_F32 ? 4 : 2);
        if (a0 < c1 && c0 < a1) return fail(QMM_ERR_INVALID_ARGUMENT, "C must not overlap A (in-place GEMM is not supported).");
    }
    return QMM_OK;
}

int check_dequant_args(int t, const void* W, void* out, int out_dtype, int64_t n, bool device_out) {
    if (!known_type(t)) return fail(QMM_ERR_INVALID_ARGUMENT, "Unsupported ggml_type " + std::to_string(t) + ".");
    if (out_dtype != QMM_DTYPE_F32 && out_dtype != QMM_DTYPE_F16 && out_dtype != QMM_DTYPE_BF16)
        return fail(QMM_ERR_INVALID_ARGUMENT, "out_dtype must be QMM_DTYPE_F32, QMM_DTYPE_F16 or QMM_DTYPE_BF16.");
    const int qk = qmm::block_elems(t);
    if (n < 0 || n % qk != 0)
        return fail(QMM_ERR_INVALID_ARGUMENT, std::string("num_elements must be a multiple of ") +
                                                  std::to_string(qk) + " for " + type_name(t) + " dequantization.");
    if (n > 0 && (W == nullptr || out == nullptr))
        return fail(QMM_ERR_INVALID_ARGUMENT, "W and out must be non-null device pointers.");
    if (device_out && n > 0 && (reinterpret_cast<uintptr_t>(out) & 15u) != 0)
        return fail(QMM_ERR_INVALID_ARGUMENT, "out must be 16-byte aligned.");
    return QMM_OK;
}

// gmax: the GEMV / prefill threshold the call was issued under (qmm::gemv_max_m() read once);
// ident: every GEMV-range M on the kernel family of M = 1 (rows bit-identical across M).
int gemm_impl(int t, const void* A, int a_dtype, const void* W, void* C, int c_dtype, int M, int N, int K,
              hipStream_t stream, int gmax, bool ident) {
    int rc = check_gemm_args(t, A, a_dtype, W, C, c_dtype, M, N, K);
    if (rc != QMM_OK) return rc;
    if (M == 0 || N == 0) return QMM_OK;
    hipError_t e;
    if (M >= gmax && qmm::gemm_prefill_supported(t, a_dtype, c_dtype, M, N, K, A, W, C))
        e = qmm::launch_gemm_prefill(t, A, a_dtype, W, C, c_dtype, M, N, K, stream);
    else
        e = qmm::launch_gemv(t, A, a_dtype, W, C, c_dtype, M, N, K, stream, ident);
    if (e != hipSuccess) return hip_fail(e, "qmm_gemm kernel launch");
    return QMM_OK;
}

// Grow-only per-device workspace for the host-pointer API (the reference's Q4Workspace,
// src/kernels/dequantize.hip:689-725).
struct Workspace {
    void* buf[3] = {nullptr, nullptr, nullptr};
    size_t cap[3] = {0, 0, 0};
};

std::mutex g_ws_mutex;
std::unordered_map<int, Workspace> g_ws;

hipError_t ws_ensure(Workspace& ws, const size_t need[3]) {
    for (int i = 0; i < 3; ++i) {
        if (need[i] <= ws.cap[i]) continue;
        if (ws.buf[i]) {
            hipError_t e = hipFree(ws.buf[i]);
            ws.buf[i] = nullptr;
            ws.cap[i] = 0;
            if (e != hipSuccess) return e;
        }
        hipError_t e = hipMalloc(&ws.buf[i], need[i]);
        if (e != hipSuccess) {
            ws.buf[i] = nullptr;
            return e;
        }
        ws.cap[i] = need[i];
    }
    return hipSuccess;
}

// Byte ranges for the fusion checks of qmm_gemm_batch.
struct Span {
    uintptr_t lo, hi;
    bool overlaps(const Span& o) const { return lo < o.hi && o.lo < hi; }
};
Span span_of(const void* p, size_t bytes) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    return Span{a, a + bytes};
}
size_t dtype_bytes(int dt) { return dt == QMM_DTYPE_F32 ? 4 : 2; }
Span a_span(const qmm_gemm_desc& d) { return span_of(d.A, static_cast<size_t>(d.M) * d.K * dtype_bytes(d.a_dtype)); }
Span w_span(const qmm_gemm_desc& d) {
    return span_of(d.W, static_cast<size_t>(d.N) * (d.K / qmm::block_elems(d.ggml_type)) * qmm::block_bytes(d.ggml_type));
}
Span c_span(const qmm_gemm_desc& d) { return span_of(d.C, static_cast<size_t>(d.M) * d.N * dtype_bytes(d.c_dtype)); }

// Descriptors [i, j) may run as one launch: same activations, dtypes, type, M and K; no events
// between them; no output overlapping another output or any input, so the fused launch computes
// what the sequential launches would; and, for prefill sizes, weights the prefill kernel takes.
bool fusable(const qmm_gemm_desc* d, int i, int j, int gmax) {
    const qmm_gemm_desc& h = d[i];
    if (h.M <= 0) return false;
    const bool prefill = h.M >= gmax;
    for (int x = i; x < j; ++x) {
        const qmm_gemm_desc& e = d[x];
        if (e.N <= 0 || e.A != h.A || e.a_dtype != h.a_dtype || e.ggml_type != h.ggml_type ||
            e.c_dtype != h.c_dtype || e.M != h.M || e.K != h.K)
            return false;
        if (prefill && !qmm::gemm_prefill_supported(e.ggml_type, e.a_dtype, e.c_dtype, e.M, e.N, e.K, e.A, e.W, e.C))
            return false;
        if ((x > i && e.ev_before) || (x + 1 < j && e.ev_after)) return false;
        const Span c = c_span(e);
        if (c.overlaps(a_span(h))) return false;
        for (int y = i; y < j; ++y) {
            if (y != x && c.overlaps(c_span(d[y]))) return false;
            if (c.overlaps(w_span(d[y]))) return false;
        }
    }
    return true;
}

int matmul_host(int t, const void* hA, const void* hB, void* hC, int M, int N, int K) {
    int rc = check_gemm_args(t, hA, QMM_DTYPE_F16, hB, hC, QMM_DTYPE_F16, M, N, K);
    if (rc != QMM_OK) return rc;
    if (M == 0 || N == 0) return QMM_OK;
    const size_t sa = static_cast<size_t>(M) * K * 2;
    const size_t sb = static_cast<size_t>(N) * (K / qmm::block_elems(t)) * qmm::block_bytes(t);
    const size_t sc = static_cast<size_t>(M) * N * 2;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    Workspace& ws = g_ws[dev];
    const size_t need[3] = {sa, sb, sc};
    if ((e = ws_ensure(ws, need)) != hipSuccess) return hip_fail(e, "workspace hipMalloc");
    if ((e = hipMemcpy(ws.buf[0], hA, sa, hipMemcpyHostToDevice)) != hipSuccess) return hip_fail(e, "hipMemcpy A");
    if ((e = hipMemcpy(ws.buf[1], hB, sb, hipMemcpyHostToDevice)) != hipSuccess) return hip_fail(e, "hipMemcpy B");
    // the reference's host launchers: rows bit-identical across M, as its tests assert
    rc = gemm_impl(t, ws.buf[0], QMM_DTYPE_F16, ws.buf[1], ws.buf[2], QMM_DTYPE_F16, M, N, K, nullptr, qmm::gemv_max_m(),
                   true);
    if (rc != QMM_OK) return rc;
    if ((e = hipMemcpy(hC, ws.buf[2], sc, hipMemcpyDeviceToHost)) != hipSuccess) return hip_fail(e, "hipMemcpy C");
    return QMM_OK;
}

int dequant_host(int t, const void* hq, void* hout, int num_elements) {
    int rc = check_dequant_args(t, hq, hout, QMM_DTYPE_F16, num_elements, false);
    if (rc != QMM_OK) return rc;
    if (num_elements == 0) return QMM_OK;
    const size_t si = static_cast<size_t>(num_elements / qmm::block_elems(t)) * qmm::block_bytes(t);
    const size_t so = static_cast<size_t>(num_elements) * 2;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    Workspace& ws = g_ws[dev];
    const size_t need[3] = {si, so, 0};
    if ((e = ws_ensure(ws, need)) != hipSuccess) return hip_fail(e, "workspace hipMalloc");
    if ((e = hipMemcpy(ws.buf[0], hq, si, hipMemcpyHostToDevice)) != hipSuccess) return hip_fail(e, "hipMemcpy q");
    if ((e = qmm::launch_dequantize(t, ws.buf[0], ws.buf[1], QMM_DTYPE_F16, num_elements, nullptr)) != hipSuccess)
        return hip_fail(e, "dequantize kernel launch");
    if ((e = hipMemcpy(hout, ws.buf[1], so, hipMemcpyDeviceToHost)) != hipSuccess) return hip_fail(e, "hipMemcpy out");
    return QMM_OK;
}

}  // namespace

int qmm::set_last_error(int code, const std::string& msg) { return fail(code, msg); }

int qmm::gemv_max_m() {
    return g_thread_gemv_max_m > 0 ? g_thread_gemv_max_m : g_gemv_max_m.load(std::memory_order_relaxed);
}

extern "C" {

const char* qmm_last_error(void) { return g_last_error.c_str(); }

int qmm_version(void) { return 1000; }

int qmm_gemv_max_m(void) { return qmm::gemv_max_m(); }

int qmm_set_gemv_max_m(int m) {
    if (m < 1 || m > qmm::kGemvMaxMLimit)
        return fail(QMM_ERR_INVALID_ARGUMENT, "qmm_set_gemv_max_m: m must be in [1, " + std::to_string(qmm::kGemvMaxMLimit) +
                                                  "], got " + std::to_string(m) + ".");
    g_gemv_max_m.store(m, std::memory_order_relaxed);
    return QMM_OK;
}

int qmm_set_thread_gemv_max_m(int m) {
    if (m < 0 || m > qmm::kGemvMaxMLimit)
        return fail(QMM_ERR_INVALID_ARGUMENT, "qmm_set_thread_gemv_max_m: m must be 0 or in [1, " +
                                                  std::to_string(qmm::kGemvMaxMLimit) + "], got " + std::to_string(m) + ".");
    g_thread_gemv_max_m = m;
    return QMM_OK;
}

int qmm_set_row_identity(int on) {
    if (on != 0 && on != 1) return fail(QMM_ERR_INVALID_ARGUMENT, "qmm_set_row_identity: on must be 0 or 1.");
    g_row_identity = on;
    return QMM_OK;
}

int qmm_row_identity(void) { return g_row_identity; }

size_t qmm_weight_bytes(int ggml_type, int64_t n, int64_t k) {
    if (!gemm_type(ggml_type) || n < 0 || k < 0) return 0;
    const int qk = qmm::block_elems(ggml_type);
    if (k % qk != 0) return 0;
    return static_cast<size_t>(n) * static_cast<size_t>(k / qk) * static_cast<size_t>(qmm::block_bytes(ggml_type));
}

int qmm_gemm(int ggml_type, const void* A, int a_dtype, const void* W, void* C, int c_dtype, int M, int N, int K,
             void* stream) {
    return gemm_impl(ggml_type, A, a_dtype, W, C, c_dtype, M, N, K, static_cast<hipStream_t>(stream), qmm::gemv_max_m(),
                     g_row_identity != 0);
}

int qmm_gemm_noalloc(int ggml_type, const void* A, int a_dtype, const void* W, void* C, int c_dtype, int M, int N, int K,
                     void* stream) {
    int rc = check_gemm_args(ggml_type, A, a_dtype, W, C, c_dtype, M, N, K);
    if (rc != QMM_OK) return rc;
    if (M == 0 || N == 0) return QMM_OK;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e;
    if (M >= qmm::gemv_max_m() && qmm::gemm_prefill_supported(ggml_type, a_dtype, c_dtype, M, N, K, A, W, C)) {
        size_t need = 0;
        e = qmm::launch_gemm_prefill_noalloc(ggml_type, A, a_dtype, W, C, c_dtype, M, N, K, s, &need);
        if (e == hipErrorOutOfMemory && need > qmm::kNoAllocScratchBytes)
            return fail(QMM_ERR_UNSUPPORTED, "qmm_gemm_noalloc: M=" + std::to_string(M) + " N=" + std::to_string(N) +
                                                  " K=" + std::to_string(K) + " needs " + std::to_string(need) +
                                                  " bytes of scratch; the static scratch holds " +
                                                  std::to_string(qmm::kNoAllocScratchBytes) + " bytes.");
    } else {
        e = qmm::launch_gemv(ggml_type, A, a_dtype, W, C, c_dtype, M, N, K, s, g_row_identity != 0);  // allocates nothing
    }
    if (e != hipSuccess) return hip_fail(e, "qmm_gemm_noalloc kernel launch");
    return QMM_OK;
}

size_t qmm_noalloc_scratch_bytes(void) { return qmm::kNoAllocScratchBytes; }

int qmm_gemm_batch(const qmm_gemm_desc* descs, int count, void* stream) {
    if (count < 0 || (count > 0 && descs == nullptr))
        return fail(QMM_ERR_INVALID_ARGUMENT, "descs must hold count >= 0 descriptors.");
    for (int i = 0; i < count; ++i) {
        const qmm_gemm_desc& d = descs[i];
        int rc = check_gemm_args(d.ggml_type, d.A, d.a_dtype, d.W, d.C, d.c_dtype, d.M, d.N, d.K);
        if (rc != QMM_OK) return fail(rc, "descriptor " + std::to_string(i) + ": " + g_last_error);
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto record = [&](void* ev) -> int {
        hipError_t e;
        if (ev && (e = hipEventRecord(static_cast<hipEvent_t>(ev), s)) != hipSuccess) return hip_fail(e, "hipEventRecord");
        return QMM_OK;
    };
    const int gmax = qmm::gemv_max_m();  // one threshold (and kernel policy) for the whole batch
    const bool ident = g_row_identity != 0;
    int i = 0;
    while (i < count) {
        // longest run starting at i that one launch can serve
        const int max_fused = descs[i].M >= gmax ? qmm::prefill_max_fused() : qmm::gemv_max_fused();
        int j = i + 1;
        while (j < count && j - i < max_fused && fusable(descs, i, j + 1, gmax)) ++j;
        if (j - i >= 2) {
            const void* W[8];
            void* C[8];
            int N[8];
            for (int x = i; x < j; ++x) {
                W[x - i] = descs[x].W;
                C[x - i] = descs[x].C;
                N[x - i] = descs[x].N;
            }
            const qmm_gemm_desc& h = descs[i];
            int rc = record(h.ev_before);
            if (rc != QMM_OK) return rc;
            hipError_t e = h.M >= gmax
                               ? qmm::launch_gemm_prefill_fused(h.ggml_type, h.A, h.a_dtype, h.c_dtype, h.M, h.K, W, C, N,
                                                                j - i, s)
                               : qmm::launch_gemv_fused(h.ggml_type, h.A, h.a_dtype, h.c_dtype, h.M, h.K, W, C, N, j - i, s,
                                                        ident);
            if (e == hipSuccess) {
                if ((rc = record(descs[j - 1].ev_after)) != QMM_OK) return rc;
                i = j;
                continue;
            }
            if (e != hipErrorNotSupported) return hip_fail(e, "qmm_gemm_batch fused kernel launch");
            // not fusable after all (e.g. byte-load fallback): run the first one alone
            if ((rc = gemm_impl(h.ggml_type, h.A, h.a_dtype, h.W, h.C, h.c_dtype, h.M, h.N, h.K, s, gmax, ident)) != QMM_OK)
                return rc;
            if ((rc = record(h.ev_after)) != QMM_OK) return rc;
            ++i;
            continue;
        }
        const qmm_gemm_desc& d = descs[i];
        int rc = record(d.ev_before);
        if (rc != QMM_OK) return rc;
        if ((rc = gemm_impl(d.ggml_type, d.A, d.a_dtype, d.W, d.C, d.c_dtype, d.M, d.N, d.K, s, gmax, ident)) != QMM_OK) return rc;
        if ((rc = record(d.ev_after)) != QMM_OK) return rc;
        ++i;
    }
    return QMM_OK;
}

// ---- transformer layer -------------------------------------------------------------------
static int layer_status(const qmm::LayerStatus& st) { return st.code == QMM_OK ? QMM_OK : fail(st.code, st.msg); }

static int norm_dtype_ok(int dt) { return dt == QMM_DTYPE_F16 || dt == QMM_DTYPE_F32; }

int qmm_rmsnorm(const void* x, const void* weight, int weight_dtype, void* out, int M, int K, float eps, void* stream) {
    if (M < 0 || K < 0) return fail(QMM_ERR_INVALID_ARGUMENT, "M and K must be non-negative.");
    if (!norm_dtype_ok(weight_dtype)) return fail(QMM_ERR_INVALID_ARGUMENT, "weight_dtype must be QMM_DTYPE_F16 or QMM_DTYPE_F32.");
    if (M > 0 && K > 0 && (!x || !weight || !out)) return fail(QMM_ERR_INVALID_ARGUMENT, "x, weight and out must be non-null.");
    hipError_t e = qmm::launch_rmsnorm(x, nullptr, weight, weight_dtype == QMM_DTYPE_F32, nullptr, out, M, K, eps,
                                       static_cast<hipStream_t>(stream));
    return e == hipSuccess ? QMM_OK : hip_fail(e, "rmsnorm kernel launch");
}

int qmm_rmsnorm_residual(const void* x, const void* residual, const void* weight, int weight_dtype, void* h_out,
                         void* norm_out, int M, int K, float eps, void* stream) {
    if (M < 0 || K < 0) return fail(QMM_ERR_INVALID_ARGUMENT, "M and K must be non-negative.");
    if (!norm_dtype_ok(weight_dtype)) return fail(QMM_ERR_INVALID_ARGUMENT, "weight_dtype must be QMM_DTYPE_F16 or QMM_DTYPE_F32.");
    if (M > 0 && K > 0 && (!x || !residual || !weight || !h_out || !norm_out))
        return fail(QMM_ERR_INVALID_ARGUMENT, "x, residual, weight, h_out and norm_out must be non-null.");
    hipError_t e = qmm::launch_rmsnorm(x, residual, weight, weight_dtype == QMM_DTYPE_F32, h_out, norm_out, M, K, eps,
                                       static_cast<hipStream_t>(stream));
    return e == hipSuccess ? QMM_OK : hip_fail(e, "rmsnorm_residual kernel launch");
}

int qmm_residual_add(const void* x, const void* residual, void* out, int64_t n, void* stream) {
    if (n < 0) return fail(QMM_ERR_INVALID_ARGUMENT, "num_elements must be non-negative.");
    if (n > 0 && (!x || !residual || !out)) return fail(QMM_ERR_INVALID_ARGUMENT, "x, residual and out must be non-null.");
    hipError_t e = qmm::launch_residual_add(x, residual, out, n, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? QMM_OK : hip_fail(e, "residual_add kernel launch");
}

int qmm_swiglu(const void* gate, const void* up, void* out, int64_t n, void* stream) {
    if (n < 0) return fail(QMM_ERR_INVALID_ARGUMENT, "num_elements must be non-negative.");
    if (n > 0 && (!gate || !up || !out)) return fail(QMM_ERR_INVALID_ARGUMENT, "gate, up and out must be non-null.");
    hipError_t e = qmm::launch_swiglu(gate, up, out, n, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? QMM_OK : hip_fail(e, "swiglu kernel launch");
}

int qmm_rope(const void* x_in, void* x_out, int seq_len, int num_heads, int head_dim, int pos_offset, float freq_base,
             int neox, void* stream) {
    if (seq_len < 0 || num_heads < 0 || pos_offset < 0)
        return fail(QMM_ERR_INVALID_ARGUMENT, "seq_len, num_heads and pos_offset must be non-negative.");
    if (head_dim <= 0 || head_dim % 2 != 0)
        return fail(QMM_ERR_INVALID_ARGUMENT, "head_dim must be a positive even integer for RoPE.");
    if (head_dim > 256) return fail(QMM_ERR_INVALID_ARGUMENT, "head_dim must be at most 256 for RoPE.");
    if (seq_len > 0 && num_heads > 0 && (!x_in || !x_out)) return fail(QMM_ERR_INVALID_ARGUMENT, "x_in and x_out must be non-null.");
    hipError_t e = qmm::launch_rope(x_in, x_out, num_heads, nullptr, nullptr, nullptr, nullptr, 0, seq_len, head_dim,
                                    pos_offset, freq_base, neox != 0, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? QMM_OK : hip_fail(e, "rope kernel launch");
}

static int attention_args(int q_len, int kv_len, int num_heads, int num_kv_heads, int head_dim, int start_pos) {
    if (head_dim <= 0 || head_dim > 256) return fail(QMM_ERR_INVALID_ARGUMENT, "head_dim must be in (0, 256] for gqa_attention.");
    if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0)
        return fail(QMM_ERR_INVALID_ARGUMENT, "num_heads must be divisible by num_kv_heads.");
    if (q_len < 0 || kv_len < 0 || start_pos < 0)
        return fail(QMM_ERR_INVALID_ARGUMENT, "q_len, kv_len and start_pos must be non-negative.");
    return QMM_OK;
}

int qmm_gqa_attention(const void* Q, const void* K, const void* V, void* out, int q_len, int kv_len, int num_heads,
                      int num_kv_heads, int head_dim, int start_pos, float scale, int causal, void* stream) {
    int rc = attention_args(q_len, kv_len, num_heads, num_kv_heads, head_dim, start_pos);
    if (rc != QMM_OK) return rc;
    if (q_len == 0) return QMM_OK;
    if (!Q || !out || (kv_len > 0 && (!K || !V))) return fail(QMM_ERR_INVALID_ARGUMENT, "Q, K, V and Out must be non-null.");
    hipStream_t s = static_cast<hipStream_t>(stream);
    void* part = nullptr;
    const size_t pb = qmm::attention_workspace_bytes(q_len, num_heads, head_dim, kv_len);
    hipError_t e;
    if (pb > 0 && (e = qmm::layer_scratch(s, pb, &part)) != hipSuccess) return hip_fail(e, "attention workspace");
    const float sc = scale != 0.0f ? scale : 1.0f / std::sqrt(static_cast<float>(head_dim));
    e = qmm::launch_attention(Q, K, V, out, part, q_len, kv_len, num_heads, num_kv_heads, head_dim, start_pos, sc,
                              causal != 0, s);
    return e == hipSuccess ? QMM_OK : hip_fail(e, "gqa_attention kernel launch");
}

int qmm_kv_cache_init(int num_layers, int max_seq_len, int num_kv_heads, int head_dim) {
    return layer_status(qmm::kv_cache_init(num_layers, max_seq_len, num_kv_heads, head_dim));
}

int qmm_kv_cache_free(void) { return layer_status(qmm::kv_cache_free()); }

int qmm_gqa_attention_cached(const void* Q, const void* K_new, const void* V_new, void* out, int layer_idx, int q_len,
                             int start_pos, int num_heads, int num_kv_heads, int head_dim, float scale, int causal,
                             void* stream) {
    _Float16 *kc = nullptr, *vc = nullptr;
    int rc = layer_status(qmm::kv_cache_layer(layer_idx, start_pos, q_len, num_kv_heads, head_dim, &kc, &vc, nullptr));
    if (rc != QMM_OK) return rc;
    if ((rc = attention_args(q_len, start_pos + q_len, num_heads, num_kv_heads, head_dim, start_pos)) != QMM_OK) return rc;
    if (q_len == 0) return QMM_OK;
    if (!Q || !K_new || !V_new || !out) return fail(QMM_ERR_INVALID_ARGUMENT, "Q, K_new, V_new and Out must be non-null.");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t row = static_cast<size_t>(num_kv_heads) * head_dim;
    const size_t bytes = static_cast<size_t>(q_len) * row * 2;
    hipError_t e;
    if ((e = hipMemcpyAsync(kc + static_cast<size_t>(start_pos) * row, K_new, bytes, hipMemcpyDeviceToDevice, s)) != hipSuccess ||
        (e = hipMemcpyAsync(vc + static_cast<size_t>(start_pos) * row, V_new, bytes, hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return hip_fail(e, "KV cache update");
    return qmm_gqa_attention(Q, kc, vc, out, q_len, start_pos + q_len, num_heads, num_kv_heads, head_dim, start_pos, scale,
                             causal, stream);
}

int qmm_forward_layer(const qmm_layer_config* cfg, const qmm_layer_weights* w, const void* x_in, void* x_out,
                      int layer_idx, int seq_len, int pos_offset, void* stream) {
    if (!cfg || !w) return fail(QMM_ERR_INVALID_ARGUMENT, "cfg and w must be non-null.");
    if (!norm_dtype_ok(w->attn_norm_dtype) || !norm_dtype_ok(w->ffn_norm_dtype))
        return fail(QMM_ERR_INVALID_ARGUMENT, "norm weights must be QMM_DTYPE_F16 or QMM_DTYPE_F32.");
    const int types[7] = {w->wq_type, w->wk_type, w->wv_type, w->wo_type, w->wgate_type, w->wup_type, w->wdown_type};
    for (int t : types)
        if (!gemm_type(t))
            return fail(QMM_ERR_UNSUPPORTED, "projection weights must be F16, Q4_0, Q8_0, Q4_K or Q6_K (type " + std::to_string(t) + ").");
    return layer_status(qmm::forward_layer(*cfg, *w, x_in, x_out, layer_idx, seq_len, pos_offset,
                                           static_cast<hipStream_t>(stream)));
}

int qmm_upload_file(const char* path, const qmm_file_range* ranges, int count, int64_t chunk_bytes, int depth,
                    int threads, void* stream) {
    const qmm::UploadStatus st =
        qmm::upload_file_ranges(path, ranges, count, chunk_bytes, depth, threads, static_cast<hipStream_t>(stream));
    return st.code == QMM_OK ? QMM_OK : fail(st.code, st.msg);
}

int qmm_read_file(const char* path, const qmm_file_range* ranges, int count, int threads) {
    const qmm::UploadStatus st = qmm::read_file_ranges(path, ranges, count, threads);
    return st.code == QMM_OK ? QMM_OK : fail(st.code, st.msg);
}

int qmm_embed(int ggml_type, const void* table, int64_t n_rows, int hidden, const int64_t* ids, int64_t n_ids,
              void* out, int out_dtype, int* bad, void* stream) {
    const bool dense = ggml_type == QMM_TYPE_F16 || ggml_type == QMM_TYPE_F32;
    if (!dense && !known_type(ggml_type))
        return fail(QMM_ERR_INVALID_ARGUMENT, "Unsupported token_embd.weight type: " + std::to_string(ggml_type));
    if (out_dtype != QMM_DTYPE_F32 && out_dtype != QMM_DTYPE_F16 && out_dtype != QMM_DTYPE_BF16)
        return fail(QMM_ERR_INVALID_ARGUMENT, "out_dtype must be QMM_DTYPE_F32, QMM_DTYPE_F16 or QMM_DTYPE_BF16.");
    const int qk = dense ? 32 : qmm::block_elems(ggml_type);
    if (hidden <= 0 || hidden % qk != 0)
        return fail(QMM_ERR_INVALID_ARGUMENT, "hidden must be a positive multiple of " + std::to_string(qk) + ".");
    if (n_ids < 0 || n_rows < 0) return fail(QMM_ERR_INVALID_ARGUMENT, "n_ids and n_rows must be non-negative.");
    if (n_ids == 0) return QMM_OK;
    if (n_rows == 0) return fail(QMM_ERR_INVALID_ARGUMENT, "the embedding table has no rows.");
    if (table == nullptr || ids == nullptr || out == nullptr)
        return fail(QMM_ERR_INVALID_ARGUMENT, "table, ids and out must be non-null device pointers.");
    if ((reinterpret_cast<uintptr_t>(out) & 15u) != 0) return fail(QMM_ERR_INVALID_ARGUMENT, "out must be 16-byte aligned.");
    const uintptr_t ta = reinterpret_cast<uintptr_t>(table);
    if ((ggml_type == QMM_TYPE_F32 && (ta & 3u)) || (ggml_type == QMM_TYPE_F16 && (ta & 1u)))
        return fail(QMM_ERR_INVALID_ARGUMENT, "table must be aligned to its element size.");
    if ((reinterpret_cast<uintptr_t>(ids) & 7u) != 0) return fail(QMM_ERR_INVALID_ARGUMENT, "ids must be 8-byte aligned.");
    const int64_t row_bytes = dense ? static_cast<int64_t>(hidden) * (ggml_type == QMM_TYPE_F32 ? 4 : 2)
                                    : static_cast<int64_t>(hidden / qk) * qmm::block_bytes(ggml_type);
    hipError_t e = qmm::launch_embed(ggml_type, table, n_rows, row_bytes, hidden, ids, n_ids, out, out_dtype, bad,
                                     static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "qmm_embed kernel launch");
    return QMM_OK;
}

int qmm_dequantize(int ggml_type, const void* W, void* out, int out_dtype, int64_t num_elements, void* stream) {
    int rc = check_dequant_args(ggml_type, W, out, out_dtype, num_elements, true);
    if (rc != QMM_OK) return rc;
    if (num_elements == 0) return QMM_OK;
    hipError_t e = qmm::launch_dequantize(ggml_type, W, out, out_dtype, num_elements,
                                          static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "qmm_dequantize kernel launch");
    return QMM_OK;
}

int qmm_matmul_q4_0_device(const void* a, const void* b, void* c, int M, int N, int K, void* s) {
    return gemm_impl(QMM_TYPE_Q4_0, a, QMM_DTYPE_F16, b, c, QMM_DTYPE_F16, M, N, K, static_cast<hipStream_t>(s),
                     qmm::gemv_max_m(), true);
}
int qmm_matmul_q8_0_device(const void* a, const void* b, void* c, int M, int N, int K, void* s) {
    return gemm_impl(QMM_TYPE_Q8_0, a, QMM_DTYPE_F16, b, c, QMM_DTYPE_F16, M, N, K, static_cast<hipStream_t>(s),
                     qmm::gemv_max_m(), true);
}
int qmm_matmul_q4_k_device(const void* a, const void* b, void* c, int M, int N, int K, void* s) {
    return gemm_impl(QMM_TYPE_Q4_K, a, QMM_DTYPE_F16, b, c, QMM_DTYPE_F16, M, N, K, static_cast<hipStream_t>(s),
                     qmm::gemv_max_m(), true);
}
int qmm_matmul_q6_k_device(const void* a, const void* b, void* c, int M, int N, int K, void* s) {
    return gemm_impl(QMM_TYPE_Q6_K, a, QMM_DTYPE_F16, b, c, QMM_DTYPE_F16, M, N, K, static_cast<hipStream_t>(s),
                     qmm::gemv_max_m(), true);
}

int qmm_matmul_q4_0_host(const void* a, const void* b, void* c, int M, int N, int K) {
    return matmul_host(QMM_TYPE_Q4_0, a, b, c, M, N, K);
}
int qmm_matmul_q8_0_host(const void* a, const void* b, void* c, int M, int N, int K) {
    return matmul_host(QMM_TYPE_Q8_0, a, b, c, M, N, K);
}
int qmm_matmul_q4_k_host(const void* a, const void* b, void* c, int M, int N, int K) {
    return matmul_host(QMM_TYPE_Q4_K, a, b, c, M, N, K);
}
int qmm_matmul_q6_k_host(const void* a, const void* b, void* c, int M, int N, int K) {
    return matmul_host(QMM_TYPE_Q6_K, a, b, c, M, N, K);
}

int qmm_dequantize_q4_0_host(const void* q, void* out, int n) { return dequant_host(QMM_TYPE_Q4_0, q, out, n); }
int qmm_dequantize_q8_0_host(const void* q, void* out, int n) { return dequant_host(QMM_TYPE_Q8_0, q, out, n); }
int qmm_dequantize_q4_k_host(const void* q, void* out, int n) { return dequant_host(QMM_TYPE_Q4_K, q, out, n); }
int qmm_dequantize_q6_k_host(const void* q, void* out, int n) { return dequant_host(QMM_TYPE_Q6_K, q, out, n); }

int qmm_release_workspace(void) {
    qmm::release_upload_staging();
    {
        hipError_t le = qmm::release_layer_workspaces();
        if (le != hipSuccess) return hip_fail(le, "releasing the layer workspaces");
        if ((le = qmm::release_host_staging()) != hipSuccess) return hip_fail(le, "releasing the host staging buffer");
    }
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    for (auto& kv : g_ws) {
        if ((e = hipSetDevice(kv.first)) != hipSuccess) return hip_fail(e, "hipSetDevice");
        for (int i = 0; i < 3; ++i) {
            if (kv.second.buf[i]) (void)hipFree(kv.second.buf[i]);
            kv.second.buf[i] = nullptr;
            kv.second.cap[i] = 0;
        }
    }
    g_ws.clear();
    if ((e = hipSetDevice(cur)) != hipSuccess) return hip_fail(e, "hipSetDevice");
    if ((e = qmm::release_prefill_workspaces()) != hipSuccess) return hip_fail(e, "release prefill workspace");
    return QMM_OK;
}

}  // extern "C"
