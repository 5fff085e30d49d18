// Internal declarations shared by the HIP translation units of libqmm_gfx950.so.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>

#include "qmm.h"

#include <string>

namespace qmm {

// GGUF block geometry (reference src/kernels/dequantize.h:6-22).
constexpr int kQK4_0 = 32, kBytesQ4_0 = 18;
constexpr int kQK8_0 = 32, kBytesQ8_0 = 34;
constexpr int kQK_K = 256, kBytesQ4_K = 144, kBytesQ6_K = 210;

// Sets the calling thread's qmm_last_error() text and returns `code` (for entry points defined
// outside the file that owns the error state).
int set_last_error(int code, const std::string& msg);

// Frees the host-pointer entry points' staging buffers (after synchronizing each device).
hipError_t release_host_staging();

// M below gemv_max_m() runs the GEMV family (row m bit-identical to the M = 1 call for every such
// M, as the reference asserts for M = 4, 7 and 16: tests/test_phase5_scale.py:274-310); M at or
// above it runs the MFMA prefill GEMM (its 32-row tile up to M = 32), whose rows agree with M = 1
// within the prefill bound.  The GEMV's per-row vector work grows with M, the MFMA tile's does
// not: at M = 17..31 the 32-row tile is 3.5-6x faster on the 70B shapes.  The default is 17;
// qmm_set_gemv_max_m moves it (up to 65536, the GEMV kernels' grid rows), e.g. for callers that
// need every M bit-identical to M = 1, as the reference's TILE_M = 4 kernels give.
constexpr int kGemvMaxMDefault = 17;
constexpr int kGemvMaxMLimit = 65536;
int gemv_max_m();

inline int block_elems(int t) {
    switch (t) {
        case QMM_TYPE_Q4_0: return kQK4_0;
        case QMM_TYPE_Q8_0: return kQK8_0;
        case QMM_TYPE_Q4_K: return kQK_K;
        case QMM_TYPE_Q6_K: return kQK_K;
        case QMM_TYPE_F16: return 1;
        default: return 0;
    }
}

inline int block_bytes(int t) {
    switch (t) {
        case QMM_TYPE_Q4_0: return kBytesQ4_0;
        case QMM_TYPE_Q8_0: return kBytesQ8_0;
        case QMM_TYPE_Q4_K: return kBytesQ4_K;
        case QMM_TYPE_Q6_K: return kBytesQ6_K;
        case QMM_TYPE_F16: return 2;
        default: return 0;
    }
}

// Work folded into a GEMV launch with fp16 activations (the decode layer's neighbours of its
// projections).  Activation prologue, applied while the activations are staged:
//   kind 0: A as given;
//   kind 1: half(A * rsqrt(mean(A^2) + eps) * w), w F16 or F32 (w_f32) of length K;
//   kind 2: the same on v = half(A + R).
// Output epilogue (ea != nullptr, fp16 output): C = half(half(ea + eb) + half(acc)), ea / eb of
// C's shape.
// Paired rows (pair != 0; two matrices of N rows, one fp16 row of activations): row n of the first
// matrix (gate) and row n of the second (up) are multiplied by one wave and C[n] (the first
// output) = half(silu(half(gate)) * half(up)), silu(g) = g / (1 + exp(-g)).
struct GemvFuse {
    int pair = 0;
    int kind = 0;
    const void* R = nullptr;
    const void* w = nullptr;
    int w_f32 = 0;
    float eps = 0.0f;
    const void* ea = nullptr;
    const void* eb = nullptr;
};

// Kernel launchers (validated arguments; return a hipError_t from the launch).
// GEMV kernel families: M = 1 runs the v_dot2 kernels; 2 <= M < gemv_max_m() runs the matrix-core GEMV
// where it is faster (Q4_K), else the v_dot2 kernels.  identity: every M on the family of M = 1's
// choice for identity (the matrix-core GEMV for Q4_K), so that row m of any M is bit-identical to the
// M = 1 call, the reference's invariant (tests/test_phase5_scale.py:274-310, 360-379).
hipError_t launch_gemv(int ggml_type, const void* A, int a_dtype, const void* W, void* C,
                       int c_dtype, int M, int N, int K, hipStream_t stream, bool identity);
// Several weight matrices (same type and K) times the same activations in one launch; returns
// hipErrorNotSupported when the fused path does not apply (the caller then launches each).
hipError_t launch_gemv_fused(int ggml_type, const void* A, int a_dtype, int c_dtype, int M, int K,
                             const void* const* W, void* const* C, const int* N, int count, hipStream_t stream,
                             bool identity);
// GEMV of up to gemv_max_fused() matrices sharing fp16 activations A [M, K] (M < gemv_max_m()), with
// work folded in (`fz`); hipErrorNotSupported when the shapes or alignments need a kernel without
// the folding (the caller then runs the separate kernels).
hipError_t launch_gemv_ex(int ggml_type, const void* A, int c_dtype, int M, int K, const void* const* W, void* const* C,
                          const int* N, int count, const GemvFuse& fz, hipStream_t stream);
int gemv_max_fused();
// Matrix-core GEMV (qmm_gemv_mfma.hip) for the GEMV family's M: Q4_K and Q6_K weights, `count` (1..4)
// matrices sharing the activations; hipErrorNotSupported when the shape is outside it (then no row of
// any M of that shape takes it, so rows stay bit-identical across M).  gemv_mfma_min_m: the smallest M
// that runs it for the format (INT_MAX: none), in row-identity mode or not.
int gemv_mfma_min_m(int ggml_type, bool identity);
hipError_t launch_gemv_mfma(int ggml_type, const void* A, int a_dtype, int c_dtype, int M, int K, const void* const* W,
                            void* const* C, const int* N, int count, hipStream_t stream);
hipError_t launch_gemm_prefill(int ggml_type, const void* A, int a_dtype, const void* W, void* C,
                               int c_dtype, int M, int N, int K, hipStream_t stream);
bool gemm_prefill_supported(int ggml_type, int a_dtype, int c_dtype, int M, int N, int K,
                            const void* A, const void* W, const void* C);
// Prefill of several weight matrices (same type and K, each passing gemm_prefill_supported) times
// the same activations in one launch: their output tiles share one grid.
hipError_t launch_gemm_prefill_fused(int ggml_type, const void* A, int a_dtype, int c_dtype, int M, int K,
                                     const void* const* W, void* const* C, const int* N, int count, hipStream_t stream);
int prefill_max_fused();
// The prefill of qmm_gemm_noalloc: the workspace (f16 activations, split-K partials) is a static
// per-device scratch array of kNoAllocScratchBytes; nothing is allocated.  `need` receives the
// bytes the launch plan uses; when it exceeds the array, nothing is launched and the call returns
// hipErrorOutOfMemory.  Calls that overlap on one device share the array and race.
constexpr size_t kNoAllocScratchBytes = size_t{64} << 20;
hipError_t launch_gemm_prefill_noalloc(int ggml_type, const void* A, int a_dtype, const void* W, void* C, int c_dtype,
                                       int M, int N, int K, hipStream_t stream, size_t* need);
// Frees the prefill workspaces (f16 activations, split-K partials) of every device, after
// synchronizing each device.
hipError_t release_prefill_workspaces();
hipError_t launch_embed(int ggml_type, const void* table, int64_t n_rows, int64_t row_bytes, int hidden,
                        const int64_t* ids, int64_t n_ids, void* out, int out_dtype, int* bad, hipStream_t stream);
hipError_t launch_dequantize(int ggml_type, const void* W, void* out, int out_dtype,
                             int64_t num_elements, hipStream_t stream);

// File -> memory loading (qmm_upload.hip).  Status code (QMM_*) and message.
struct UploadStatus {
    int code;
    std::string msg;
};
using FileRange = qmm_file_range;
UploadStatus read_file_ranges(const char* path, const FileRange* ranges, int count, int threads);
UploadStatus upload_file_ranges(const char* path, const FileRange* ranges, int count, int64_t chunk_bytes, int depth,
                                int threads, hipStream_t stream);
// Frees the pinned staging buffers that upload_file_ranges keeps between calls.
void release_upload_staging();

// Layer kernels and pipeline (qmm_layer.hip).  fp16 activations; launchers return the launch's
// hipError_t, the pool / pipeline calls a status and message.
using LayerStatus = UploadStatus;
hipError_t launch_rmsnorm(const void* x, const void* res, const void* w, int w_f32, void* h_out, void* out, int M, int K,
                          float eps, hipStream_t stream);
hipError_t launch_residual_add(const void* x, const void* r, void* out, int64_t n, hipStream_t stream);
hipError_t launch_swiglu(const void* g, const void* u, void* out, int64_t n, hipStream_t stream);
hipError_t launch_rope(const void* q, void* q_out, int n_q, const void* k, void* k_out, const void* v, void* v_out, int n_k,
                       int seq_len, int head_dim, int pos_offset, float freq_base, bool neox, hipStream_t stream);
size_t attention_workspace_bytes(int q_len, int heads, int head_dim, int kv_len);
hipError_t launch_attention(const void* Q, const void* K, const void* V, void* out, void* part, int q_len, int kv_len,
                            int heads, int kv_heads, int head_dim, int start_pos, float scale, bool causal,
                            hipStream_t stream);
LayerStatus kv_cache_init(int layers, int max_seq, int kv_heads, int head_dim);
LayerStatus kv_cache_free();
LayerStatus kv_cache_layer(int layer, int start, int q_len, int kv_heads, int head_dim, _Float16** k, _Float16** v,
                           int* max_seq);
LayerStatus forward_layer(const qmm_layer_config& cfg, const qmm_layer_weights& w, const void* x_in, void* x_out,
                          int layer_idx, int seq_len, int pos_offset, hipStream_t stream);
hipError_t layer_scratch(hipStream_t stream, size_t bytes, void** out);
hipError_t release_layer_workspaces();

}  // namespace qmm
