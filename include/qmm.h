/*
 * qmm.h - C ABI of libqmm_gfx950.so: fused dequantize-and-multiply over GGUF
 * Q4_0 / Q8_0 / Q4_K / Q6_K weight blocks on MI355X (gfx950).
 *
 * Conventions
 *   - Weights are N x K, row-major, packed in native GGUF blocks along K
 *     (GGUF ne[0] = K; reference src/gguf_parser.py:89-101).  C = A @ W^T.
 *   - Every function returns a qmm_status; on failure qmm_last_error() returns a
 *     thread-local message.  No C++ exception crosses this boundary.
 *   - `stream` is a hipStream_t passed as an opaque pointer (NULL = the null
 *     stream).  Device-pointer entry points are asynchronous on that stream.
 *   - Type ids are the GGMLType integers (reference src/gguf_parser.py:22-36):
 *     1 = F16, 2 = Q4_0, 8 = Q8_0, 12 = Q4_K, 14 = Q6_K.
 *   - Activation/output dtypes: QMM_DTYPE_F32, QMM_DTYPE_F16 (IEEE binary16),
 *     QMM_DTYPE_BF16 (dequantize output only).
 */
#ifndef QMM_H
#define QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum qmm_status {
    QMM_OK = 0,
    QMM_ERR_INVALID_ARGUMENT = 1, /* maps to the reference's std::invalid_argument / ValueError */
    QMM_ERR_UNSUPPORTED = 2,      /* valid request the library does not implement */
    QMM_ERR_HIP = 3,              /* HIP runtime error; maps to std::runtime_error / RuntimeError */
    QMM_ERR_IO = 4,               /* file open / read failure (qmm_upload_file, qmm_read_file); OSError */
    QMM_ERR_OUT_OF_RANGE = 5      /* index outside the KV cache pool (std::out_of_range); IndexError */
};

enum qmm_ggml_type {
    QMM_TYPE_F32 = 0,   /* token-embedding tables only (qmm_embed) */
    QMM_TYPE_F16 = 1,   /* dense fp16 rows: GEMM weights (matmul_nt) and embedding tables */
    QMM_TYPE_Q4_0 = 2,
    QMM_TYPE_Q8_0 = 8,
    QMM_TYPE_Q4_K = 12,
    QMM_TYPE_Q6_K = 14
};

enum qmm_dtype {
    QMM_DTYPE_F32 = 0,
    QMM_DTYPE_F16 = 1,
    QMM_DTYPE_BF16 = 2
};

/* Thread-local message of the last failed call on this thread ("" if none). */
const char* qmm_last_error(void);

/* ABI version of this library (major * 1000 + minor). */
int qmm_version(void);

/* Packed byte size of an N x K weight; 0 if K is not a multiple of the block size.
 * Replaces weight_bytes_for_type (reference src/kernels/attention.hip:553-570). */
size_t qmm_weight_bytes(int ggml_type, int64_t n, int64_t k);

/* ---------------------------------------------------------------------------------
 * Device-pointer API (primary).
 * --------------------------------------------------------------------------------- */

/* C[M,N] (c_dtype) = A[M,K] (a_dtype) @ dequant(W)[N,K]^T with fp32 accumulation.
 * M < qmm_gemv_max_m() (17) runs the bandwidth-bound GEMV kernels; larger M runs the f16-MFMA
 * prefill GEMM (a 32-row tile up to M = 32), whose rows agree with the M = 1 call within the
 * prefill accuracy bound.  Among GEMV sizes each format takes the faster of two kernel families:
 * Q4_K the matrix-core GEMV from M = 2, Q6_K from M = 3 (16-byte aligned weights, K a multiple of
 * 2048), and the v_dot2 GEMV below that and for the other formats.  Rows are bit-identical for
 * every M within one family, and the two families agree within the GEMV accuracy bound.  With
 * qmm_set_row_identity(1) every GEMV-size M runs one family (Q4_K the matrix-core GEMV, the other
 * formats the v_dot2 GEMV), so that every row is bit-identical to the M = 1 call, as in the
 * reference.
 * Generalises launch_matmul_q{4_0,8_0,4_k,6_k}_device (reference
 * src/kernels/dequantize.h:98-132, dispatch at dequantize.hip:778/896/1014/1132). */
int qmm_gemm(int ggml_type, const void* A, int a_dtype, const void* W, void* C, int c_dtype,
             int M, int N, int K, void* stream);

/* qmm_gemm that allocates nothing (no counterpart in the reference): for callers that cannot
 * call hipMalloc - code under HIP graph capture, tight serving loops, harnesses that forbid it.
 * Same arguments, kernels and results as qmm_gemm.  The prefill sizes' workspace (f16 copy of
 * fp32 or unaligned activations, split-K partial tiles) is a static per-device scratch array of
 * qmm_noalloc_scratch_bytes() bytes, held by every GPU the library runs on until the process
 * ends; a call needing more returns QMM_ERR_UNSUPPORTED and launches nothing.  All calls on one
 * GPU share that array.  Eager calls take turns on it: a call on another stream than the previous
 * one that used the array waits for that call's kernels (hipStreamWaitEvent on a per-device event
 * created by the first call).  Calls under stream capture are not ordered that way: replays of a
 * captured call that overlap other calls on the same GPU race, and the caller orders them. */
int qmm_gemm_noalloc(int ggml_type, const void* A, int a_dtype, const void* W, void* C, int c_dtype,
                     int M, int N, int K, void* stream);
size_t qmm_noalloc_scratch_bytes(void);

/* One GEMM of a batch.  ev_before / ev_after are optional hipEvent_t handles (NULL = none)
 * recorded on the batch's stream immediately before / after this GEMM's kernel. */
typedef struct qmm_gemm_desc {
    int ggml_type;
    const void* A;
    int a_dtype;
    const void* W;
    void* C;
    int c_dtype;
    int M, N, K;
    void* ev_before;
    void* ev_after;
} qmm_gemm_desc;

/* Validates every descriptor, then launches them back to back on `stream` in order
 * (no host synchronisation).  Replaces the per-projection launches of the reference's
 * device-resident layer pipeline (src/kernels/attention.hip:650-687, project_on_device
 * :572-599) for callers that keep weights resident.
 * Consecutive descriptors with the same A, a_dtype, c_dtype, ggml_type, M and K, no event
 * between them and no output overlapping another output or any input (q/k/v, gate/up) run as
 * one launch.  GEMV sizes (M < qmm_gemv_max_m()) give results bit-identical to separate calls;
 * prefill sizes share one grid, which may change how K is split over workgroups and therefore
 * the fp32 summation order (within the prefill accuracy bound). */
int qmm_gemm_batch(const qmm_gemm_desc* descs, int count, void* stream);

/* dequant(W) -> out[num_elements] in out_dtype (F16, BF16 or F32), bit-exact.
 * Generalises dequantize_{q4_0,q8_0,q4_k,q6_k}_kernel launches
 * (reference src/kernels/dequantize.hip:68-88, 213-229, 335-371, 508-544). */
int qmm_dequantize(int ggml_type, const void* W, void* out, int out_dtype,
                   int64_t num_elements, void* stream);

/* Token-embedding lookup: out[i, :] = dequant(table row ids[i]) for i < n_ids, `hidden` elements
 * per row, in out_dtype (F16 as the reference, BF16 or F32), bit-exact with the reference's CPU
 * dequantizers.  Replaces embed_tokens (reference src/tokenizer.py:336-389), which gathers the
 * packed rows of token_embd.weight and dequantizes them on the CPU.
 * table: n_rows rows of GGUF blocks (Q4_0, Q8_0, Q4_K, Q6_K) or of F16 / F32 values (ggml_type
 * QMM_TYPE_F16 / QMM_TYPE_F32), device memory; ids: n_ids int64 device values; out: 16-byte
 * aligned device buffer.  hidden must be a positive multiple of 32 (256 for Q4_K / Q6_K).
 * The reference raises ValueError for an id outside [0, n_rows) before any work; ids here live
 * on the device, so such an id reads nothing out of bounds: its output row is zero-filled and
 * *bad (a device int the caller zeroes first; may be NULL) is set to 1.  The Python wrapper
 * qmm.embed_tokens validates host ids exactly like the reference. */
int qmm_embed(int ggml_type, const void* table, int64_t n_rows, int hidden, const int64_t* ids,
              int64_t n_ids, void* out, int out_dtype, int* bad, void* stream);

/* Largest M served by the GEMV family (exclusive bound; 17 by default), and the prefill threshold. */
int qmm_gemv_max_m(void);

/* Sets that threshold for the process (1 <= m <= 65536; QMM_ERR_INVALID_ARGUMENT otherwise).
 * No counterpart in the reference, whose TILE_M = 4 kernels keep every row of every M
 * bit-identical to the M = 1 call (src/kernels/dequantize.hip:152-210, 440-505, 616-685); a
 * caller that needs that invariant beyond M = 16 raises the threshold above its largest M and
 * gets the GEMV family's rows, at the GEMV's cost (its per-row vector work grows with M).  Calls
 * read the threshold once (a qmm_gemm_batch call for all its descriptors); changing it while
 * other threads issue calls changes which family their later calls take. */
int qmm_set_gemv_max_m(int m);

/* Per-thread threshold for calls issued by the calling thread (1 <= m <= 65536), or 0 to use the
 * process value again; QMM_ERR_INVALID_ARGUMENT otherwise.  No counterpart in the reference: lets
 * one caller keep bit-identical rows beyond M = 16 without moving the threshold for every other
 * caller.  qmm_gemv_max_m() reports the calling thread's effective threshold. */
int qmm_set_thread_gemv_max_m(int m);

/* Row-identity mode of the calling thread (0 or 1; QMM_ERR_INVALID_ARGUMENT otherwise); 0 by
 * default.  No counterpart in the reference, whose kernels keep every row of every GEMV-size M
 * bit-identical to the M = 1 call (its tests assert it, tests/test_phase5_scale.py:274-310).
 * With 1, qmm_gemm, qmm_gemm_noalloc and qmm_gemm_batch run every M < qmm_gemv_max_m() of a
 * format on one kernel family, so that rows match the M = 1 call bit for bit: Q4_K on the
 * matrix-core GEMV (its M = 1 a few microseconds slower than the v_dot2 GEMV on large matrices),
 * Q6_K and the other formats on the v_dot2 GEMV (Q6_K's M >= 3 then slower than the matrix-core
 * GEMV).  The reference-API launchers (qmm_matmul_q*_device / _host) always run in this mode. */
int qmm_set_row_identity(int on);
int qmm_row_identity(void);

/* Per-type device launchers with the reference's argument meaning: fp16 A [M,K],
 * packed B [N,K], fp16 C [M,N], all device pointers, on `stream`.
 * Replace launch_matmul_q4_0_device / _q8_0_ / _q4_k_ / _q6_k_device
 * (reference src/kernels/dequantize.h:98-132, dequantize.hip:764-818, 882-936,
 * 1000-1054, 1118-1172). */
int qmm_matmul_q4_0_device(const void* d_A_fp16, const void* d_B_q4, void* d_C_fp16,
                           int M, int N, int K, void* stream);
int qmm_matmul_q8_0_device(const void* d_A_fp16, const void* d_B_q8, void* d_C_fp16,
                           int M, int N, int K, void* stream);
int qmm_matmul_q4_k_device(const void* d_A_fp16, const void* d_B_q4k, void* d_C_fp16,
                           int M, int N, int K, void* stream);
int qmm_matmul_q6_k_device(const void* d_A_fp16, const void* d_B_q6k, void* d_C_fp16,
                           int M, int N, int K, void* stream);
/* Dense fp16: C[M,N] = A[M,K] @ B_nt[N,K]^T (qmm_gemm with QMM_TYPE_F16).  Replaces
 * launch_matmul_fp16_nt_device (reference src/kernels/matmul.hip:397-439). */
int qmm_matmul_fp16_nt_device(const void* d_A, const void* d_B_nt, void* d_C, int M, int N, int K, void* stream);

/* ---------------------------------------------------------------------------------
 * Host-pointer API: the reference's synchronous copy-in / compute / copy-out
 * semantics through a grow-only device workspace.
 * --------------------------------------------------------------------------------- */

/* Replace launch_matmul_q{4_0,8_0,4_k,6_k} (reference src/kernels/dequantize.h:34-41,
 * 51-58, 69-76, 86-93; dequantize.hip:820-845, 938-963, 1056-1081, 1174-1199). */
int qmm_matmul_q4_0_host(const void* h_A_fp16, const void* h_B_q4, void* h_C_fp16,
                         int M, int N, int K);
int qmm_matmul_q8_0_host(const void* h_A_fp16, const void* h_B_q8, void* h_C_fp16,
                         int M, int N, int K);
int qmm_matmul_q4_k_host(const void* h_A_fp16, const void* h_B_q4k, void* h_C_fp16,
                         int M, int N, int K);
int qmm_matmul_q6_k_host(const void* h_A_fp16, const void* h_B_q6k, void* h_C_fp16,
                         int M, int N, int K);

/* Replace launch_dequantize_q{4_0,8_0,4_k,6_k} (reference src/kernels/dequantize.h:25-29,
 * 44-48, 62-66, 79-83; dequantize.hip:729-762, 847-880, 965-998, 1083-1116). */
int qmm_dequantize_q4_0_host(const void* h_q4, void* h_fp16_out, int num_elements);
int qmm_dequantize_q8_0_host(const void* h_q8, void* h_fp16_out, int num_elements);
int qmm_dequantize_q4_k_host(const void* h_q4k, void* h_fp16_out, int num_elements);
int qmm_dequantize_q6_k_host(const void* h_q6k, void* h_fp16_out, int num_elements);

/* ---------------------------------------------------------------------------------
 * Transformer layer around the projections (device pointers, fp16 activations,
 * asynchronous on `stream`).  fp32 arithmetic, one rounding per stored fp16 value, as the
 * reference's kernels (src/kernels/rmsnorm.hip, rope.hip, attention.hip, mlp.hip).
 * --------------------------------------------------------------------------------- */

/* out[m, :] = half(x[m, :] * rsqrt(mean(x[m, :]^2) + eps) * weight); weight_dtype F16 or F32
 * (an F32 weight is rounded to f16 first, as the reference's host does).
 * Replaces launch_rmsnorm_fp16_device (src/kernels/rmsnorm.h:44-51). */
int qmm_rmsnorm(const void* x, const void* weight, int weight_dtype, void* out, int M, int K, float eps,
                void* stream);
/* h_out = half(x + residual); norm_out = rmsnorm(h_out).  Replaces
 * launch_rmsnorm_residual_fp16_device (src/kernels/rmsnorm.h:53-62). */
int qmm_rmsnorm_residual(const void* x, const void* residual, const void* weight, int weight_dtype, void* h_out,
                         void* norm_out, int M, int K, float eps, void* stream);
/* out = half(x + residual), n elements.  Replaces launch_residual_add_fp16_device (:64-69). */
int qmm_residual_add(const void* x, const void* residual, void* out, int64_t n, void* stream);
/* out = half(silu(gate) * up), n elements.  Replaces launch_swiglu_fp16_device (src/kernels/mlp.h:13-18). */
int qmm_swiglu(const void* gate, const void* up, void* out, int64_t n, void* stream);
/* RoPE of x [seq_len, num_heads, head_dim] at positions pos_offset + row: pairs (2i, 2i + 1), or
 * (i, i + head_dim / 2) when neox != 0; inv_freq_i = 1 / freq_base^(2i / head_dim).
 * Replaces launch_rope_fp16_device (src/kernels/rope.h:21-30). */
int qmm_rope(const void* x_in, void* x_out, int seq_len, int num_heads, int head_dim, int pos_offset,
             float freq_base, int neox, void* stream);
/* Grouped-query attention: Q [q_len, num_heads, head_dim], K / V [kv_len, num_kv_heads, head_dim],
 * query head h reads KV head h / (num_heads / num_kv_heads); causal rows m see keys
 * < min(kv_len, start_pos + m + 1); scale 0 means 1 / sqrt(head_dim); head_dim <= 256.
 * Replaces launch_gqa_attention_fp16 (src/kernels/attention.hip:228-284). */
int qmm_gqa_attention(const void* Q, const void* K, const void* V, void* out, int q_len, int kv_len, int num_heads,
                      int num_kv_heads, int head_dim, int start_pos, float scale, int causal, void* stream);

/* KV cache pool of the current device: [num_layers][max_seq_len][num_kv_heads][head_dim] fp16 for
 * K and for V (grow-only).  Replace init_device_kv_cache_fp16 / free_device_kv_cache_fp16
 * (src/kernels/attention.hip:286-300). */
int qmm_kv_cache_init(int num_layers, int max_seq_len, int num_kv_heads, int head_dim);
int qmm_kv_cache_free(void);
/* Writes K_new / V_new ([q_len, num_kv_heads, head_dim], rotated) into layer `layer_idx` of the
 * pool at start_pos, then attends over [0, start_pos + q_len).  Replaces
 * launch_gqa_attention_cached_fp16_device (src/kernels/attention.hip:376-440). */
int qmm_gqa_attention_cached(const void* Q, const void* K_new, const void* V_new, void* out, int layer_idx, int q_len,
                             int start_pos, int num_heads, int num_kv_heads, int head_dim, float scale, int causal,
                             void* stream);

typedef struct qmm_layer_config {
    int hidden_size, intermediate_size, num_heads, num_kv_heads, head_dim;
    float rms_norm_eps, rope_freq_base;
    int rope_neox;
    float scale; /* 0: 1 / sqrt(head_dim) */
} qmm_layer_config;

/* Device-resident weights of one layer: norms are F16 or F32 vectors (dtype QMM_DTYPE_*);
 * projections are F16 rows or packed GGUF matrices (type 1 / 2 / 8 / 12 / 14), N x K as in qmm_gemm. */
typedef struct qmm_layer_weights {
    const void* attn_norm;
    int attn_norm_dtype;
    const void* wq;
    int wq_type;
    const void* wk;
    int wk_type;
    const void* wv;
    int wv_type;
    const void* wo;
    int wo_type;
    const void* ffn_norm;
    int ffn_norm_dtype;
    const void* wgate;
    int wgate_type;
    const void* wup;
    int wup_type;
    const void* wdown;
    int wdown_type;
    /* Optional fp16 biases (NULL = none): q [num_heads * head_dim], k and v [num_kv_heads * head_dim],
     * attention output [hidden_size].  Each is added in fp32 to its projection's fp16 output, which
     * is rounded to fp16 once more, as the reference's layer does (src/layer.py:274-282, 344-346;
     * an F32 GGUF bias is rounded to fp16 first, layer.py:161-167). */
    const void* bq;
    const void* bk;
    const void* bv;
    const void* bo;
} qmm_layer_weights;

/* x_out [seq_len, hidden] = one Llama layer on x_in (fp16, device): RMSNorm, q/k/v (one fused
 * launch), RoPE with the K/V cache write at pos_offset, causal GQA over the cache, o, residual +
 * RMSNorm, gate/up (one fused launch), SwiGLU, down, residual.  Weights stay where they are (no
 * per-call copies); activations use a grow-only per-stream workspace.  Replaces
 * launch_forward_layer_cached_fp16 (src/kernels/attention.hip:603-695), which copies the hidden
 * state and every weight from the host per call. */
int qmm_forward_layer(const qmm_layer_config* cfg, const qmm_layer_weights* w, const void* x_in, void* x_out,
                      int layer_idx, int seq_len, int pos_offset, void* stream);

/* ---------------------------------------------------------------------------------
 * Host-pointer forms of the dense matmuls and layer operations: the reference's synchronous
 * launchers (operands copied in, result copied out, null stream).  fp16 throughout; the KV
 * pool is the device pool above.
 * --------------------------------------------------------------------------------- */

/* C[M,N] = A[M,K] @ B_nt[N,K]^T.  Replaces launch_matmul_fp16_nt (src/kernels/matmul.hip:441-463). */
int qmm_matmul_fp16_nt_host(const void* h_A, const void* h_B_nt, void* h_C, int M, int N, int K);
/* C[M,N] = A[M,K] @ B[K,N] (B transposed on the device, then as above).  Replaces
 * launch_matmul_fp16 (src/kernels/matmul.hip:340-395). */
int qmm_matmul_fp16_host(const void* h_A, const void* h_B, void* h_C, int M, int N, int K);
/* Replace launch_rmsnorm_fp16, launch_rmsnorm_residual_fp16, launch_residual_add_fp16
 * (src/kernels/rmsnorm.h:10-42). */
int qmm_rmsnorm_host(const void* h_x, const void* h_weight, void* h_out, int M, int K, float eps);
int qmm_rmsnorm_residual_host(const void* h_x, const void* h_residual, const void* h_weight, void* h_h_out,
                              void* h_norm_out, int M, int K, float eps);
int qmm_residual_add_host(const void* h_x, const void* h_residual, void* h_out, int64_t num_elements);
/* Replaces launch_swiglu_fp16 (src/kernels/mlp.h:6-11). */
int qmm_swiglu_host(const void* h_gate, const void* h_up, void* h_out, int64_t num_elements);
/* Replaces launch_rope_fp16 (src/kernels/rope.h:10-19). */
int qmm_rope_host(const void* h_in, void* h_out, int seq_len, int num_heads, int head_dim, int pos_offset,
                  float freq_base, int neox);
/* Replaces launch_gqa_attention_fp16 (src/kernels/attention.hip:228-284). */
int qmm_gqa_attention_host(const void* h_Q, const void* h_K, const void* h_V, void* h_out, int q_len, int kv_len,
                           int num_heads, int num_kv_heads, int head_dim, int start_pos, float scale, int causal);
/* Replaces launch_gqa_attention_cached_fp16 (src/kernels/attention.hip:302-374). */
int qmm_gqa_attention_cached_host(const void* h_Q, const void* h_K_new, const void* h_V_new, void* h_out, int layer_idx,
                                  int q_len, int start_pos, int num_heads, int num_kv_heads, int head_dim, float scale,
                                  int causal);
/* qmm_forward_layer with host activations and host weights (all copied to the device per call,
 * as the reference does).  Replaces launch_forward_layer_cached_fp16
 * (src/kernels/attention.hip:603-695). */
int qmm_forward_layer_host(const qmm_layer_config* cfg, const qmm_layer_weights* w, const void* h_x_in, void* h_x_out,
                           int layer_idx, int seq_len, int pos_offset);

/* One byte range of a file and its destination. */
typedef struct qmm_file_range {
    int64_t offset; /* byte offset in the file */
    int64_t bytes;
    void* dst;      /* device memory (qmm_upload_file) or host memory (qmm_read_file) */
} qmm_file_range;

/* Copies byte ranges of a file (the packed tensors of a GGUF model) into device memory once, so
 * the model stays resident in HBM.  Replaces the reference's per-call weight copies (the host
 * wrappers, src/kernels/dequantize.hip:729-762 and siblings; project_on_device,
 * src/kernels/attention.hip:572-586) and its mmap weight streaming (WeightStreamer,
 * src/weight_loader.py:99-187) for MI355X, whose HBM holds a whole quantized model.
 * `threads` reader threads pread() pieces of each chunk of at most chunk_bytes (4 MiB .. 4 GiB)
 * into one of `depth` (2..8) pinned staging buffers, and each chunk is copied with
 * hipMemcpyAsync on `stream`, so reading the next chunk overlaps the copy of the previous one.
 * Returns after every copy has completed.  Ranges must lie inside the file.  The staging
 * buffers are kept for the next call (grow-only) and freed by qmm_release_workspace(); loads
 * from several threads run one at a time. */
int qmm_upload_file(const char* path, const qmm_file_range* ranges, int count, int64_t chunk_bytes, int depth,
                    int threads, void* stream);

/* The same parallel reader into host memory (no staging, no GPU).  The reference's analogue is
 * the zero-copy mmap view (WeightStreamer.get_tensor_view, src/weight_loader.py:99-110). */
int qmm_read_file(const char* path, const qmm_file_range* ranges, int count, int threads);

/* Release the host-API workspace (the reference frees its static Q4Workspace at exit,
 * dequantize.hip:715-719) and the prefill workspaces of qmm_gemm (f16 activations, split-K
 * partials; grow-only per device and stream).  Synchronizes each device that holds one, so it
 * is safe to call at any time; the next call that needs a workspace re-grows it. */
int qmm_release_workspace(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* QMM_H */
