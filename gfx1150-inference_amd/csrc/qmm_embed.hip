// Embedding lookup with dequantization: out[i, :] = dequant(row ids[i] of the token table).
// Replaces the reference's CPU embed_tokens (src/tokenizer.py:336-389: gather the packed rows,
// then dequantize_*_cpu), so token embeddings are produced in HBM next to the layer inputs.
//
// One thread produces one 32-element group of one output row (16-byte stores), with the same
// per-group decoder as the dequantize kernel, so results are bit-exact with the reference's CPU
// dequantizers.  F16 tables are copied, F32 tables rounded once (RNE).  An id outside
// [0, n_rows) never addresses the table: its row is read as row 0, its output is zero-filled and
// *bad (when given) is set to 1.
#include "qmm_device.h"

namespace qmm {
namespace {

template <int T>
__device__ __forceinline__ void row_group(const uint8_t* __restrict__ row, int64_t j, float w[32]) {
    if constexpr (T == QMM_TYPE_F16) {
        const uint16_t* p = reinterpret_cast<const uint16_t*>(row) + 32 * j;
#pragma unroll
        for (int e = 0; e < 32; ++e) w[e] = half_bits_to_float(p[e]);
    } else if constexpr (T == QMM_TYPE_F32) {
        const float* p = reinterpret_cast<const float*>(row) + 32 * j;
#pragma unroll
        for (int e = 0; e < 32; ++e) w[e] = p[e];
    } else {
        group_weights_bytewise<T>(row, j, w);
    }
}

template <int T, int OUT>
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t* __restrict__ table, int64_t n_rows,
                                                    int64_t row_bytes, int groups_per_row,
                                                    const int64_t* __restrict__ ids, int64_t n_ids,
                                                    void* __restrict__ out, int* __restrict__ bad) {
    const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= n_ids * groups_per_row) return;
    const int64_t i = g / groups_per_row;
    const int64_t j = g - i * groups_per_row;
    const int64_t id = ids[i];
    const bool ok = id >= 0 && id < n_rows;
    if constexpr (T == QMM_TYPE_F16 && OUT == QMM_DTYPE_F16) {
        // fp16 table to fp16 output: the bits are copied (NaN payloads included)
        const uint16_t* p = reinterpret_cast<const uint16_t*>(table + (ok ? id : 0) * row_bytes) + 32 * j;
        uint32_t q[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) q[e] = ok ? (static_cast<uint32_t>(p[2 * e]) | (static_cast<uint32_t>(p[2 * e + 1]) << 16)) : 0u;
        if (!ok && bad != nullptr && j == 0) *bad = 1;
        uint4* o = reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + 32 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = make_uint4(q[4 * e], q[4 * e + 1], q[4 * e + 2], q[4 * e + 3]);
        return;
    }
    float w[32];
    row_group<T>(table + (ok ? id : 0) * row_bytes, j, w);
    if (!ok) {
#pragma unroll
        for (int e = 0; e < 32; ++e) w[e] = 0.0f;
        if (bad != nullptr && j == 0) *bad = 1;
    }
    if constexpr (OUT == QMM_DTYPE_F32) {
        float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + 32 * g);
#pragma unroll
        for (int q = 0; q < 8; ++q) o[q] = make_float4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
    } else {
        uint32_t p[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const uint32_t lo = OUT == QMM_DTYPE_F16 ? float_to_half_bits(w[2 * q]) : float_to_bf16_bits(w[2 * q]);
            const uint32_t hi = OUT == QMM_DTYPE_F16 ? float_to_half_bits(w[2 * q + 1]) : float_to_bf16_bits(w[2 * q + 1]);
            p[q] = lo | (hi << 16);
        }
        uint4* o = reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + 32 * g);
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = make_uint4(p[4 * q], p[4 * q + 1], p[4 * q + 2], p[4 * q + 3]);
    }
}

template <int T>
hipError_t launch_t(const void* table, int64_t n_rows, int64_t row_bytes, int hidden, const int64_t* ids,
                    int64_t n_ids, void* out, int out_dtype, int* bad, hipStream_t stream) {
    const int gpr = hidden / 32;
    const int64_t total = n_ids * gpr;
    const dim3 block(256), grid(static_cast<unsigned>((total + 255) / 256));
    const uint8_t* tb = static_cast<const uint8_t*>(table);
    switch (out_dtype) {
        case QMM_DTYPE_F32:
            hipLaunchKernelGGL((embed_kernel<T, QMM_DTYPE_F32>), grid, block, 0, stream, tb, n_rows, row_bytes, gpr, ids,
                               n_ids, out, bad);
            break;
        case QMM_DTYPE_F16:
            hipLaunchKernelGGL((embed_kernel<T, QMM_DTYPE_F16>), grid, block, 0, stream, tb, n_rows, row_bytes, gpr, ids,
                               n_ids, out, bad);
            break;
        default:
            hipLaunchKernelGGL((embed_kernel<T, QMM_DTYPE_BF16>), grid, block, 0, stream, tb, n_rows, row_bytes, gpr,
                               ids, n_ids, out, bad);
            break;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_embed(int ggml_type, const void* table, int64_t n_rows, int64_t row_bytes, int hidden,
                        const int64_t* ids, int64_t n_ids, void* out, int out_dtype, int* bad, hipStream_t stream) {
    if (n_ids == 0) return hipSuccess;
    switch (ggml_type) {
        case QMM_TYPE_F32: return launch_t<QMM_TYPE_F32>(table, n_rows, row_bytes, hidden, ids, n_ids, out, out_dtype, bad, stream);
        case QMM_TYPE_F16: return launch_t<QMM_TYPE_F16>(table, n_rows, row_bytes, hidden, ids, n_ids, out, out_dtype, bad, stream);
        case QMM_TYPE_Q4_0: return launch_t<QMM_TYPE_Q4_0>(table, n_rows, row_bytes, hidden, ids, n_ids, out, out_dtype, bad, stream);
        case QMM_TYPE_Q8_0: return launch_t<QMM_TYPE_Q8_0>(table, n_rows, row_bytes, hidden, ids, n_ids, out, out_dtype, bad, stream);
        case QMM_TYPE_Q4_K: return launch_t<QMM_TYPE_Q4_K>(table, n_rows, row_bytes, hidden, ids, n_ids, out, out_dtype, bad, stream);
        case QMM_TYPE_Q6_K: return launch_t<QMM_TYPE_Q6_K>(table, n_rows, row_bytes, hidden, ids, n_ids, out, out_dtype, bad, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qmm
