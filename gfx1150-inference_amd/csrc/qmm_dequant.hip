// Dequantize packed GGUF blocks to fp16 / bf16 / fp32, bit-exact with the reference's CPU
// dequantizers (src/gguf_parser.py:374-589): every weight is a*code (exact in fp32) minus b,
// rounded once to fp32, then once (round-to-nearest-even) to the output type.
//
// Replaces dequantize_{q4_0,q8_0,q4_k,q6_k}_kernel (reference src/kernels/dequantize.hip:68-88,
// 213-229, 335-371, 508-544).  One thread produces one 32-weight group and writes it with
// 16-byte stores; consecutive threads write consecutive groups.
#include "qmm_device.h"

namespace qmm {
namespace {

template <int T, int OUT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ W, void* __restrict__ out,
                                                      int64_t groups) {
    const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    float w[32];
    group_weights_bytewise<T>(W, g, w);
    if constexpr (OUT == QMM_DTYPE_F32) {
        float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + 32 * g);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = make_float4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
    } else {
        uint32_t p[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            uint32_t lo, hi;
            if constexpr (OUT == QMM_DTYPE_F16) {
                lo = float_to_half_bits(w[2 * i]);
                hi = float_to_half_bits(w[2 * i + 1]);
            } else {
                lo = float_to_bf16_bits(w[2 * i]);
                hi = float_to_bf16_bits(w[2 * i + 1]);
            }
            p[i] = lo | (hi << 16);
        }
        uint4* o = reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + 32 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = make_uint4(p[4 * i], p[4 * i + 1], p[4 * i + 2], p[4 * i + 3]);
    }
}

template <int T>
hipError_t launch_t(const void* W, void* out, int out_dtype, int64_t groups, hipStream_t stream) {
    const dim3 block(256);
    const dim3 grid(static_cast<unsigned>((groups + 255) / 256));
    const uint8_t* w = static_cast<const uint8_t*>(W);
    switch (out_dtype) {
        case QMM_DTYPE_F32:
            hipLaunchKernelGGL((dequant_kernel<T, QMM_DTYPE_F32>), grid, block, 0, stream, w, out, groups);
            break;
        case QMM_DTYPE_F16:
            hipLaunchKernelGGL((dequant_kernel<T, QMM_DTYPE_F16>), grid, block, 0, stream, w, out, groups);
            break;
        default:
            hipLaunchKernelGGL((dequant_kernel<T, QMM_DTYPE_BF16>), grid, block, 0, stream, w, out, groups);
            break;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_dequantize(int ggml_type, const void* W, void* out, int out_dtype, int64_t num_elements,
                             hipStream_t stream) {
    const int64_t groups = num_elements / 32;
    if (groups == 0) return hipSuccess;
    switch (ggml_type) {
        case QMM_TYPE_Q4_0: return launch_t<QMM_TYPE_Q4_0>(W, out, out_dtype, groups, stream);
        case QMM_TYPE_Q8_0: return launch_t<QMM_TYPE_Q8_0>(W, out, out_dtype, groups, stream);
        case QMM_TYPE_Q4_K: return launch_t<QMM_TYPE_Q4_K>(W, out, out_dtype, groups, stream);
        case QMM_TYPE_Q6_K: return launch_t<QMM_TYPE_Q6_K>(W, out, out_dtype, groups, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qmm
