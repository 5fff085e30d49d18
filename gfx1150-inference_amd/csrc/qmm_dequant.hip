// Dequantize packed GGUF blocks to fp16 / bf16 / fp32, bit-exact with the reference's CPU
// dequantizers (src/gguf_parser.py:374-589): every weight is a*code (exact in fp32) minus b,
// rounded once to fp32, then once (round-to-nearest-even) to the output type.
//
// Replaces dequantize_{q4_0,q8_0,q4_k,q6_k}_kernel (reference src/kernels/dequantize.hip:68-88,
// 213-229, 335-371, 508-544), which run one thread per block with byte loads and strided stores.
// Here 16 lanes share a unit of 256 weights (a Q4_K / Q6_K super-block, eight Q4_0 / Q8_0
// blocks): lane j produces weights 16j..16j+15 of the unit, read with at most two 16-byte loads
// (its half of a Q4_K qs chunk and the super-block header; its Q6_K ql and qh slices; its Q8_0 /
// Q4_0 block's codes), and writes them as contiguous 16-byte stores, so a wave reads four units'
// packed bytes and writes 2 KiB (fp16) of contiguous output.  HBM-bound: packed bytes in, output out.
#include "qmm_device.h"

namespace qmm {
namespace {

typedef uint32_t u32x4d __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4d ld16(const uint8_t* p) {
    u32x4d v;
    __builtin_memcpy(&v, p, 16);  // global_load_dwordx4, any alignment
    return v;
}
__device__ __forceinline__ uint32_t byte_of(const u32x4d& v, int i) { return (v[i >> 2] >> (8 * (i & 3))) & 0xFFu; }

// Weights 16j..16j+15 of unit u (as the reference computes them, fp32).
template <int T>
__device__ __forceinline__ void unit_weights(const uint8_t* __restrict__ W, int64_t u, int j, float w[16]) {
    if constexpr (T == QMM_TYPE_Q4_K) {
        // sub-block s = j/2, half h = j%2: qs bytes 32(s/2) + 16h .. +15, nibble s%2
        const uint8_t* blk = W + u * kBytesQ4_K;
        const int s = j >> 1;
        const u32x4d hd = ld16(blk);
        const u32x4d q = ld16(blk + 16 + 32 * (s >> 1) + 16 * (j & 1));
        uint32_t sc, m;
        q4k_scale_min(s, hd[1], hd[2], hd[3], sc, m);
        const float a = half_bits_to_float(hd[0]) * static_cast<float>(sc);
        const float b = half_bits_to_float(hd[0] >> 16) * static_cast<float>(m);
        const int sh = 4 * (s & 1);
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = __fmaf_rn(a, static_cast<float>((byte_of(q, i) >> sh) & 15u), -b);
    } else if constexpr (T == QMM_TYPE_Q6_K) {
        // half n = j/8, quarter t = (j/2)%4, column half h = j%2: weights 128n + 32t + 16h + i
        const uint8_t* blk = W + u * kBytesQ6_K;
        const int n = j >> 3, t = (j >> 1) & 3, h = j & 1;
        // A block 2 bytes past a 4-byte boundary (every other one) is read with 4-aligned loads
        // from 2 bytes lower, plus the dword after each slice, and shifted back (v_alignbyte):
        // 16-byte loads at such addresses made this kernel 10 % slower.  Never below W: the
        // first unit keeps its loads as they are.
        const int f = u > 0 && (reinterpret_cast<uintptr_t>(blk) & 3) == 2 ? 2 : 0;
        const uint8_t* pl = blk + 64 * n + 32 * (t & 1) + 16 * h;
        const uint8_t* ph = blk + 128 + 32 * n + 16 * h;
        u32x4d ql = ld16(pl - f), qh = ld16(ph - f);
        uint32_t tl, th;
        __builtin_memcpy(&tl, pl + 12 + f, 4);  // f = 2: the dword after the slice; f = 0: unused
        __builtin_memcpy(&th, ph + 12 + f, 4);
        {
            const u32x4d a = ql, b = qh;
            ql[0] = __builtin_amdgcn_alignbyte(a[1], a[0], f);
            ql[1] = __builtin_amdgcn_alignbyte(a[2], a[1], f);
            ql[2] = __builtin_amdgcn_alignbyte(a[3], a[2], f);
            ql[3] = __builtin_amdgcn_alignbyte(tl, a[3], f);
            qh[0] = __builtin_amdgcn_alignbyte(b[1], b[0], f);
            qh[1] = __builtin_amdgcn_alignbyte(b[2], b[1], f);
            qh[2] = __builtin_amdgcn_alignbyte(b[3], b[2], f);
            qh[3] = __builtin_amdgcn_alignbyte(th, b[3], f);
        }
        const float d = half_bits_to_float(blk[208] | (static_cast<uint32_t>(blk[209]) << 8));
        const float a = d * static_cast<float>(static_cast<int8_t>(blk[192 + 8 * n + h + 2 * t]));
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int q = static_cast<int>(((byte_of(ql, i) >> (4 * (t >> 1))) & 15u) | (((byte_of(qh, i) >> (2 * t)) & 3u) << 4)) - 32;
            w[i] = a * static_cast<float>(q);
        }
    } else if constexpr (T == QMM_TYPE_Q8_0) {
        const uint8_t* blk = W + (8 * u + (j >> 1)) * kBytesQ8_0;
        const u32x4d q = ld16(blk + 2 + 16 * (j & 1));
        const float d = half_bits_to_float(blk[0] | (static_cast<uint32_t>(blk[1]) << 8));
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = static_cast<float>(static_cast<int8_t>(byte_of(q, i))) * d;
    } else {  // Q4_0: half j%2 of block j/2 (low nibbles = weights 0..15, high = 16..31)
        const uint8_t* blk = W + (8 * u + (j >> 1)) * kBytesQ4_0;
        const u32x4d q = ld16(blk + 2);
        const float d = half_bits_to_float(blk[0] | (static_cast<uint32_t>(blk[1]) << 8));
        const int sh = 4 * (j & 1);
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = static_cast<float>(static_cast<int>((byte_of(q, i) >> sh) & 15u) - 8) * d;
    }
}

// One lane per 16 outputs; n (a multiple of 32) weights in all.
template <int T, int OUT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ W, void* __restrict__ out, int64_t n) {
    const int64_t piece = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t first = 16 * piece;  // = 256 * unit + 16 * j
    if (first >= n) return;            // n % 32 == 0: a started Q4_0 / Q8_0 block is whole
    float w[16];
    unit_weights<T>(W, piece >> 4, static_cast<int>(piece & 15), w);
    if constexpr (OUT == QMM_DTYPE_F32) {
        float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + first);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = make_float4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
    } else {
        uint32_t p[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
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
        uint4* o = reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + first);
        o[0] = make_uint4(p[0], p[1], p[2], p[3]);
        o[1] = make_uint4(p[4], p[5], p[6], p[7]);
    }
}

template <int T>
hipError_t launch_t(const void* W, void* out, int out_dtype, int64_t n, hipStream_t stream) {
    const dim3 block(256);
    const dim3 grid(static_cast<unsigned>((n / 16 + 255) / 256));
    const uint8_t* w = static_cast<const uint8_t*>(W);
    switch (out_dtype) {
        case QMM_DTYPE_F32:
            hipLaunchKernelGGL((dequant_kernel<T, QMM_DTYPE_F32>), grid, block, 0, stream, w, out, n);
            break;
        case QMM_DTYPE_F16:
            hipLaunchKernelGGL((dequant_kernel<T, QMM_DTYPE_F16>), grid, block, 0, stream, w, out, n);
            break;
        default:
            hipLaunchKernelGGL((dequant_kernel<T, QMM_DTYPE_BF16>), grid, block, 0, stream, w, out, n);
            break;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_dequantize(int ggml_type, const void* W, void* out, int out_dtype, int64_t num_elements,
                             hipStream_t stream) {
    const int64_t n = num_elements / 32 * 32;
    if (n == 0) return hipSuccess;
    switch (ggml_type) {
        case QMM_TYPE_Q4_0: return launch_t<QMM_TYPE_Q4_0>(W, out, out_dtype, n, stream);
        case QMM_TYPE_Q8_0: return launch_t<QMM_TYPE_Q8_0>(W, out, out_dtype, n, stream);
        case QMM_TYPE_Q4_K: return launch_t<QMM_TYPE_Q4_K>(W, out, out_dtype, n, stream);
        case QMM_TYPE_Q6_K: return launch_t<QMM_TYPE_Q6_K>(W, out, out_dtype, n, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace qmm
