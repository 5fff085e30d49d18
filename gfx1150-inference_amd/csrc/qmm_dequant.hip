// Dequantize packed GGUF blocks to fp16 / bf16 / fp32, bit-exact with the reference's CPU
// dequantizers (src/gguf_parser.py:374-589): every weight is a*code (exact in fp32) minus b,
// rounded once to fp32, then once (round-to-nearest-even) to the output type.
//
// Replaces dequantize_{q4_0,q8_0,q4_k,q6_k}_kernel (reference src/kernels/dequantize.hip:68-88,
// 213-229, 335-371, 508-544), which run one thread per block with byte loads and strided stores.
// Here 16 lanes share a unit of 256 weights (a Q4_K super-block, eight Q4_0 / Q8_0 blocks): lane j
// produces weights 16j..16j+15 of the unit, read with at most two 16-byte loads (its half of a
// Q4_K qs chunk and the super-block header; its Q8_0 / Q4_0 block's codes), and writes them as
// contiguous 16-byte stores, so a wave reads four units' packed bytes and writes 2 KiB (fp16) of
// contiguous output.  K-quant weights that are 16-byte aligned take the staged kernels below
// instead: whole batches of super-blocks copied into LDS with direct global -> LDS loads (every load
// instruction reads 1 KiB of contiguous memory), and lanes mapped so that every store instruction
// writes whole 128-byte lines.  HBM-bound: packed bytes in, output out.
#include <type_traits>

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

// Q6_K straight from memory, eight lanes per super-block: lane (hf, h) of super-block u produces
// weights 128 hf + 32 t + 8 h + (0..7) for the four groups t, so that one 8-byte slice of ql at
// 64 hf + 8 h (groups 0 and 2), one at 64 hf + 32 + 8 h (groups 1 and 3) and one of qh at
// 128 + 32 hf + 8 h (all four) serve 32 weights, with the half's eight sub-scales and d: five
// reads per 32 weights, four 16-byte stores of 8 consecutive outputs.  A super-block whose byte
// offset is 2 mod 4 has its slices read as 12 bytes from the 4-byte boundary below (f = 2) and
// shifted back (v_alignbyte); 12-byte reads stay inside the block for either f.
template <int OUT>
__device__ __forceinline__ void q6k_lane_out(uint2 qa, uint2 qb, uint2 qh, uint32_t s0, uint32_t s1, float d, int hf, int h,
                                             int64_t u, void* __restrict__ out) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        // sc[8 hf + 2t + l/16], l/16 = h/2
        const int si = 2 * t + (h >> 1);
        const uint32_t sw = si < 4 ? s0 : s1;
        const float a = d * static_cast<float>(static_cast<int8_t>(sw >> (8 * (si & 3))));
        const uint2 ql = (t & 1) ? qb : qa;
        float w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lb = ((i < 4 ? ql.x : ql.y) >> (8 * (i & 3))) & 0xFFu;
            const uint32_t hb = ((i < 4 ? qh.x : qh.y) >> (8 * (i & 3))) & 0xFFu;
            const int q = static_cast<int>(((lb >> (4 * (t >> 1))) & 15u) | (((hb >> (2 * t)) & 3u) << 4)) - 32;
            w[i] = a * static_cast<float>(q);
        }
        const int64_t first = 256 * u + 128 * hf + 32 * t + 8 * h;
        if constexpr (OUT == QMM_DTYPE_F32) {
            float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + first);
            o[0] = make_float4(w[0], w[1], w[2], w[3]);
            o[1] = make_float4(w[4], w[5], w[6], w[7]);
        } else {
            uint32_t pk[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo = OUT == QMM_DTYPE_F16 ? float_to_half_bits(w[2 * i]) : float_to_bf16_bits(w[2 * i]);
                const uint32_t hi = OUT == QMM_DTYPE_F16 ? float_to_half_bits(w[2 * i + 1]) : float_to_bf16_bits(w[2 * i + 1]);
                pk[i] = lo | (hi << 16);
            }
            *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + first) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        }
    }
}

// The slices straight from memory (any alignment of W; n a multiple of 256 weights).
template <int OUT>
__global__ __launch_bounds__(256) void dequant_q6k_kernel(const uint8_t* __restrict__ W, void* __restrict__ out,
                                                          int64_t n) {
    const int64_t lid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t u = lid >> 3;
    if (256 * u >= n) return;  // n % 256 == 0
    const int hf = static_cast<int>(lid >> 2) & 1, h = static_cast<int>(lid) & 3;
    const uint8_t* blk = W + u * kBytesQ6_K;
    // never below W: the first block keeps its loads as they lie
    const int f = u > 0 && (reinterpret_cast<uintptr_t>(blk) & 3) == 2 ? 2 : 0;
    auto ld8 = [&](const uint8_t* p) {  // 8 bytes at p
        uint32_t v[3];
        __builtin_memcpy(v, p - f, 12);
        return make_uint2(__builtin_amdgcn_alignbyte(v[1], v[0], f), __builtin_amdgcn_alignbyte(v[2], v[1], f));
    };
    const uint2 qa = ld8(blk + 64 * hf + 8 * h);       // ql[l], l = 8h..8h+7: groups 0 (low), 2 (high)
    const uint2 qb = ld8(blk + 64 * hf + 32 + 8 * h);  // ql[l + 32]: groups 1, 3
    const uint2 qh = ld8(blk + 128 + 32 * hf + 8 * h);
    uint32_t sv[3];  // sub-scales 8 hf .. 8 hf + 7 at bytes 4 - f ..
    __builtin_memcpy(sv, blk + 188 + 8 * hf + f, 12);
    const uint32_t s0 = f ? __builtin_amdgcn_alignbyte(sv[1], sv[0], 2) : sv[1];
    const uint32_t s1 = f ? __builtin_amdgcn_alignbyte(sv[2], sv[1], 2) : sv[2];
    uint16_t dv;
    __builtin_memcpy(&dv, blk + 208, 2);
    q6k_lane_out<OUT>(qa, qb, qh, s0, s1, half_bits_to_float(dv), hf, h, u, out);
}

// Q6_K through LDS (16-byte aligned W): a workgroup takes kQ6Batch consecutive super-blocks (3360
// bytes, 210 16-byte pieces) with direct global -> LDS loads, then sixteen lanes per super-block
// read their slices from LDS: lane (t, h) produces weights 128 hf + 32 t + 8 h + (0..7) of half hf
// = 0, then 1 (per half: one ql slice, the qh slice, one sub-scale; the arithmetic of
// q6k_lane_out, identical outputs), so that at each of its two 16-byte stores the super-block's
// sixteen lanes write 256 contiguous bytes (fp16).
constexpr int kQ6Batch = 16;

template <int OUT>
__global__ __launch_bounds__(256) void dequant_q6k_lds_kernel(const uint8_t* __restrict__ W, void* __restrict__ out) {
    __shared__ __align__(16) uint8_t sb[kQ6Batch * kBytesQ6_K];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint8_t* src = W + static_cast<size_t>(blockIdx.x) * (kQ6Batch * kBytesQ6_K);
    constexpr int kPieces = kQ6Batch * kBytesQ6_K / 16;
    static_assert(kQ6Batch * kBytesQ6_K % 16 == 0 && kPieces <= 256, "one piece per lane");
    {
        // piece q = 64 wv + lane lands at byte 16 q: the wave's m0 is 1 KiB per instruction
        const int q = 64 * wv + lane;
        const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sb + 1024 * wv));
        if (q < kPieces) __asm__ volatile("global_load_lds_dwordx4 %0, off" ::"v"(src + 16 * q), "{m0}"(m0) : "memory");
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's pieces have landed
    __syncthreads();
    const int ub = tid >> 4, t = (tid >> 2) & 3, h = tid & 3;
    const uint8_t* blk = sb + ub * kBytesQ6_K;
    const int f = (ub & 1) ? 2 : 0;  // odd blocks start 2 bytes past a 4-byte boundary
    auto ld8 = [&](const uint8_t* ptr) {  // 8 bytes at ptr, from three aligned words
        const uint32_t* a = reinterpret_cast<const uint32_t*>(ptr - f);
        const uint32_t v0 = a[0], v1 = a[1], v2 = a[2];
        return make_uint2(__builtin_amdgcn_alignbyte(v1, v0, f), __builtin_amdgcn_alignbyte(v2, v1, f));
    };
    const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(blk + 208));
    const int64_t u = static_cast<int64_t>(blockIdx.x) * kQ6Batch + ub;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        const uint2 ql = ld8(blk + 64 * hf + 32 * (t & 1) + 8 * h);
        const uint2 qh = ld8(blk + 128 + 32 * hf + 8 * h);
        const float a = d * static_cast<float>(*reinterpret_cast<const int8_t*>(blk + 192 + 8 * hf + 2 * t + (h >> 1)));
        float w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t lb = ((i < 4 ? ql.x : ql.y) >> (8 * (i & 3))) & 0xFFu;
            const uint32_t hb = ((i < 4 ? qh.x : qh.y) >> (8 * (i & 3))) & 0xFFu;
            const int q = static_cast<int>(((lb >> (4 * (t >> 1))) & 15u) | (((hb >> (2 * t)) & 3u) << 4)) - 32;
            w[i] = a * static_cast<float>(q);
        }
        const int64_t first = 256 * u + 128 * hf + 32 * t + 8 * h;
        if constexpr (OUT == QMM_DTYPE_F32) {
            float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + first);
            o[0] = make_float4(w[0], w[1], w[2], w[3]);
            o[1] = make_float4(w[4], w[5], w[6], w[7]);
        } else {
            uint32_t pk[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo = OUT == QMM_DTYPE_F16 ? float_to_half_bits(w[2 * i]) : float_to_bf16_bits(w[2 * i]);
                const uint32_t hi = OUT == QMM_DTYPE_F16 ? float_to_half_bits(w[2 * i + 1]) : float_to_bf16_bits(w[2 * i + 1]);
                pk[i] = lo | (hi << 16);
            }
            *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + first) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        }
    }
}


// Q4_K through LDS (16-byte aligned W): a workgroup takes kQ4Batch consecutive super-blocks (2304
// bytes, 144 16-byte pieces) with direct global -> LDS loads; lane j (of 16 per super-block)
// produces weights 8j + 128k + (0..7), k = 0, 1 (sub-blocks j/4 and 4 + j/4), so that at each of
// its two 16-byte stores the super-block's 16 lanes write 256 contiguous bytes (fp16), where the
// unit map of dequant_kernel writes every other 16 bytes.  Same arithmetic as unit_weights
// (identical outputs).
constexpr int kQ4Batch = 16;

template <int OUT>
__global__ __launch_bounds__(256) void dequant_q4k_lds_kernel(const uint8_t* __restrict__ W, void* __restrict__ out) {
    __shared__ __align__(16) uint8_t sb[kQ4Batch * kBytesQ4_K];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint8_t* src = W + static_cast<size_t>(blockIdx.x) * (kQ4Batch * kBytesQ4_K);
    constexpr int kPieces = kQ4Batch * kBytesQ4_K / 16;
    static_assert(kQ4Batch * kBytesQ4_K % 16 == 0 && kPieces <= 256, "one piece per lane");
    {
        const int q = 64 * wv + lane;
        const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sb + 1024 * wv));
        if (q < kPieces) __asm__ volatile("global_load_lds_dwordx4 %0, off" ::"v"(src + 16 * q), "{m0}"(m0) : "memory");
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const int ub = tid >> 4, j = tid & 15;
    const uint8_t* blk = sb + ub * kBytesQ4_K;
    const u32x4d hd = *reinterpret_cast<const u32x4d*>(blk);
    const float d = half_bits_to_float(hd[0]), dmin = half_bits_to_float(hd[0] >> 16);
    const int64_t u = static_cast<int64_t>(blockIdx.x) * kQ4Batch + ub;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int s = (j >> 2) + 4 * k;
        uint32_t sc, m;
        q4k_scale_min(s, hd[1], hd[2], hd[3], sc, m);
        const float a = d * static_cast<float>(sc);
        const float b = dmin * static_cast<float>(m);
        const uint2 q = *reinterpret_cast<const uint2*>(blk + 16 + 32 * (s >> 1) + 8 * (j & 3));
        const int sh = 4 * (s & 1);
        float w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            w[i] = __fmaf_rn(a, static_cast<float>((((i < 4 ? q.x : q.y) >> (8 * (i & 3))) >> sh) & 15u), -b);
        const int64_t first = 256 * u + 8 * j + 128 * k;
        if constexpr (OUT == QMM_DTYPE_F32) {
            float4* o = reinterpret_cast<float4*>(static_cast<float*>(out) + first);
            o[0] = make_float4(w[0], w[1], w[2], w[3]);
            o[1] = make_float4(w[4], w[5], w[6], w[7]);
        } else {
            uint32_t pk[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo = OUT == QMM_DTYPE_F16 ? float_to_half_bits(w[2 * i]) : float_to_bf16_bits(w[2 * i]);
                const uint32_t hi = OUT == QMM_DTYPE_F16 ? float_to_half_bits(w[2 * i + 1]) : float_to_bf16_bits(w[2 * i + 1]);
                pk[i] = lo | (hi << 16);
            }
            *reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + first) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        }
    }
}

template <int T>
hipError_t launch_t(const void* W, void* out, int out_dtype, int64_t n, hipStream_t stream) {
    // Q6_K: one lane per 32 outputs; the other formats: one lane per 16
    const dim3 grid(static_cast<unsigned>((n / (T == QMM_TYPE_Q6_K ? 32 : 16) + 255) / 256));
    const uint8_t* w = static_cast<const uint8_t*>(W);
    auto go = [&](auto oc) {
        constexpr int OUT = decltype(oc)::value;
        if constexpr (T == QMM_TYPE_Q6_K) {
            // whole batches of kQ6Batch super-blocks through LDS when W is 16-byte aligned, the rest
            // (or everything) straight from memory
            const int64_t blocks = n / 256;
            const int64_t batches = (reinterpret_cast<uintptr_t>(w) & 15u) == 0 ? blocks / kQ6Batch : 0;
            if (batches > 0)
                hipLaunchKernelGGL((dequant_q6k_lds_kernel<OUT>), dim3(static_cast<unsigned>(batches)), dim3(256), 0, stream,
                                   w, out);
            const int64_t done = batches * kQ6Batch;
            if (done < blocks) {
                const size_t esz = OUT == QMM_DTYPE_F32 ? 4 : 2;
                const int64_t rest = 256 * (blocks - done);
                hipLaunchKernelGGL((dequant_q6k_kernel<OUT>), dim3(static_cast<unsigned>((rest / 32 + 255) / 256)), dim3(256),
                                   0, stream, w + done * kBytesQ6_K, static_cast<char*>(out) + 256 * done * esz, rest);
            }
        } else if constexpr (T == QMM_TYPE_Q4_K) {
            // whole batches of kQ4Batch super-blocks through LDS when W is 16-byte aligned, the rest
            // (or everything) straight from memory
            const int64_t blocks = n / 256;
            const int64_t batches = (reinterpret_cast<uintptr_t>(w) & 15u) == 0 ? blocks / kQ4Batch : 0;
            if (batches > 0)
                hipLaunchKernelGGL((dequant_q4k_lds_kernel<OUT>), dim3(static_cast<unsigned>(batches)), dim3(256), 0, stream,
                                   w, out);
            const int64_t done = batches * kQ4Batch;
            if (done < blocks) {
                const size_t esz = OUT == QMM_DTYPE_F32 ? 4 : 2;
                const int64_t rest = 256 * (blocks - done);
                hipLaunchKernelGGL((dequant_kernel<T, OUT>), dim3(static_cast<unsigned>((rest / 16 + 255) / 256)), dim3(256), 0,
                                   stream, w + done * kBytesQ4_K, static_cast<char*>(out) + 256 * done * esz, rest);
            }
        } else {
            hipLaunchKernelGGL((dequant_kernel<T, OUT>), grid, dim3(256), 0, stream, w, out, n);
        }
    };
    switch (out_dtype) {
        case QMM_DTYPE_F32: go(std::integral_constant<int, QMM_DTYPE_F32>{}); break;
        case QMM_DTYPE_F16: go(std::integral_constant<int, QMM_DTYPE_F16>{}); break;
        default: go(std::integral_constant<int, QMM_DTYPE_BF16>{}); break;
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
