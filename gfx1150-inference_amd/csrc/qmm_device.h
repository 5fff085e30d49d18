// Device-side helpers shared by the GEMV, dequantize and prefill kernels (gfx950, wave64).
#pragma once

#include "qmm_internal.h"

namespace qmm {

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(bits16 & 0xFFFFu)));
}

// Hides the known-zero bits of a packed code dword from the optimiser, so that byte
// extraction below lowers to a single v_cvt_f32_ubyte{0..3} per weight instead of a
// bit-field extract followed by a conversion.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    __asm__("" : "+v"(v));
    return v;
}

// fp32 -> fp16 bits, round to nearest even, signed zeros and subnormals kept.  The value is
// hidden from the optimiser first: otherwise fp16(a * b) is folded into
// v_fma_mixlo_f16(a, b, +0), which turns a -0 product into +0.
__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
    __asm__("" : "+v"(f));
    return __half_as_ushort(__float2half_rn(f));
}

// Byte `i` (0..3) of a dword as an exact float (v_cvt_f32_ubyte{0..3}).
__device__ __forceinline__ float ubyte_to_float(uint32_t v, int i) {
    return static_cast<float>((v >> (8 * i)) & 0xFFu);
}

__device__ __forceinline__ float dpp_quad(float v, int ctrl) {
    // ctrl is a quad_perm selector; every lane of the wave must be active.
    switch (ctrl) {
        case 0xA0: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xA0, 0xF, 0xF, false));
        case 0xF5: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xF5, 0xF, 0xF, false));
        case 0xB1: return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
        default:   return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
    }
}

// Sum over the 64 lanes of a wave, fixed order, result valid in lane 63.
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror,
// row_bcast:15 (rows 1,3), row_bcast:31 (rows 2,3).  All lanes must be active.
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));
    return v;
}

// Orders LDS traffic between the lanes of one wave (LDS ops of a wave execute in order;
// this only stops the compiler from moving them across the point).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// fp32 -> bf16 bits, round to nearest even, quiet NaN preserved.
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// Q4_K packed 6-bit (scale, min) of sub-block j from the 12 scale bytes
// (reference src/kernels/dequantize.hip:52-65), bytes given as three dwords.
__device__ __forceinline__ void q4k_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                              uint32_t& sc, uint32_t& m) {
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63u;
        m = (s1 >> (8 * j)) & 63u;
    } else {
        const int jj = 8 * (j - 4);
        sc = ((s2 >> jj) & 15u) | (((s0 >> (jj + 6)) & 3u) << 4);
        m = ((s2 >> (jj + 4)) & 15u) | (((s1 >> (jj + 6)) & 3u) << 4);
    }
}

// Weight i (0..31) of 32-weight group g of a packed row/stream, as fp32 computed the way the
// reference CPU dequantizer does (a*code exact, one rounding at "- b").  Byte loads only:
// used by the alignment-agnostic fallback kernels.
template <int T>
__device__ __forceinline__ void group_weights_bytewise(const uint8_t* __restrict__ base, int64_t g,
                                                       float w[32]) {
    if constexpr (T == QMM_TYPE_Q4_0) {
        const uint8_t* blk = base + g * kBytesQ4_0;
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t q = blk[2 + i];
            w[i] = static_cast<float>(static_cast<int>(q & 15u) - 8) * d;
            w[i + 16] = static_cast<float>(static_cast<int>(q >> 4) - 8) * d;
        }
    } else if constexpr (T == QMM_TYPE_Q8_0) {
        const uint8_t* blk = base + g * kBytesQ8_0;
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
#pragma unroll
        for (int i = 0; i < 32; ++i) w[i] = static_cast<float>(static_cast<int8_t>(blk[2 + i])) * d;
    } else if constexpr (T == QMM_TYPE_Q4_K) {
        const uint8_t* blk = base + (g >> 3) * kBytesQ4_K;
        const int s = static_cast<int>(g & 7);
        const float d = half_bits_to_float(blk[0] | (blk[1] << 8));
        const float dmin = half_bits_to_float(blk[2] | (blk[3] << 8));
        const uint32_t s0 = blk[4] | (blk[5] << 8) | (blk[6] << 16) | (static_cast<uint32_t>(blk[7]) << 24);
        const uint32_t s1 = blk[8] | (blk[9] << 8) | (blk[10] << 16) | (static_cast<uint32_t>(blk[11]) << 24);
        const uint32_t s2 = blk[12] | (blk[13] << 8) | (blk[14] << 16) | (static_cast<uint32_t>(blk[15]) << 24);
        uint32_t sc, m;
        q4k_scale_min(s, s0, s1, s2, sc, m);
        const float a = d * static_cast<float>(sc);
        const float b = dmin * static_cast<float>(m);
        const uint8_t* qs = blk + 16 + 32 * (s >> 1);
        const int sh = 4 * (s & 1);
#pragma unroll
        for (int i = 0; i < 32; ++i) w[i] = __fmaf_rn(a, static_cast<float>((qs[i] >> sh) & 15), -b);
    } else {  // Q6_K
        const uint8_t* blk = base + (g >> 3) * kBytesQ6_K;
        const int s = static_cast<int>(g & 7);  // weights 32s..32s+31
        const int n = s >> 2, t = s & 3;
        const float d = half_bits_to_float(blk[208] | (blk[209] << 8));
        const int8_t* sc = reinterpret_cast<const int8_t*>(blk + 192);
        const uint8_t* ql = blk + 64 * n + 32 * (t & 1);
        const uint8_t* qh = blk + 128 + 32 * n;
#pragma unroll
        for (int l = 0; l < 32; ++l) {
            const int q = static_cast<int>(((ql[l] >> (4 * (t >> 1))) & 15) | (((qh[l] >> (2 * t)) & 3) << 4)) - 32;
            const float a = d * static_cast<float>(sc[8 * n + l / 16 + 2 * t]);
            w[l] = a * static_cast<float>(q);
        }
    }
}

}  // namespace qmm
