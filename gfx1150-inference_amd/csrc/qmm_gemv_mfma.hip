// Small-M GEMV on the matrix cores: C[m, n] = sum_k A[m, k] * dequant(W)[n, k] for the GEMV family's M
// (16 activation rows per pass), Q4_K and Q6_K weights.
//
// MI355X design (replaces the reference's wave32 GEMV kernels and their TILE_M = 4 "prefill" variants,
// src/kernels/dequantize.hip:377-505, 549-685, whose per-row vector work grows with M):
//   * A row group is 16 weight rows: the n dimension of v_mfma_f32_16x16x32_f16.  Lane l of a wave
//     decodes weight row l % 16 into the B operand and reads activation row l % 16 into the A operand;
//     it receives the outputs of weight row l % 16 for activation rows 4 (l / 16) + r, r < 4.
//   * Lane quarter c = l / 16 owns a fixed quarter of every super-block, streamed with 16-byte loads:
//     Q4_K the 16-byte header and the 32-byte qs chunk c (sub-blocks 2c, 2c + 1); Q6_K the
//     (half c / 2, 16-column half c % 2) slice: 16 + 16 bytes of ql, 16 of qh, the 8 sub-scale bytes
//     of that half and d.
//   * Codes become exact f16 integers s * q: one v_and_or_b32 turns two codes into (1024 + q) or
//     (1024 + 16q) (0x6400 | bits), one v_pk_fma_f16 with (s, -1024 s) or (s / 16, -64 s) leaves
//     s * q exactly (|s * q| <= 2048, so no rounding).  Q4_K: s = the 6-bit sub-scale.  Q6_K: the
//     6-bit code u = ul + 16 uh is split into its nibble ul and its 2-bit top uh, s = the int8
//     sub-scale, and two MFMA chains add s * ul and s * uh (combined as T1 + 16 T2).  All products
//     of the MFMA are exact; its fp32 sums round.
//   * Per super-block and row: y += d * T - c2 * U, where U is a second MFMA over the per-group sums
//     of the staged activations (held as f16 hi + lo pairs of sum / 32) against the group minima
//     (Q4_K: the 6-bit mins, c2 = 32 dmin) or the sub-scales (Q6_K's code offset 32: c2 = 1024 d).
//   * The K range of a row group is cut into 8 fixed slots (super-blocks sb with sb % 8 = slot), one
//     per wave of the 8-wave workgroup; a wave adds its slot's super-blocks in order and the 8 slot
//     sums are added in slot order through LDS.  Every row's arithmetic is therefore the same
//     instruction sequence whatever M, the row group's place and the grid; MFMA rows are
//     independent, so row m of any M is bit-identical to the M = 1 call (the reference's
//     prefill-vs-M=1 invariant, tests/test_phase5_scale.py:274-310).
//   * Activations (16 rows per pass) are staged once per workgroup into LDS in natural k order
//     (8-k pieces with the pair order of the decoded codes), fp32 rounded to f16 with a power-of-two
//     rescale of any (row, 4096-k window) outside f16's range.
//   * Weights stream through an LDS ring of NB (3 or 4) chunks of 16 rows x 8 super-blocks, copied
//     by the whole workgroup with direct global -> LDS 16-byte loads (each instruction reads whole
//     row segments); NB - 1 chunks are in flight while one is multiplied, across row groups.
#include <climits>
#include <mutex>
#include <string>
#include <type_traits>
#include <unordered_map>

#include "qmm_device.h"

namespace qmm {
namespace {

typedef uint32_t mu4 __attribute__((ext_vector_type(4)));
typedef _Float16 mh8 __attribute__((ext_vector_type(8)));
typedef _Float16 mh2 __attribute__((ext_vector_type(2)));
typedef float mf4 __attribute__((ext_vector_type(4)));

constexpr int kSlots = 8;       // waves per workgroup = K slots of a row group
constexpr int kRows = 16;       // weight rows per row group
constexpr int kMRows = 16;      // activation rows per pass
constexpr int kWinK = 4096;     // fp32 rescale window
constexpr int kMaxWin = 16;     // K <= 65536 for fp32 activations

constexpr size_t kStaticLds = 2 * kMRows * kMaxWin * 4;  // the kernels' static LDS at most (fp32 window maxima)

__device__ __forceinline__ uint32_t mkeep(uint32_t v) {
    __asm__("" : "+v"(v));
    return v;
}
__device__ __forceinline__ uint32_t hbits2(mh2 v) {
    uint32_t u;
    __builtin_memcpy(&u, &v, 4);
    return u;
}
__device__ __forceinline__ mh2 as_mh2(uint32_t u) {
    mh2 v;
    __builtin_memcpy(&v, &u, 4);
    return v;
}
// (a, a) as an f16 pair
__device__ __forceinline__ uint32_t pair_of(_Float16 a) { return hbits2(mh2{a, a}); }
// pk_fma(code pair, s pair, o pair): exact s * q when the true result is an f16 integer
__device__ __forceinline__ uint32_t pkfma(uint32_t code, uint32_t s, uint32_t o) {
    return hbits2(__builtin_elementwise_fma(as_mh2(code), as_mh2(s), as_mh2(o)));
}
__device__ __forceinline__ uint32_t andor(uint32_t v, uint32_t m, uint32_t o) { return (v & m) | o; }

__device__ __forceinline__ mf4 mfma16(mh8 a, mh8 b, mf4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
// pk_fma of four code pairs into one B operand (the pairs land in the operand's registers directly)
__device__ __forceinline__ mh8 bop(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t s, uint32_t o) {
    const mh2 sv = as_mh2(s), ov = as_mh2(o);
    const mh2 r0 = __builtin_elementwise_fma(as_mh2(c0), sv, ov), r1 = __builtin_elementwise_fma(as_mh2(c1), sv, ov);
    const mh2 r2 = __builtin_elementwise_fma(as_mh2(c2), sv, ov), r3 = __builtin_elementwise_fma(as_mh2(c3), sv, ov);
    const _Float16 __attribute__((ext_vector_type(4))) lo = __builtin_shufflevector(r0, r1, 0, 1, 2, 3);
    const _Float16 __attribute__((ext_vector_type(4))) hi = __builtin_shufflevector(r2, r3, 0, 1, 2, 3);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// ------------------------------------------------------------------------------------------------
// Formats.  Lane quarter c's A fragment of MFMA step t starts at super-block k = k0(c, t) and covers 8
// consecutive k in the pair order (0, 2), (1, 3), (4, 6), (5, 7).  Group sums: group j of kGroups
// per super-block covers kGroupK consecutive k from gk(j); it lands in half hpos(j) (hi) and
// hpos(j) + 4 (lo)... of the 8-half sum fragment of quarter gq(j).
// ------------------------------------------------------------------------------------------------

// Q4_K (reference block_q4_k, src/kernels/dequantize.hip:31-36; get_scale_min_k4 :52-65).
struct MQ4K {
    static constexpr int kType = QMM_TYPE_Q4_K;
    static constexpr int kBlockBytes = kBytesQ4_K;
    static constexpr int kChains = 1;
    static constexpr bool kSums = true;  // group minima: a second MFMA over the activations' group sums
    static constexpr int kGroupK = 32;
    struct Raw {
        mu4 h, q0, q1;
    };
    __device__ static int k0(int c, int t) { return 64 * c + 8 * t; }
    // group j = sub-block j: quarter j / 2, hi at half j % 2, lo at half 2 + j % 2
    __device__ static int gq(int j) { return j >> 1; }
    __device__ static int hpos(int j) { return j & 1; }
    __device__ static int lpos(int j) { return 2 + (j & 1); }
    __device__ static Raw load(const uint8_t* blk, int c) {
        Raw r;
        r.h = *reinterpret_cast<const mu4*>(blk);
        r.q0 = *reinterpret_cast<const mu4*>(blk + 16 + 32 * c);
        r.q1 = *reinterpret_cast<const mu4*>(blk + 32 + 32 * c);
        return r;
    }
    struct Pre {
        uint32_t s_lo, o_lo, s_hi, o_hi;  // (sc0, sc0), (-1024 sc0, ..), (sc1 / 16, ..), (-64 sc1, ..)
        mh8 bu;                            // (m0, m1, m0 / 2048, m1 / 2048, 0, 0, 0, 0)
        float d, c2;                       // d, 32 dmin
        uint32_t sh[8];                    // chunk dwords >> 8
    };
    __device__ static Pre prep(const Raw& r, int c) {
        Pre p;
        uint32_t sc[2], mn[2];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const int sh = 8 * ((2 * c + g) & 3);
            const uint32_t sc_lo = (r.h.y >> sh) & 63u;
            const uint32_t mn_lo = (r.h.z >> sh) & 63u;
            const uint32_t sc_hi = ((r.h.w >> sh) & 15u) | (((r.h.y >> (sh + 6)) & 3u) << 4);
            const uint32_t mn_hi = ((r.h.w >> (sh + 4)) & 15u) | (((r.h.z >> (sh + 6)) & 3u) << 4);
            sc[g] = c < 2 ? sc_lo : sc_hi;
            mn[g] = c < 2 ? mn_lo : mn_hi;
        }
        const _Float16 s0 = static_cast<_Float16>(static_cast<float>(sc[0]));
        const _Float16 s1 = static_cast<_Float16>(static_cast<float>(sc[1]));
        p.s_lo = pair_of(s0);
        p.o_lo = pair_of(s0 * static_cast<_Float16>(-1024.0f));
        p.s_hi = pair_of(s1 * static_cast<_Float16>(0.0625f));
        p.o_hi = pair_of(s1 * static_cast<_Float16>(-64.0f));
        const _Float16 f0 = static_cast<_Float16>(static_cast<float>(mn[0])), f1 = static_cast<_Float16>(static_cast<float>(mn[1]));
        const _Float16 r11 = static_cast<_Float16>(1.0f / 2048.0f), z = static_cast<_Float16>(0.0f);
        p.bu = mh8{f0, f1, f0 * r11, f1 * r11, z, z, z, z};
        p.d = half_bits_to_float(r.h.x);
        p.c2 = 32.0f * half_bits_to_float(r.h.x >> 16);
        p.sh[0] = r.q0.x >> 8; p.sh[1] = r.q0.y >> 8; p.sh[2] = r.q0.z >> 8; p.sh[3] = r.q0.w >> 8;
        p.sh[4] = r.q1.x >> 8; p.sh[5] = r.q1.y >> 8; p.sh[6] = r.q1.z >> 8; p.sh[7] = r.q1.w >> 8;
        return p;
    }
    // B operand of step t (chain 0): t < 4 low nibbles of dwords 2t, 2t + 1 of the chunk, t >= 4 the
    // high nibbles of dwords 2(t - 4), 2(t - 4) + 1.
    __device__ static void steps(const Raw& r, const Pre& p, int t, uint32_t mg, mh8 (&b)[kChains]) { b[0] = step(r, p, t, mg); }
    __device__ static mh8 step(const Raw& r, const Pre& p, int t, uint32_t mg) {
        const int j = t & 3;
        const mu4& q = j < 2 ? r.q0 : r.q1;
        const uint32_t v0 = (j & 1) ? q.z : q.x;
        const uint32_t v1 = (j & 1) ? q.w : q.y;
        const uint32_t w0 = p.sh[2 * j], w1 = p.sh[2 * j + 1];
        const uint32_t m = t < 4 ? 0x000F000Fu : 0x00F000F0u;
        const uint32_t s = t < 4 ? p.s_lo : p.s_hi;
        const uint32_t o = t < 4 ? p.o_lo : p.o_hi;
        return bop(andor(v0, m, mg), andor(w0, m, mg), andor(v1, m, mg), andor(w1, m, mg), s, o);
    }
};

// Q6_K (reference block_q6_k, src/kernels/dequantize.hip:39-44): quarter c = (half hf = c / 2, column
// half h = c % 2): weights 128 hf + 32 t + 16 h + j, t < 4, j < 16; sub-scale sc[8 hf + h + 2 t].
// Step st = 2 t + (j >= 8).  The 6-bit code u (w = d sc (u - 32)) is assembled bytewise and two
// v_perm make the f16 pairs (1024 + u); the int8 sub-scale is split as sc = 16 sh + sl (sl = sc & 15,
// sh = sc >> 4), so that sl (u - 32) and sh (u - 32) are exact f16 integers (|.| <= 480, 256): two
// chains, T = T1 + 16 T2, and the code offset needs no second sum.
struct MQ6K {
    static constexpr int kType = QMM_TYPE_Q6_K;
    static constexpr int kBlockBytes = kBytesQ6_K;
    static constexpr int kChains = 2;
    static constexpr bool kSums = false;
    static constexpr int kGroupK = 16;
    struct Raw {
        mu4 la, lb, qh;
        uint32_t s0, s1, d;
    };
    __device__ static int k0(int c, int st) { return 128 * (c >> 1) + 32 * (st >> 1) + 16 * (c & 1) + 8 * (st & 1); }
    __device__ static int gq(int) { return 0; }
    __device__ static int hpos(int) { return 0; }
    __device__ static int lpos(int) { return 0; }
    __device__ static Raw load(const uint8_t* blk, int c) {
        const int hf = c >> 1, h = c & 1;
        Raw r;
        __builtin_memcpy(&r.la, blk + 64 * hf + 16 * h, 16);
        __builtin_memcpy(&r.lb, blk + 64 * hf + 32 + 16 * h, 16);
        __builtin_memcpy(&r.qh, blk + 128 + 32 * hf + 16 * h, 16);
        uint32_t s[2];
        __builtin_memcpy(s, blk + 192 + 8 * hf, 8);
        r.s0 = s[0];
        r.s1 = s[1];
        uint16_t dv;
        __builtin_memcpy(&dv, blk + 208, 2);
        r.d = dv;
        return r;
    }
    struct Pre {
        uint32_t sl[4], ol[4];  // (sl, sl), (-1056 sl, ..) per t
        uint32_t sh[4], oh[4];  // (sh, sh), (-1056 sh, ..) per t
        mh8 bu;                 // unused (no group sums)
        float d, c2;            // d, 0
    };
    __device__ static Pre prep(const Raw& r, int c) {
        Pre p;
        const int h = c & 1;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t w = t < 2 ? r.s0 : r.s1;
            const int sc = static_cast<int8_t>(w >> (8 * (h + 2 * (t & 1))));
            const _Float16 lo = static_cast<_Float16>(static_cast<float>(sc & 15));
            const _Float16 hi = static_cast<_Float16>(static_cast<float>(sc >> 4));
            p.sl[t] = pair_of(lo);
            p.ol[t] = pair_of(lo * static_cast<_Float16>(-1056.0f));
            p.sh[t] = pair_of(hi);
            p.oh[t] = pair_of(hi * static_cast<_Float16>(-1056.0f));
        }
        p.d = half_bits_to_float(r.d);
        p.c2 = 0.0f;
        return p;
    }
    // B operands of step st: chain 0 sl (u - 32), chain 1 sh (u - 32); bytes 8 (st & 1) .. + 7 of the
    // lane's slices (weights j = 8 (st & 1) + 0..7 of group t = st / 2).
    __device__ static void steps(const Raw& r, const Pre& p, int st, uint32_t mg, mh8 (&b)[kChains]) {
        const int t = st >> 1, jh = st & 1;
        const mu4& q = (t & 1) ? r.lb : r.la;
        const uint32_t L[2] = {jh ? q.z : q.x, jh ? q.w : q.y};
        const uint32_t H[2] = {jh ? r.qh.z : r.qh.x, jh ? r.qh.w : r.qh.y};
        uint32_t cd[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t lo4 = (t < 2 ? L[i] : L[i] >> 4) & 0x0F0F0F0Fu;
            // bits 2t, 2t + 1 of each qh byte -> bits 4, 5
            const uint32_t hs = t == 0 ? H[i] << 4 : t == 1 ? H[i] << 2 : t == 2 ? H[i] : H[i] >> 2;
            const uint32_t u = andor(hs, 0x30303030u, lo4);
            cd[2 * i] = __builtin_amdgcn_perm(mg, u, 0x07020500u);      // (1024 + u0, 1024 + u2)
            cd[2 * i + 1] = __builtin_amdgcn_perm(mg, u, 0x07030501u);  // (1024 + u1, 1024 + u3)
        }
        b[0] = bop(cd[0], cd[1], cd[2], cd[3], p.sl[t], p.ol[t]);
        b[1] = bop(cd[0], cd[1], cd[2], cd[3], p.sh[t], p.oh[t]);
    }
};

// ------------------------------------------------------------------------------------------------
// LDS of a workgroup (dynamic), per staged activation row m (row stride rs bytes, rs % 128 = 16 or 80
// so that the rows' fragments spread over the banks):
//   [0, 2K)            activations, natural k order, each 8-k piece in pair order (0,2,1,3,4,6,5,7)
//   [2K, 2K + 64 nsb)  per (super-block, quarter) 8 halves: group sums / 32 as f16 hi and lo
// then the slot partials: 2 buffers x 8 waves x 64 lanes x 16 bytes.
// ------------------------------------------------------------------------------------------------
extern __shared__ __attribute__((aligned(16))) uint8_t mlds[];

template <class F>
__host__ __device__ constexpr int row_stride(int K) { return 2 * K + (F::kSums ? 64 * (K / 256) : 0) + 16; }
// slot partials of a pass of `lrows` activation rows: 2 buffers x 8 waves x 16 lanes per quarter
__host__ __device__ constexpr int red_bytes(int lrows) { return 2 * kSlots * 16 * ((lrows + 3) / 4) * 16; }

__device__ __forceinline__ int win_exp(uint32_t maxbits) {
    // (row, window) maximum at or above 65504, or in [2^-126, 2^-14): scale by 2^-e with
    // e = exponent(max) - 14 (brings the maximum into [2^14, 2^15))
    const bool big = maxbits >= 0x477FE000u && maxbits < 0x7F800000u;
    const bool tiny = maxbits >= 0x00800000u && maxbits < 0x38800000u;
    return big || tiny ? static_cast<int>(maxbits >> 23) - 127 - 14 : 0;
}

template <typename TA>
__device__ __forceinline__ void load_group(const TA* p, bool vec, float x[16]);
template <>
__device__ __forceinline__ void load_group<float>(const float* p, bool vec, float x[16]) {
    if (vec) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = reinterpret_cast<const float4*>(p)[i];
            x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = p[i];
    }
}
template <>
__device__ __forceinline__ void load_group<__half>(const __half* p, bool vec, float x[16]) {
    _Float16 h[16];
    if (vec) {
        __builtin_memcpy(h, p, 32);
    } else {
        const uint16_t* s = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint16_t b = s[i];
            __builtin_memcpy(&h[i], &b, 2);
        }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = static_cast<float>(h[i]);
}

// Stages activation rows m0 .. m0 + mr - 1 into LDS, 16 k per item (fp32: after the (row, window)
// maxima are known; `wexp` holds e per (row, window)).
// Writes staging item `it` (16 consecutive activations x of one row, rows staged as in stage_rows).
template <class F, typename TA>
__device__ __forceinline__ void stage_item(int it, int per_row, int K, int rs, bool ok, const float (&x)[16], const int* wexp) {
    {
        const int m = it / per_row, k = 16 * (it - m * per_row);
        const int e = std::is_same<TA, float>::value ? wexp[m * kMaxWin + k / kWinK] : 0;
        _Float16 h[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float v = ok ? x[i] : 0.0f;
            h[i] = static_cast<_Float16>(std::is_same<TA, float>::value ? __builtin_ldexpf(v, -e) : v);
        }
        uint8_t* row = mlds + m * rs;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const mh8 v{h[8 * q], h[8 * q + 2], h[8 * q + 1], h[8 * q + 3], h[8 * q + 4], h[8 * q + 6], h[8 * q + 5],
                        h[8 * q + 7]};
            *reinterpret_cast<mh8*>(row + 2 * (k + 8 * q)) = v;
        }
        if constexpr (!F::kSums) return;
        // group sums in a fixed order, stored as f16 hi + lo of sum / 32 (exact power-of-two scaling;
        // |sum / 32| stays inside f16's range)
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) s += static_cast<float>(h[i]);
        bool store = true;
        int j = (k & 255) >> 4;
        if constexpr (F::kGroupK == 32) {
            // a 32-k group is two items of adjacent lanes (items come in pairs: per_row and the
            // stride are even); the first half's lane adds the second's sum
            const float o = __shfl_xor(s, 1, 64);
            store = (it & 1) == 0;
            s = s + o;
            j >>= 1;
        }
        if (store) {
            const int sb = k >> 8;
            const float v = s * 0.03125f;
            const _Float16 hi = static_cast<_Float16>(v);
            // the remainder scaled by 2^11 stays a normal f16 (its B halves carry the 2^-11)
            const _Float16 lo = static_cast<_Float16>((v - static_cast<float>(hi)) * 2048.0f);
            _Float16* f = reinterpret_cast<_Float16*>(row + 2 * K + 64 * sb + 16 * F::gq(j));
            f[F::hpos(j)] = hi;
            f[F::lpos(j)] = lo;
            if constexpr (F::kGroupK == 32) {
                if ((j & 1) == 0) {  // halves 4..7 of the quarter's fragment are unused: zero
                    f[4] = static_cast<_Float16>(0.0f);
                    f[5] = static_cast<_Float16>(0.0f);
                    f[6] = static_cast<_Float16>(0.0f);
                    f[7] = static_cast<_Float16>(0.0f);
                }
            }
        }
    }
}

// Stages activation rows m0 .. m0 + mr - 1 into LDS, 16 k per item, items first, first + nthreads, ...
// (fp32: after the (row, window) maxima are known; `wexp` holds e per (row, window)).
template <class F, typename TA>
__device__ __forceinline__ void stage_rows(const TA* __restrict__ A, int M, int K, int m0, int mr, bool vec, const int* wexp,
                                           int first, int nthreads) {
    const int rs = row_stride<F>(K);
    const int per_row = K / 16;
    const int items = mr * per_row;
    for (int it = first; it < items; it += nthreads) {
        const int m = it / per_row, k = 16 * (it - m * per_row);
        const bool ok = m0 + m < M;
        float x[16];
        load_group<TA>(A + static_cast<size_t>(ok ? m0 + m : 0) * K + k, vec, x);
        stage_item<F, TA>(it, per_row, K, rs, ok, x, wexp);
    }
}

// The first kEarly staging items of each thread (fp16 activations) are loaded before the weight chunks
// are requested, by loads the compiler does not track, and waited for with an explicit count that
// leaves the chunk requests in flight.
constexpr int kEarly = 4;
__device__ __forceinline__ mu4 ldg_untracked(const void* p) {
    mu4 v;
    __asm__ volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
    return v;
}
template <int N>
__device__ __forceinline__ void vm_wait_for(mu4 (&v)[kEarly][2]) {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __asm__ volatile("s_waitcnt vmcnt(%8)"
                     : "+v"(v[0][0]), "+v"(v[0][1]), "+v"(v[1][0]), "+v"(v[1][1]), "+v"(v[2][0]), "+v"(v[2][1]),
                       "+v"(v[3][0]), "+v"(v[3][1])
                     : "n"(N)
                     : "memory");
}

template <typename TC>
struct MSegs {
    const uint8_t* W[4];
    TC* C[4];
    int N[4];
    int gend[4];  // row groups [gend[s-1], gend[s]) belong to segment s; unused entries INT_MAX
};

// Segment of row group g: its weights, output, rows and first row group (selects over the fixed entries,
// so the table stays in scalar registers).
template <typename TC>
__device__ __forceinline__ void seg_pick(const MSegs<TC>& sg, int g, const uint8_t*& W, TC*& C, int& N, int& g0) {
    W = sg.W[0];
    C = sg.C[0];
    N = sg.N[0];
    g0 = 0;
#pragma unroll
    for (int j = 1; j < 4; ++j) {
        const bool in = g >= sg.gend[j - 1];
        W = in ? sg.W[j] : W;
        C = in ? sg.C[j] : C;
        N = in ? sg.N[j] : N;
        g0 = in ? sg.gend[j - 1] : g0;
    }
}

template <typename TC>
__device__ __forceinline__ void mstore(TC* p, float v);
template <>
__device__ __forceinline__ void mstore<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void mstore<__half>(__half* p, float v) { *reinterpret_cast<uint16_t*>(p) = float_to_half_bits(v); }

// Direct global -> LDS load of 16 bytes per lane (global_load_lds_dwordx4): lane l's bytes land at
// LDS address m0 + 16 l.  The compiler does not track these loads; they are waited for with explicit
// vmcnt counts.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds_m0) {
    __asm__ volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_m0) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void lds_sync() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Weight chunk of a row group: 16 rows x 8 super-blocks (one per slot), copied row by row into an LDS
// ring slot of 16 x kRP 16-byte pieces (kRP = the chunk row's pieces, plus one unused piece where that
// count is a multiple of 8, so that consecutive rows start in different LDS banks).
template <class F>
struct Chunk {
    static constexpr int kP = kSlots * F::kBlockBytes / 16;            // pieces of one chunk row
    static constexpr int kRP = kP % 8 == 0 ? kP + 1 : kP;               // LDS row stride in pieces
    static constexpr int kBytes = kRows * kRP * 16;                     // one ring slot
    static constexpr int kInstr = (2 * kRP + 63) / 64;                  // DMA instructions per wave
};

// R: accumulated values per lane (min(rows of the pass, 4) for one lane quarter holding rows;
// 4 for passes of more than 4 rows, where quarter c holds rows 4c .. 4c + 3).  NB: ring slots.
// Per chunk step: wave w waits for its own copies of the chunk, one barrier (all copies landed; every
// wave is done with the slot refilled next), then it requests chunk i + NB - 1 into that slot and
// multiplies super-block w of chunk i for the 16 rows from LDS.
template <class F, int R, int NB, typename TA, typename TC>
__global__ __launch_bounds__(64 * kSlots) void gemv_mfma_kernel(const TA* __restrict__ A, MSegs<TC> sg, int M, int K,
                                                                 int nrg, int a_vec, int lrows) {
    using CK = Chunk<F>;
    constexpr bool kF32 = std::is_same<TA, float>::value;
    __shared__ int wexp[kF32 ? kMRows * kMaxWin : 1];
    __shared__ uint32_t wmax[kF32 ? kMRows * kMaxWin : 1];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, c = lane >> 4;
    const int m0 = blockIdx.y * lrows;
    const int mr = min(lrows, M - m0);
    const int nsb = K >> 8;
    const int cpr = (nsb + kSlots - 1) / kSlots;  // chunks per row group
    const int mine = (nrg - static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
    const int total = mine * cpr;
    const int row_bytes = nsb * F::kBlockBytes;
    const int rs = row_stride<F>(K);
    const bool vec = a_vec != 0;
    uint8_t* ring = mlds + lrows * rs;
    uint8_t* red = ring + NB * CK::kBytes;
    const uint32_t ring_m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ring));

    // Per-lane constants of the copies: instruction k moves this lane's piece q = 64 k + lane of the
    // wave's two rows (row r = q / kRP, piece pc of it; the row's padding piece repeats its last piece).
    int lane_off[CK::kInstr];
    bool lane_r1[CK::kInstr];
#pragma unroll
    for (int k = 0; k < CK::kInstr; ++k) {
        const int q = 64 * k + lane;
        lane_r1[k] = q >= CK::kRP;
        lane_off[k] = 16 * min(q - (lane_r1[k] ? CK::kRP : 0), CK::kP - 1);
    }
    // Issue cursor: row group ili (of this workgroup), chunk ich, ring slot islot; the wave's two
    // source rows (row 2w + 1 clamped to the segment's last row: then d1 = 0).
    int ili = 0, ich = 0, islot = 0;
    const uint8_t* src0 = nullptr;
    int d1 = 0;
    auto rg_rows = [&](int li) {
        const int g = static_cast<int>(blockIdx.x) + li * static_cast<int>(gridDim.x);
        const uint8_t* W;
        TC* Cs;
        int N, g0;
        seg_pick(sg, g, W, Cs, N, g0);
        const int r0 = min((g - g0) * kRows + 2 * w, N - 1);
        const int r1 = min(r0 + 1, N - 1);
        src0 = W + static_cast<size_t>(r0) * row_bytes;
        d1 = (r1 - r0) * row_bytes;
    };
    rg_rows(0);
    // Requests the cursor's chunk into its slot and advances the cursor (past the workgroup's last chunk
    // it stays there: the tail requests re-read valid bytes, so every wave issues the same loads).
    auto issue = [&]() {
        const int cb = ich * kSlots * F::kBlockBytes;
        const uint32_t dst = ring_m0 + static_cast<uint32_t>(islot * CK::kBytes + 2 * w * CK::kRP * 16);
#pragma unroll
        for (int k = 0; k < CK::kInstr; ++k) {
            const int off = min(cb + lane_off[k], row_bytes - 16) + (lane_r1[k] ? d1 : 0);
            if (64 * k + 64 <= 2 * CK::kRP || 64 * k + lane < 2 * CK::kRP) dma16(src0 + off, dst + 64 * 16 * k);
        }
        islot = islot + 1 == NB ? 0 : islot + 1;
        if (ich + 1 < cpr) {
            ++ich;
        } else if (ili + 1 < mine) {
            ich = 0;
            rg_rows(++ili);
        }
    };

    // fp16 activations: the first items' loads go out first, then the first NB - 1 chunk requests
    const int per_row = K / 16;
    const int items = mr * per_row;
    const bool early = !kF32 && vec;
    mu4 ev[kEarly][2];
    if (early) {
#pragma unroll
        for (int e = 0; e < kEarly; ++e) {
            const int it = min(tid + e * 64 * kSlots, items - 1);
            const int m = it / per_row, k = 16 * (it - m * per_row);
            const TA* p = A + static_cast<size_t>(m0 + m) * K + k;
            ev[e][0] = ldg_untracked(p);
            ev[e][1] = ldg_untracked(p + 8);
        }
    }
#pragma unroll
    for (int u = 0; u < NB - 1; ++u) issue();

    // staging (fp32: window maxima first)
    if constexpr (kF32) {
        const int nwin = (K + kWinK - 1) / kWinK;
        for (int i = tid; i < kMRows * kMaxWin; i += 64 * kSlots) wmax[i] = 0u;
        __syncthreads();
        const int per_row = K / 16;
        for (int it = tid; it < mr * per_row; it += 64 * kSlots) {
            const int m = it / per_row, k = 16 * (it - m * per_row);
            float x[16];
            load_group<float>(A + static_cast<size_t>(m0 + m) * K + k, vec, x);
            float mx = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(x[i]));
            atomicMax(&wmax[m * kMaxWin + k / kWinK], __float_as_uint(mx));
        }
        __syncthreads();
        for (int i = tid; i < kMRows * kMaxWin; i += 64 * kSlots) {
            const int m = i / kMaxWin, wi = i - m * kMaxWin;
            wexp[i] = (m < mr && wi < nwin) ? win_exp(wmax[i]) : 0;
        }
        __syncthreads();
    }
    if (early) {
        vm_wait_for<(NB - 1) * CK::kInstr>(ev);  // the early items have landed; the chunks may still fly
#pragma unroll
        for (int e = 0; e < kEarly; ++e) {
            const int it = tid + e * 64 * kSlots;
            if (it < items) {
                _Float16 h[16];
                __builtin_memcpy(h, &ev[e][0], 16);
                __builtin_memcpy(h + 8, &ev[e][1], 16);
                float x[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) x[i] = static_cast<float>(h[i]);
                stage_item<F, TA>(it, per_row, K, rs, true, x, wexp);
            }
        }
        stage_rows<F, TA>(A, M, K, m0, mr, vec, wexp, tid + kEarly * 64 * kSlots, 64 * kSlots);
    } else {
        stage_rows<F, TA>(A, M, K, m0, mr, vec, wexp, tid, 64 * kSlots);
    }

    // activation row read by this lane: rows past the pass read row 0 (their MFMA output rows are never
    // stored; MFMA rows are independent)
    const uint8_t* abase = mlds + (n < mr ? n : 0) * rs;
    const uint32_t mg = mkeep(0x64006400u);
    const int qrows = (mr + 3) >> 2;  // lane quarters holding output rows
    const int qa = (lrows + 3) >> 2;  // lane quarters with partial-sum space

    float y[R];
#pragma unroll
    for (int r = 0; r < R; ++r) y[r] = 0.0f;

    // Adds the 8 slot partials of the workgroup's li-th row group (written before the last barrier) in
    // slot order and stores its outputs (wave li % 8).
    auto reduce_store = [&](int li) {
        if (w != (li & (kSlots - 1)) || c >= qrows) return;
        const uint8_t* rb = red + (li & 1) * (kSlots * 16 * qa * 16);
        mf4 v[kSlots];
#pragma unroll
        for (int q = 0; q < kSlots; ++q) v[q] = *reinterpret_cast<const mf4*>(rb + (q * 16 * qa + lane) * 16);
        mf4 sum = v[0];
#pragma unroll
        for (int q = 1; q < kSlots; ++q)
#pragma unroll
            for (int r = 0; r < R; ++r) sum[r] += v[q][r];
        const int g = static_cast<int>(blockIdx.x) + li * static_cast<int>(gridDim.x);
        const uint8_t* W;
        TC* Cp;
        int N, g0;
        seg_pick(sg, g, W, Cp, N, g0);
        const int row = (g - g0) * kRows + n;
        if (row < N) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int m = 4 * c + r;
                if (m < mr) mstore<TC>(Cp + static_cast<size_t>(m0 + m) * N + row, sum[r]);
            }
        }
    };

    int cli = 0, cch = 0, cslot = 0;  // compute cursor
    for (int i = 0; i < total; ++i) {
        // this wave's copies of chunk i have landed (chunks i + 1 .. i + NB - 2 may still be in flight)
        vm_wait<(NB - 2) * CK::kInstr>();
        lds_sync();
        if (cch == 0 && cli > 0) reduce_store(cli - 1);
        issue();
        const int li = cli, ch = cch;
        const int sbr = ch * kSlots + w;
        const bool take = sbr < nsb;
        const int sb = min(sbr, nsb - 1);
        const typename F::Raw raw = F::load(ring + cslot * CK::kBytes + n * CK::kRP * 16 + w * F::kBlockBytes, c);
        const typename F::Pre p = F::prep(raw, c);
        mf4 T = {0.0f, 0.0f, 0.0f, 0.0f};
        mf4 T2 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const mh8 af = *reinterpret_cast<const mh8*>(abase + 2 * (256 * sb + F::k0(c, t)));
            mh8 bw[F::kChains];
            F::steps(raw, p, t, mg, bw);
            T = mfma16(af, bw[0], T);
            if constexpr (F::kChains == 2) T2 = mfma16(af, bw[1], T2);
        }
        mf4 U = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (F::kSums) {
            const mh8 as = *reinterpret_cast<const mh8*>(abase + 2 * K + 64 * sb + 16 * c);
            U = mfma16(as, p.bu, U);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float tv = T[r];
            if constexpr (F::kChains == 2) tv = __fmaf_rn(16.0f, T2[r], tv);
            const float uv = U[r];
            float yn;
            const int e = kF32 ? wexp[min(4 * c + r, kMRows - 1) * kMaxWin + (sb >> 4)] : 0;
            if (kF32 && e != 0) {
                // rescaled window: the super-block's net d T - dmin U first (its two terms can
                // leave the fp32 range where their difference does not), then times 2^e
                const float net = F::kSums ? __fmaf_rn(p.d, tv, -(p.c2 * uv)) : p.d * tv;
                yn = y[r] + __builtin_ldexpf(net, e);
            } else {
                const float yd = __fmaf_rn(p.d, tv, y[r]);
                yn = F::kSums ? __fmaf_rn(-p.c2, uv, yd) : yd;
            }
            y[r] = take ? yn : y[r];
        }
        if (ch == cpr - 1) {
            // row group done: this slot's partial goes to LDS; added after the next barrier
            if (c < qrows) {
                mf4 v = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int r = 0; r < R; ++r) v[r] = y[r];
                *reinterpret_cast<mf4*>(red + (li & 1) * (kSlots * 16 * qa * 16) + (w * 16 * qa + lane) * 16) = v;
            }
#pragma unroll
            for (int r = 0; r < R; ++r) y[r] = 0.0f;
        }
        cslot = cslot + 1 == NB ? 0 : cslot + 1;
        if (++cch == cpr) {
            cch = 0;
            ++cli;
        }
    }
    vm_wait<0>();  // the tail requests land before the wave ends
    lds_sync();
    reduce_store(mine - 1);
}

// ------------------------------------------------------------------------------------------------
// Host side.
// ------------------------------------------------------------------------------------------------
std::mutex g_mm_mutex;

struct MDev {
    int cus = 0;
    size_t max_lds = 0;
};

hipError_t mdev(MDev& out) {
    static std::unordered_map<int, MDev> cache;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(g_mm_mutex);
    auto it = cache.find(dev);
    if (it != cache.end()) {
        out = it->second;
        return hipSuccess;
    }
    MDev d;
    int v = 0;
    if ((e = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    d.cus = v;
    if ((e = hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev)) != hipSuccess) return e;
    d.max_lds = static_cast<size_t>(v);
    cache[dev] = d;
    out = d;
    return hipSuccess;
}

hipError_t mocc(const void* kern, size_t lds, int& blocks) {
    static std::unordered_map<std::string, int> cache;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const std::string key = std::to_string(dev) + ":" + std::to_string(reinterpret_cast<uintptr_t>(kern)) + ":" + std::to_string(lds);
    std::unique_lock<std::mutex> lock(g_mm_mutex);
    auto it = cache.find(key);
    if (it != cache.end()) {
        blocks = it->second;
        return hipSuccess;
    }
    if (lds > 65536) {
        // the kernel's limit is raised to the device's maximum (a per-kernel attribute: setting it to this
        // call's size would lower it for a later, larger call that finds its occupancy cached)
        MDev di;
        lock.unlock();
        if ((e = mdev(di)) != hipSuccess) return e;
        lock.lock();
        hipFuncAttributes fa;
        if ((e = hipFuncGetAttributes(&fa, kern)) != hipSuccess) return e;
        e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                static_cast<int>(di.max_lds - fa.sharedSizeBytes));
        if (e != hipSuccess) return e;
    }
    int nb = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern, 64 * kSlots, lds);
    if (e != hipSuccess) return e;
    blocks = nb > 0 ? nb : 1;
    cache[key] = blocks;
    return hipSuccess;
}


template <class F>
size_t mlds_bytes(int lrows, int K, int nb) {
    return static_cast<size_t>(lrows) * row_stride<F>(K) + static_cast<size_t>(nb) * Chunk<F>::kBytes + red_bytes(lrows);
}

// Activation rows per pass: up to 16, as many as the LDS holds beside a ring of nb weight chunks (rows
// of a pass share every weight byte loaded; each further pass streams the weights again).  0 when not
// even one row fits.
template <class F>
int pass_rows(int M, int K, int nb, size_t max_lds) {
    max_lds -= kStaticLds;
    int best = 0;
    for (int r = 1; r <= min(M, kMRows); ++r)
        if (mlds_bytes<F>(r, K, nb) <= max_lds) best = r;
    if (best == 0) return 0;
    // balance the passes: the fewest rows per pass that keep the same pass count
    const int passes = (M + best - 1) / best;
    return (M + passes - 1) / passes;
}

template <class F, int R, int NB, typename TA, typename TC>
const void* mkern() {
    return reinterpret_cast<const void*>(&gemv_mfma_kernel<F, R, NB, TA, TC>);
}

template <class F, int R, int NB, typename TA, typename TC>
hipError_t mlaunch(const void* A, const MSegs<TC>& sg, int nrg, int M, int K, bool a_vec, int lrows, int occ, int cus,
                   hipStream_t stream) {
    const size_t lds = mlds_bytes<F>(lrows, K, NB);
    const int fill = max(1, occ * cus);
    const dim3 grid(min(nrg, fill), (M + lrows - 1) / lrows);
    hipLaunchKernelGGL((gemv_mfma_kernel<F, R, NB, TA, TC>), grid, dim3(64 * kSlots), lds, stream,
                       static_cast<const TA*>(A), sg, M, K, nrg, a_vec ? 1 : 0, lrows);
    return hipGetLastError();
}

template <class F, int R, typename TA, typename TC>
hipError_t mlaunch_ring(const void* A, const MSegs<TC>& sg, int nrg, int M, int K, bool a_vec, const MDev& di,
                        hipStream_t stream) {
    // ring of 3 or 4 chunks: fewer passes first, then more chunks in flight per CU (workgroups per CU
    // times ring depth - 1), then the shallower ring
    const int lr3 = pass_rows<F>(M, K, 3, di.max_lds), lr4 = pass_rows<F>(M, K, 4, di.max_lds);
    if (lr3 == 0) return hipErrorNotSupported;
    hipError_t e;
    int occ3 = 0, occ4 = 0;
    if ((e = mocc(mkern<F, R, 3, TA, TC>(), mlds_bytes<F>(lr3, K, 3), occ3)) != hipSuccess) return e;
    const int p3 = (M + lr3 - 1) / lr3;
    bool use4 = false;
    if (lr4 > 0) {
        if ((e = mocc(mkern<F, R, 4, TA, TC>(), mlds_bytes<F>(lr4, K, 4), occ4)) != hipSuccess) return e;
        const int p4 = (M + lr4 - 1) / lr4;
        use4 = p4 < p3 || (p4 == p3 && 3 * occ4 > 2 * occ3);
    }
    if (use4) return mlaunch<F, R, 4, TA, TC>(A, sg, nrg, M, K, a_vec, lr4, occ4, di.cus, stream);
    return mlaunch<F, R, 3, TA, TC>(A, sg, nrg, M, K, a_vec, lr3, occ3, di.cus, stream);
}

template <class F, typename TA, typename TC>
hipError_t mdispatch(const void* A, const void* const* W, void* const* C, const int* N, int count, int M, int K,
                     hipStream_t stream) {
    MSegs<TC> sg;
    int nrg = 0;
    for (int j = 0; j < 4; ++j) {
        if (j < count) {
            sg.W[j] = static_cast<const uint8_t*>(W[j]);
            sg.C[j] = static_cast<TC*>(C[j]);
            sg.N[j] = N[j];
            nrg += (N[j] + kRows - 1) / kRows;
            sg.gend[j] = nrg;
        } else {
            sg.W[j] = sg.W[0];
            sg.C[j] = sg.C[0];
            sg.N[j] = sg.N[0];
            sg.gend[j] = INT_MAX;
        }
    }
    MDev di;
    hipError_t e = mdev(di);
    if (e != hipSuccess) return e;
    const bool a_vec = (reinterpret_cast<uintptr_t>(A) & 15u) == 0;
    // R by the rows of a pass: a ring of 3 bounds them from above (a ring of 4 holds no more)
    const int lrows = pass_rows<F>(M, K, 3, di.max_lds);
    if (lrows == 0) return hipErrorNotSupported;
    if (lrows <= 1) return mlaunch_ring<F, 1, TA, TC>(A, sg, nrg, M, K, a_vec, di, stream);
    if (lrows <= 2) return mlaunch_ring<F, 2, TA, TC>(A, sg, nrg, M, K, a_vec, di, stream);
    return mlaunch_ring<F, 4, TA, TC>(A, sg, nrg, M, K, a_vec, di, stream);
}

template <class F>
hipError_t mdtypes(int a_dtype, int c_dtype, const void* A, const void* const* W, void* const* C, const int* N, int count,
                   int M, int K, hipStream_t stream) {
    if (a_dtype == QMM_DTYPE_F32) {
        if (c_dtype == QMM_DTYPE_F32) return mdispatch<F, float, float>(A, W, C, N, count, M, K, stream);
        return mdispatch<F, float, __half>(A, W, C, N, count, M, K, stream);
    }
    if (c_dtype == QMM_DTYPE_F32) return mdispatch<F, __half, float>(A, W, C, N, count, M, K, stream);
    return mdispatch<F, __half, __half>(A, W, C, N, count, M, K, stream);
}

}  // namespace

// Q4_K takes the matrix-core GEMV.  Q6_K is not dispatched here: the v_dot2 kernels are faster for it
// at every measured shape (its activations and 26 KiB weight chunks leave one workgroup per CU).
bool gemv_mfma_type(int ggml_type) { return ggml_type == QMM_TYPE_Q4_K; }

hipError_t launch_gemv_mfma(int ggml_type, const void* A, int a_dtype, int c_dtype, int M, int K, const void* const* W,
                            void* const* C, const int* N, int count, hipStream_t stream) {
    if (count < 1 || count > 4 || M < 1 || K < 256 || K % 256 != 0 || K > kMaxWin * kWinK) return hipErrorNotSupported;
    for (int j = 0; j < count; ++j)
        if (N[j] < 1 || (reinterpret_cast<uintptr_t>(W[j]) & 15u) != 0) return hipErrorNotSupported;
    // the weight chunks are copied in 16-byte pieces: rows must be whole pieces
    if (ggml_type == QMM_TYPE_Q6_K && K % 2048 != 0) return hipErrorNotSupported;
    switch (ggml_type) {
        case QMM_TYPE_Q4_K: return mdtypes<MQ4K>(a_dtype, c_dtype, A, W, C, N, count, M, K, stream);
        case QMM_TYPE_Q6_K: return mdtypes<MQ6K>(a_dtype, c_dtype, A, W, C, N, count, M, K, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace qmm
