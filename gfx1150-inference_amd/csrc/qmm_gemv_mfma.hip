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
//   * Q4_K codes become exact f16 integers s * q: one v_and_or_b32 turns two codes into (1024 + q)
//     or (1024 + 16q) (0x6400 | bits), one v_pk_fma_f16 with (s, -1024 s) or (s / 16, -64 s) leaves
//     s * q exactly (s the 6-bit sub-scale, |s * q| <= 945).  Q6_K: two v_perm make the f16 pairs
//     (1024 + u) of the byte-assembled 6-bit codes, v_pk_add_f16 with -1056 leaves u - 32 exactly and
//     v_pk_mul_f16 by the int8 sub-scale s gives s (u - 32), exact while |s (u - 32)| <= 2048 and
//     otherwise rounded once (|s (u - 32)| <= 4096: an error of at most 1, below the f16 rounding of
//     d s (u - 32) in the reference's dequantized weights).  The MFMA's products of these operands
//     are exact; its fp32 sums round.
//   * Per super-block and row: Q4_K y += d * T - c2 * U, where U is a second MFMA over the per-group
//     sums of the staged activations (held as f16 hi + lo pairs of sum / 32) against the 6-bit group
//     minima (c2 = 32 dmin); Q6_K y += d * T (its code offset is inside the B operand).
//   * The K range of a row group is cut into 8 fixed slots (super-blocks sb with sb % 8 = slot), one
//     per wave of the 8-wave workgroup; a wave adds its slot's super-blocks in order and the 8 slot
//     sums are added in slot order through LDS.  Every row's arithmetic is therefore the same
//     instruction sequence whatever M, the row group's place and the grid; MFMA rows are
//     independent, so row m of any M is bit-identical to the M = 1 call (the reference's
//     prefill-vs-M=1 invariant, tests/test_phase5_scale.py:274-310).
//   * Weights stream through an LDS ring of NB (3 or 4) chunks of 16 rows x 8 super-blocks (a window of
//     K), copied by the whole workgroup with direct global -> LDS 16-byte loads (each instruction reads
//     whole row segments); NB - 1 chunks are in flight while one is multiplied.
//   * Windows are the outer loop over a batch of up to 4 row groups: a wave holds the activation
//     operands of its super-block of the window in registers (up to 16 rows per pass) and applies them
//     to every row group of the batch, whose accumulators stay in registers.  fp16 activations reach
//     registers through a per-wave LDS area filled by the same direct loads one window ahead; fp32
//     activations are loaded directly and rounded to f16, with a power-of-two rescale of any
//     (row, super-block) outside f16's range.  The work of a pass hardly depends on its row count.
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
// consecutive k in the pair order (0, 2), (1, 3), (4, 6), (5, 7).  Q4_K's group sums (group_sums):
// quarter c holds sub-blocks 2c and 2c + 1, their hi halves at 0, 1 and lo halves at 2, 3 of the sum
// fragment.
// ------------------------------------------------------------------------------------------------

// Q4_K (reference block_q4_k, src/kernels/dequantize.hip:31-36; get_scale_min_k4 :52-65).
struct MQ4K {
    static constexpr int kType = QMM_TYPE_Q4_K;
    static constexpr int kBlockBytes = kBytesQ4_K;
    static constexpr bool kSums = true;  // group minima: a second MFMA over the activations' group sums
    struct Raw {
        mu4 h, q0, q1;
    };
    __device__ static int k0(int c, int t) { return 64 * c + 8 * t; }
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
        // Sub-blocks j = 2c + g.  j < 4 (c < 2): 6-bit scale and min at byte j of words 1 and 2.
        // j >= 4: low 4 bits in byte j - 4 of word 3 (scale: low nibble, min: high nibble), top 2 bits
        // in bits 6..7 of byte j - 4 of words 1 and 2.  Per lane: the word of the low bits and the bit
        // offsets (loop-invariant), then three field extracts per value.
        const bool lo = c < 2;
        const uint32_t ws = lo ? r.h.y : r.h.w, wm = lo ? r.h.z : r.h.w;
        uint32_t sc[2], mn[2];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const uint32_t b = 8 * ((2 * c + g) & 3);
            const uint32_t top = b + (lo ? 4u : 6u);
            sc[g] = __builtin_amdgcn_ubfe(ws, b, 4) | (__builtin_amdgcn_ubfe(r.h.y, top, 2) << 4);
            mn[g] = __builtin_amdgcn_ubfe(wm, b + (lo ? 0u : 4u), 4) | (__builtin_amdgcn_ubfe(r.h.z, top, 2) << 4);
        }
        const _Float16 s0 = static_cast<_Float16>(static_cast<uint16_t>(sc[0]));  // exact: < 64
        const _Float16 s1 = static_cast<_Float16>(static_cast<uint16_t>(sc[1]));
        p.s_lo = pair_of(s0);
        p.o_lo = pair_of(s0 * static_cast<_Float16>(-1024.0f));
        p.s_hi = pair_of(s1 * static_cast<_Float16>(0.0625f));
        p.o_hi = pair_of(s1 * static_cast<_Float16>(-64.0f));
        const _Float16 f0 = static_cast<_Float16>(static_cast<uint16_t>(mn[0])), f1 = static_cast<_Float16>(static_cast<uint16_t>(mn[1]));
        const _Float16 r11 = static_cast<_Float16>(1.0f / 2048.0f), z = static_cast<_Float16>(0.0f);
        p.bu = mh8{f0, f1, f0 * r11, f1 * r11, z, z, z, z};
        p.d = half_bits_to_float(r.h.x);
        p.c2 = 32.0f * half_bits_to_float(r.h.x >> 16);
        p.sh[0] = r.q0.x >> 8; p.sh[1] = r.q0.y >> 8; p.sh[2] = r.q0.z >> 8; p.sh[3] = r.q0.w >> 8;
        p.sh[4] = r.q1.x >> 8; p.sh[5] = r.q1.y >> 8; p.sh[6] = r.q1.z >> 8; p.sh[7] = r.q1.w >> 8;
        return p;
    }
    // B operand of step t: t < 4 low nibbles of dwords 2t, 2t + 1 of the chunk, t >= 4 the high nibbles
    // of dwords 2(t - 4), 2(t - 4) + 1.
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
// Step st = 2 t + (j >= 8).  The 6-bit code u (w = d sc (u - 32)) is assembled bytewise, two v_perm
// make the f16 pairs (1024 + u), and the B operand is sc (u - 32): one chain, and the code offset
// needs no second sum.
struct MQ6K {
    static constexpr int kType = QMM_TYPE_Q6_K;
    static constexpr int kBlockBytes = kBytesQ6_K;
    static constexpr bool kSums = false;
    struct Raw {
        mu4 la, lb, qh;
        uint32_t s0, s1, d;
    };
    __device__ static int k0(int c, int st) { return 128 * (c >> 1) + 32 * (st >> 1) + 16 * (c & 1) + 8 * (st & 1); }
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
        uint32_t s[4];  // (sc, sc) per t
        mh8 bu;         // unused (no group sums)
        float d, c2;    // d, 0
    };
    __device__ static Pre prep(const Raw& r, int c) {
        Pre p;
        const int h = c & 1;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t w = t < 2 ? r.s0 : r.s1;
            const _Float16 sc = static_cast<_Float16>(static_cast<float>(static_cast<int8_t>(w >> (8 * (h + 2 * (t & 1))))));
            p.s[t] = pair_of(sc);
        }
        p.d = half_bits_to_float(r.d);
        p.c2 = 0.0f;
        return p;
    }
    // B operand of step st: sc (u - 32) for bytes 8 (st & 1) .. + 7 of the lane's slices (weights
    // j = 8 (st & 1) + 0..7 of group t = st / 2).
    __device__ static mh8 step(const Raw& r, const Pre& p, int st, uint32_t mg) {
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
        // (1024 + u) - 1056 = u - 32 exactly, then times sc: one rounding where |sc (u - 32)| > 2048
        const mh2 off = {static_cast<_Float16>(-1056.0f), static_cast<_Float16>(-1056.0f)};
        const mh2 sv = as_mh2(p.s[t]);
        const mh2 r0 = (as_mh2(cd[0]) + off) * sv, r1 = (as_mh2(cd[1]) + off) * sv;
        const mh2 r2 = (as_mh2(cd[2]) + off) * sv, r3 = (as_mh2(cd[3]) + off) * sv;
        const _Float16 __attribute__((ext_vector_type(4))) lo = __builtin_shufflevector(r0, r1, 0, 1, 2, 3);
        const _Float16 __attribute__((ext_vector_type(4))) hi = __builtin_shufflevector(r2, r3, 0, 1, 2, 3);
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
};

// ------------------------------------------------------------------------------------------------
// LDS of a workgroup (dynamic):
//   ring  NB weight chunks of Chunk<F>::kBytes;
//   act   fp16 activations only: per wave, the pass's rows of the wave's super-block of the current
//         window, lrows rows x 32 16-byte pieces (the 512 bytes of a row), piece p of row r at slot
//         p ^ r, so that the 16 rows' pieces p fall in different banks;
//   red   slot partials of a batch: bg (up to kBG) row groups x 8 waves x 16 qa lanes x 16 bytes.
// ------------------------------------------------------------------------------------------------
extern __shared__ __attribute__((aligned(16))) uint8_t mlds[];

constexpr int kBG = 4;     // row groups per batch at most: their accumulators stay in registers across the windows
constexpr int kActP = 32;  // 16-byte pieces of one super-block of one fp16 activation row

__host__ __device__ constexpr int act_bytes(int lrows) { return kSlots * lrows * kActP * 16; }
__host__ __device__ constexpr int red_bytes(int lrows, int bg) { return bg * kSlots * 16 * ((lrows + 3) / 4) * 16; }

__device__ __forceinline__ int win_exp(uint32_t maxbits) {
    // (row, super-block) maximum at or above 65504, or in [2^-126, 2^-14): scale by 2^-e with
    // e = exponent(max) - 14 (brings the maximum into [2^14, 2^15))
    const bool big = maxbits >= 0x477FE000u && maxbits < 0x7F800000u;
    const bool tiny = maxbits >= 0x00800000u && maxbits < 0x38800000u;
    return big || tiny ? static_cast<int>(maxbits >> 23) - 127 - 14 : 0;
}

// Activation operands of one super-block for lane (n, c): the A operand of each MFMA step (8 k in the
// pair order of the decoded codes) and, for formats with group sums, the sums operand.
struct AOps {
    mh8 a[8];
    mh8 s;
};

// (x0, x1, .., x7) -> (x0, x2, x1, x3, x4, x6, x5, x7)
__device__ __forceinline__ mh8 pair_order(mu4 v) {
    mu4 r;
    r.x = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);
    r.y = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);
    r.z = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);
    r.w = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);
    mh8 h;
    __builtin_memcpy(&h, &r, 16);
    return h;
}

// Group sums of the 8 fragments (Q4_K: steps 0..3 and 4..7 are the lane's two 32-k groups), summed in a
// fixed order and held as f16 hi + lo * 2^-11 of sum / 32 (exact power-of-two scalings; the remainder
// scaled by 2^11 stays a normal f16, and the B operand's halves carry the 2^-11).
template <class F>
__device__ __forceinline__ void group_sums(AOps& ao) {
    if constexpr (F::kSums) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        const h2 one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
        _Float16 hi[2], lo[2];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            float s = 0.0f;
#pragma unroll
            for (int t = 4 * g; t < 4 * g + 4; ++t) {
                const mh8 v = ao.a[t];
#pragma unroll
                for (int i = 0; i < 4; ++i) s = __builtin_amdgcn_fdot2(h2{v[2 * i], v[2 * i + 1]}, one, s, false);
            }
            const float x = s * 0.03125f;
            hi[g] = static_cast<_Float16>(x);
            lo[g] = static_cast<_Float16>((x - static_cast<float>(hi[g])) * 2048.0f);
        }
        const _Float16 z = static_cast<_Float16>(0.0f);
        ao.s = mh8{hi[0], hi[1], lo[0], lo[1], z, z, z, z};
    }
}

// fp16 activations of the current window from this wave's LDS area (row n of the pass; lanes of rows
// past the pass read row 0: their MFMA output rows are never stored, and MFMA rows are independent).
template <class F>
__device__ __forceinline__ void read_act(const uint8_t* wact, int n, int c, int mr, AOps& ao) {
    const int r = n < mr ? n : 0;
    const uint8_t* row = wact + r * kActP * 16;
#pragma unroll
    for (int t = 0; t < 8; ++t)
        ao.a[t] = pair_order(*reinterpret_cast<const mu4*>(row + 16 * ((F::k0(c, t) >> 3) ^ r)));
    group_sums<F>(ao);
}

// Activations straight from memory (fp32, or fp16 not 16-byte aligned): row n of the pass, super-block
// sb.  fp32 rows are rounded to f16 after scaling by 2^-e, e from the maximum over the row's super-block
// (the four lane quarters of row n together hold it), and e is returned (0 for fp16).
template <class F, typename TA>
__device__ __forceinline__ int load_act(const TA* __restrict__ A, int K, int row, int sb, int c, bool vec, AOps& ao) {
    const TA* p = A + static_cast<size_t>(row) * K + 256 * sb;
    float x[8][8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const TA* q = p + F::k0(c, t);
        if constexpr (std::is_same<TA, float>::value) {
            if (vec) {
                const float4 u = reinterpret_cast<const float4*>(q)[0], v = reinterpret_cast<const float4*>(q)[1];
                x[t][0] = u.x; x[t][1] = u.y; x[t][2] = u.z; x[t][3] = u.w;
                x[t][4] = v.x; x[t][5] = v.y; x[t][6] = v.z; x[t][7] = v.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) x[t][i] = q[i];
            }
        } else {
            const uint16_t* s = reinterpret_cast<const uint16_t*>(q);
#pragma unroll
            for (int i = 0; i < 8; ++i) x[t][i] = half_bits_to_float(s[i]);
        }
    }
    int e = 0;
    if constexpr (std::is_same<TA, float>::value) {
        float mx = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(x[t][i]));
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        e = win_exp(__float_as_uint(mx));
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        _Float16 h[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) h[i] = static_cast<_Float16>(__builtin_ldexpf(x[t][i], -e));
        ao.a[t] = mh8{h[0], h[2], h[1], h[3], h[4], h[6], h[5], h[7]};
    }
    group_sums<F>(ao);
    return e;
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
// LDS address m0 + 16 l (m0 is an operand, so the compiler sets it).  The compiler does not track
// these loads; they are waited for with explicit vmcnt counts (vector memory operations complete in
// issue order, so waiting until at most N remain outstanding completes every operation issued before
// the last N).
__device__ __forceinline__ void dma16(const void* g, uint32_t lds_m0) {
    __asm__ volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds_m0) : "memory");
}
// The same from a buffer (raw, stride 0): 16 bytes at voff of the resource, where a read at or past the
// resource's size returns zeros; the base address and size live in scalar registers, so a lane's
// address is one 32-bit offset.
constexpr uint32_t kBufferWord3 = 0x00020000u;  // buffer resource word 3: raw dword access
__device__ __forceinline__ void dma16b(mu4 rsrc, uint32_t voff, uint32_t lds_m0) {
    __asm__ volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(lds_m0) : "memory");
}
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// vm_wait with a wave-uniform count; counts above 15 wait for 15 (more than needed).
__device__ __forceinline__ void vm_wait_rt(int n) {
    switch (n) {
        case 0: vm_wait<0>(); break;
        case 1: vm_wait<1>(); break;
        case 2: vm_wait<2>(); break;
        case 3: vm_wait<3>(); break;
        case 4: vm_wait<4>(); break;
        case 5: vm_wait<5>(); break;
        case 6: vm_wait<6>(); break;
        case 7: vm_wait<7>(); break;
        case 8: vm_wait<8>(); break;
        case 9: vm_wait<9>(); break;
        case 10: vm_wait<10>(); break;
        case 11: vm_wait<11>(); break;
        case 12: vm_wait<12>(); break;
        case 13: vm_wait<13>(); break;
        case 14: vm_wait<14>(); break;
        default: vm_wait<15>(); break;
    }
}
__device__ __forceinline__ void lds_sync() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void lds_reads_done() { __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

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

// A pass of lrows (<= 16) activation rows over the workgroup's row groups.  K is cut into windows of 8
// super-blocks; window j's super-block 8 j + w belongs to wave w (its slot).  Row groups are taken in
// batches of kBG: for each window, every row group of the batch multiplies its chunk (16 rows x the
// window's 8 super-blocks) by the window's activations, which each wave holds in registers for its own
// super-block, so the activations are read once per batch and window whatever the number of rows.
// Accumulators of the batch stay in registers; at the batch's end the 8 slot partials of each row group
// are added in slot order through LDS.  A row's arithmetic (slot w adds its super-blocks in order, then
// the slots are added in order) does not depend on M, the batch or the grid.
// Per chunk step: wave w waits for its own copies of the chunk, one barrier (all copies landed; every
// wave is done with the slot refilled next), then it requests chunk i + NB - 1 into that slot and
// multiplies super-block w of chunk i for the 16 rows from LDS.  Chunks are requested in the order they
// are multiplied: batch, window, row group.
// R: accumulated values per lane (min(rows of the pass, 4) for one lane quarter holding rows;
// 4 for passes of more than 4 rows, where quarter c holds rows 4c .. 4c + 3).  NB: ring slots.
template <class F, int R, int NB, typename TA, typename TC>
__global__ __launch_bounds__(64 * kSlots) void gemv_mfma_kernel(const TA* __restrict__ A, MSegs<TC> sg, int M, int K,
                                                                 int nrg, int a_vec, int lrows, int bg) {
    using CK = Chunk<F>;
    constexpr bool kF32 = std::is_same<TA, float>::value;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n = lane & 15, c = lane >> 4;
    const int m0 = blockIdx.y * lrows;
    const int mr = min(lrows, M - m0);
    const int nsb = K >> 8;
    const int nwin = (nsb + kSlots - 1) / kSlots;
    const int mine = (nrg - static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) - 1) / static_cast<int>(gridDim.x);
    const int row_bytes = nsb * F::kBlockBytes;
    const bool vec = a_vec != 0;
    // activations through this wave's LDS area (fp16, 16-byte aligned), else straight from memory
    const bool staged = !kF32 && vec;
    uint8_t* ring = mlds;
    uint8_t* wact = ring + NB * CK::kBytes + w * lrows * kActP * 16;
    uint8_t* red = ring + NB * CK::kBytes + (kF32 ? 0 : act_bytes(lrows));
    const uint32_t ring_m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ring));
    const uint32_t wact_m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(wact));
    const int qa = (lrows + 3) >> 2;  // lane quarters with partial-sum space
    const int qrows = (mr + 3) >> 2;  // lane quarters holding output rows

    // Per-lane constants of the chunk copies: instruction k moves this lane's piece q = 64 k + lane of the
    // wave's two rows (row r = q / kRP, piece pc of it; the row's padding piece repeats its last piece),
    // at byte lane_vo[k] from the window's start in the first row.
    uint32_t lane_vo[CK::kInstr];
    bool lane_r1[CK::kInstr];
#pragma unroll
    for (int k = 0; k < CK::kInstr; ++k) {
        const int q = 64 * k + lane;
        lane_r1[k] = q >= CK::kRP;
        lane_vo[k] = 16 * min(q - (lane_r1[k] ? CK::kRP : 0), CK::kP - 1) + (lane_r1[k] ? row_bytes : 0);
    }
    // Issue cursor: batch start ib0 (row groups of this workgroup), its size ibs, window ij, row group iq
    // of the batch, ring slot islot.
    int ib0 = 0, ibs = min(bg, mine), ij = 0, iq = 0, islot = 0;
    // Requests the cursor's chunk into its slot and advances the cursor (past the workgroup's last chunk
    // it stays there: the tail requests re-read valid bytes, so every wave issues the same loads).
    auto issue = [&]() {
        const int g = static_cast<int>(blockIdx.x) + (ib0 + iq) * static_cast<int>(gridDim.x);
        const uint8_t* W;
        TC* Cs;
        int N, g0;
        seg_pick(sg, g, W, Cs, N, g0);
        // the wave's two source rows (row 2w + 1 clamped to the segment's last row)
        const int r0 = min((g - g0) * kRows + 2 * w, N - 1);
        const int r1 = min(r0 + 1, N - 1);
        const int cb = ij * kSlots * F::kBlockBytes;
        // the window of row r0 through the end of row r1 as a buffer: the last window's padding pieces
        // (unused) read past a row's end into the next row or, past row r1, zeros; with one row left
        // (r1 = r0) the second row's pieces read zeros (a row past the segment, never stored)
        const uint64_t base = reinterpret_cast<uint64_t>(W + static_cast<size_t>(r0) * row_bytes + cb);
        const mu4 rs = {static_cast<uint32_t>(base), static_cast<uint32_t>(base >> 32) & 0xFFFFu,
                        static_cast<uint32_t>((r1 - r0 + 1) * row_bytes - cb), kBufferWord3};
        const uint32_t dst = ring_m0 + static_cast<uint32_t>(islot * CK::kBytes + 2 * w * CK::kRP * 16);
#pragma unroll
        for (int k = 0; k < CK::kInstr; ++k)
            if (64 * k + 64 <= 2 * CK::kRP || 64 * k + lane < 2 * CK::kRP) dma16b(rs, lane_vo[k], dst + 64 * 16 * k);
        islot = islot + 1 == NB ? 0 : islot + 1;
        if (iq + 1 < ibs) {
            ++iq;
        } else if (ij + 1 < nwin) {
            iq = 0;
            ++ij;
        } else if (ib0 + ibs < mine) {
            ib0 += ibs;
            ibs = min(bg, mine - ib0);
            iq = 0;
            ij = 0;
        }
    };
    // Requests window j's activations (fp16, staged) into this wave's area: the pass's rows of super-block
    // 8 j + w; lane slot q = 64 i + lane of instruction i is row q / 32, slot q % 32, which holds the
    // row's piece (q % 32) ^ row.
    const int act_instr = (mr * kActP + 63) / 64;
    auto issue_act = [&](int j) {
        const int sb = min(kSlots * j + w, nsb - 1);
        const TA* base = A + static_cast<size_t>(m0) * K + 256 * sb;
        for (int i = 0; i < act_instr; ++i) {
            const int q = 64 * i + lane;
            const int r = q >> 5;
            const int pc = (q & (kActP - 1)) ^ r;
            if (q < mr * kActP) dma16(base + static_cast<size_t>(r) * K + 8 * pc, wact_m0 + 64 * 16 * i);
        }
    };

    if (staged) issue_act(0);
#pragma unroll
    for (int u = 0; u < NB - 1; ++u) issue();
    int act_after = (NB - 1) * CK::kInstr;  // vector memory operations issued after the pending activation copy

    const uint32_t mg = mkeep(0x64006400u);
    float acc[kBG][R];
    AOps ao;
    int eo[R];  // fp32: e of output rows 4c + r in the current window
#pragma unroll
    for (int r = 0; r < R; ++r) eo[r] = 0;
    int cslot = 0;

    for (int b0 = 0; b0 < mine; b0 += bg) {
        const int bs = min(bg, mine - b0);
#pragma unroll
        for (int q = 0; q < kBG; ++q)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[q][r] = 0.0f;
        for (int j = 0; j < nwin; ++j) {
            const int sbr = kSlots * j + w;
            const bool take = sbr < nsb;
            if (staged) {
                if (nwin > 1 || b0 == 0) {
                    vm_wait_rt(act_after);  // window j's activations have landed
                    read_act<F>(wact, n, c, mr, ao);
                    if (nwin > 1) {
                        lds_reads_done();  // the area is refilled with the next window's activations
                        issue_act(j + 1 < nwin ? j + 1 : 0);
                        act_after = 0;
                    }
                }
            } else {
                const int e = load_act<F, TA>(A, K, m0 + (n < mr ? n : 0), min(sbr, nsb - 1), c, vec, ao);
#pragma unroll
                for (int r = 0; r < R; ++r) eo[r] = __shfl(e, 4 * c + r, 64);
            }
#pragma unroll
            for (int q = 0; q < kBG; ++q) {
                if (q < bs) {
                    // this wave's copies of the chunk have landed (the next NB - 2 may still be in flight)
                    vm_wait<(NB - 2) * CK::kInstr>();
                    lds_sync();
                    issue();
                    act_after += CK::kInstr;
                    const typename F::Raw raw =
                        F::load(ring + cslot * CK::kBytes + n * CK::kRP * 16 + w * F::kBlockBytes, c);
                    const typename F::Pre p = F::prep(raw, c);
                    mf4 T = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int t = 0; t < 8; ++t) T = mfma16(ao.a[t], F::step(raw, p, t, mg), T);
                    mf4 U = {0.0f, 0.0f, 0.0f, 0.0f};
                    if constexpr (F::kSums) U = mfma16(ao.s, p.bu, U);
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const float tv = T[r];
                        const float uv = U[r];
                        float yn;
                        if (kF32 && eo[r] != 0) {
                            // rescaled activations: the super-block's net d T - dmin U first (its two terms
                            // can leave the fp32 range where their difference does not), then times 2^e
                            const float net = F::kSums ? __fmaf_rn(p.d, tv, -(p.c2 * uv)) : p.d * tv;
                            yn = acc[q][r] + __builtin_ldexpf(net, eo[r]);
                        } else {
                            const float yd = __fmaf_rn(p.d, tv, acc[q][r]);
                            yn = F::kSums ? __fmaf_rn(-p.c2, uv, yd) : yd;
                        }
                        acc[q][r] = take ? yn : acc[q][r];
                    }
                    cslot = cslot + 1 == NB ? 0 : cslot + 1;
                }
            }
        }
        // batch done: slot partials to LDS, one barrier, then wave q adds row group b0 + q's partials in
        // slot order and stores its outputs (the area is next written after at least one more barrier)
        if (c < qrows) {
#pragma unroll
            for (int q = 0; q < kBG; ++q) {
                if (q < bs) {
                    mf4 v = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int r = 0; r < R; ++r) v[r] = acc[q][r];
                    *reinterpret_cast<mf4*>(red + ((q * kSlots + w) * 16 * qa + lane) * 16) = v;
                }
            }
        }
        lds_sync();
        if (w < bs && c < qrows) {
            mf4 v[kSlots];
#pragma unroll
            for (int s = 0; s < kSlots; ++s) v[s] = *reinterpret_cast<const mf4*>(red + ((w * kSlots + s) * 16 * qa + lane) * 16);
            mf4 sum = v[0];
#pragma unroll
            for (int s = 1; s < kSlots; ++s)
#pragma unroll
                for (int r = 0; r < R; ++r) sum[r] += v[s][r];
            const int g = static_cast<int>(blockIdx.x) + (b0 + w) * static_cast<int>(gridDim.x);
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
        }
    }
    vm_wait<0>();  // the tail requests land before the wave ends
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


template <class F, typename TA>
size_t mlds_bytes(int lrows, int nb, int bg) {
    return static_cast<size_t>(nb) * Chunk<F>::kBytes + (std::is_same<TA, float>::value ? 0 : act_bytes(lrows)) +
           red_bytes(lrows, bg);
}

// Launch plan for a ring of nb chunks: activation rows per pass (up to 16, as many as the LDS holds
// beside the ring: rows of a pass share every weight byte loaded, each further pass streams the weights
// again; balanced over the passes) and row groups per batch (4, or fewer where that lets a pass hold more
// rows).  rows == 0 when not even one row fits.
struct MPlan {
    int rows = 0, bg = 0, passes = 0;
};
template <class F, typename TA>
MPlan mplan(int M, int nb, size_t max_lds) {
    MPlan best;
    for (int bg = kBG; bg >= 1; bg >>= 1) {
        int r = 0;
        for (int t = 1; t <= min(M, kMRows); ++t)
            if (mlds_bytes<F, TA>(t, nb, bg) <= max_lds) r = t;
        if (r == 0) continue;
        const int passes = (M + r - 1) / r;
        if (best.rows == 0 || passes < best.passes) best = MPlan{(M + passes - 1) / passes, bg, passes};
    }
    return best;
}

template <class F, int R, int NB, typename TA, typename TC>
const void* mkern() {
    return reinterpret_cast<const void*>(&gemv_mfma_kernel<F, R, NB, TA, TC>);
}

template <class F, int R, int NB, typename TA, typename TC>
hipError_t mlaunch(const void* A, const MSegs<TC>& sg, int nrg, int M, int K, bool a_vec, const MPlan& pl, int occ,
                   int cus, hipStream_t stream) {
    const size_t lds = mlds_bytes<F, TA>(pl.rows, NB, pl.bg);
    const int fill = max(1, occ * cus);
    const dim3 grid(min(nrg, fill), pl.passes);
    hipLaunchKernelGGL((gemv_mfma_kernel<F, R, NB, TA, TC>), grid, dim3(64 * kSlots), lds, stream,
                       static_cast<const TA*>(A), sg, M, K, nrg, a_vec ? 1 : 0, pl.rows, pl.bg);
    return hipGetLastError();
}

template <class F, int R, typename TA, typename TC>
hipError_t mlaunch_ring(const void* A, const MSegs<TC>& sg, int nrg, int M, int K, bool a_vec, const MDev& di,
                        hipStream_t stream) {
    // ring of 3 or 4 chunks: fewer passes first, then more chunks in flight per CU (workgroups per CU
    // times ring depth - 1), then the shallower ring.  Q6_K (one 26 KiB chunk of 16 rows x 8
    // super-blocks) takes a ring of 2 where that lets two workgroups share a CU (M <= 4): the second
    // workgroup's arithmetic then overlaps the first's waits (70B down at M = 4: 55 -> 51 us).
    const MPlan p3 = mplan<F, TA>(M, 3, di.max_lds), p4 = mplan<F, TA>(M, 4, di.max_lds);
    if (p3.rows == 0) return hipErrorNotSupported;
    hipError_t e;
    int occ3 = 0, occ4 = 0;
    if ((e = mocc(mkern<F, R, 3, TA, TC>(), mlds_bytes<F, TA>(p3.rows, 3, p3.bg), occ3)) != hipSuccess) return e;
    bool use4 = false;
    if (p4.rows > 0) {
        if ((e = mocc(mkern<F, R, 4, TA, TC>(), mlds_bytes<F, TA>(p4.rows, 4, p4.bg), occ4)) != hipSuccess) return e;
        use4 = p4.passes < p3.passes || (p4.passes == p3.passes && p4.bg >= p3.bg && 3 * occ4 > 2 * occ3);
    }
    if constexpr (F::kType == QMM_TYPE_Q6_K) {
        const MPlan p2 = mplan<F, TA>(M, 2, di.max_lds);  // (its rows per pass at most p3's)
        int occ2 = 0;
        if (p2.rows > 0 && p2.passes <= p3.passes) {
            if ((e = mocc(mkern<F, R, 2, TA, TC>(), mlds_bytes<F, TA>(p2.rows, 2, p2.bg), occ2)) != hipSuccess) return e;
            if (occ2 > occ3 && occ2 > occ4) return mlaunch<F, R, 2, TA, TC>(A, sg, nrg, M, K, a_vec, p2, occ2, di.cus, stream);
        }
    }
    if (use4) return mlaunch<F, R, 4, TA, TC>(A, sg, nrg, M, K, a_vec, p4, occ4, di.cus, stream);
    return mlaunch<F, R, 3, TA, TC>(A, sg, nrg, M, K, a_vec, p3, occ3, di.cus, stream);
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
    const int lrows = mplan<F, TA>(M, 3, di.max_lds).rows;
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

// Where the matrix-core GEMV runs.  Q4_K: from M = 2 (the v_dot2 GEMV is faster at M = 1; 70B gate
// 28672 x 8192: 26 against 30 us), and at M = 1 too in row-identity mode.  Q6_K: from M = 3 (70B down
// 8192 x 28672: 49-52 us at M = 3, 4 and 55-58 us at M = 8..16 against 41, 42, 72 and 98 us for v_dot2
// at M = 1, 2, 4, 8: its decode takes about 1.5 times the VALU work of Q4_K); row-identity mode keeps
// Q6_K on v_dot2 for every M, so that its M = 1 calls (decode) keep the faster kernel.
int gemv_mfma_min_m(int ggml_type, bool identity) {
    if (ggml_type == QMM_TYPE_Q4_K) return identity ? 1 : 2;
    if (ggml_type == QMM_TYPE_Q6_K) return identity ? INT_MAX : 3;
    return INT_MAX;
}

hipError_t launch_gemv_mfma(int ggml_type, const void* A, int a_dtype, int c_dtype, int M, int K, const void* const* W,
                            void* const* C, const int* N, int count, hipStream_t stream) {
    if (count < 1 || count > 4 || M < 1 || K < 256 || K % 256 != 0) return hipErrorNotSupported;
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
