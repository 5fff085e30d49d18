// Decode-path GEMV family (M < gemv_max_m(), 17 by default): C[m, n] = sum_k A[m, k] * dequant(W)[n, k].
//
// MI355X design (replaces the reference's wave32 one-output-per-wave kernels,
// src/kernels/dequantize.hip:97-148, 152-210, 232-332, 377-505, 549-685):
//   * K is walked in windows of 4096 weights.  In every window each of the 64 lanes of a wave
//     owns a fixed 64-weight slot of the packed row (a Q4_K 32-byte qs chunk, a Q6_K
//     (half, 16-column) slice, two Q8_0 / Q4_0 blocks) and streams it with 16-byte loads.
//   * A workgroup of NW waves owns NW * YT consecutive weight rows.  The window's activations
//     are staged once per workgroup into LDS as fp16 pairs, already in each lane's slot order,
//     together with per-16-k sums of the same fp16 values; the next window is staged and the
//     next window's weight bytes are loaded while the current window is multiplied.
//   * Codes are never converted one by one: a single v_and_or_b32 / v_perm_b32 turns two codes
//     q into the fp16 pair (1024 + q) (0x6400 | q), and v_dot2_f32_f16 multiplies two of them by
//     two activations and accumulates in fp32.  Per group g of the slot,
//         sum_k x_k * w_k = a_g * S_g - B_g * sx_g,   S_g = sum_k x_k * (1024 + q_k),
//     where sx_g is the sum of the group's fp16 activations and B_g folds the 1024 offset, the
//     format's code offset and the Q4_K min.  All products are exact; only fp32 sums round.
//   * fp32 activations are rounded to fp16 once, when staged; a (row, window) whose largest
//     magnitude lies outside f16's range is staged scaled by a power of two that the window's
//     group coefficients undo exactly (window_exp below).
//   * Activation rows are tiled in blocks of MR = 1, 2, 4 or 8 per workgroup (all rows of a
//     block share each weight byte loaded); blocks of 8 for M > 4 where they add no padded rows.
//   * The arithmetic of row (m, n) is the same instruction sequence for every M, YT and grid,
//     so every M < gemv_max_m() is bit-identical to M = 1 (the reference's prefill-vs-M=1
//     invariant, tests/test_phase5_scale.py:274-310); the cross-lane reduction is a fixed DPP
//     sequence (no atomics, deterministic).
#include <climits>
#include <mutex>
#include <string>
#include <type_traits>
#include <unordered_map>

#include "qmm_device.h"

namespace qmm {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));

constexpr int kGemvWindow = 4096;   // weights per row per window (64 lanes x 64)
constexpr int kChunks = 8;          // 8-weight activation chunks per lane slot

// Waves per workgroup of the v_dot2 kernels.
constexpr int kGemvNW = 8;
// LDS window slots per wave of the streamed kernel (one window is in flight while one is multiplied).
constexpr int kGemvNS = 2;
// Largest M whose launches switch to 16-wave workgroups when the staged activations exceed
// 40 KB of LDS (fewer workgroups per CU fit then; larger ones keep the waves per CU up).
constexpr int kGemvNW16MaxM = 2;

// Register-resident constants (v_and_or_b32 on gfx9 takes no literal operands).
struct Consts {
    uint32_t mg;   // 0x64006400: fp16 pair (1024, 1024)
    uint32_t m0f;  // 0x000F000F
    uint32_t mf0;  // 0x00F000F0
    uint32_t m3f;  // 0x003F003F
    uint32_t m3f0; // 0x03F003F0
    uint32_t mff;  // 0x00FF00FF
};

__device__ __forceinline__ uint32_t keep_v(uint32_t v) {
    __asm__("" : "+v"(v));
    return v;
}
__device__ __forceinline__ uint32_t keep_s(uint32_t v) {
    __asm__("" : "+s"(v));
    return v;
}

__device__ __forceinline__ Consts make_consts() {
    Consts c;
    c.mg = keep_v(0x64006400u);
    c.m0f = keep_s(0x000F000Fu);
    c.mf0 = keep_s(0x00F000F0u);
    c.m3f = keep_s(0x003F003Fu);
    c.m3f0 = keep_s(0x03F003F0u);
    c.mff = keep_s(0x00FF00FFu);
    return c;
}

__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t orv) { return (v & mask) | orv; }

__device__ __forceinline__ float dot2(uint32_t x, uint32_t c, float acc) {
    h16x2 a, b;
    __builtin_memcpy(&a, &x, 4);
    __builtin_memcpy(&b, &c, 4);
    return __builtin_amdgcn_fdot2(a, b, acc, false);
}

// x . c + 0 in one instruction: the VOP3 form takes the zero as an inline constant, where the
// accumulating form would need the zero moved into its destination first.
// (16 fewer VALU instructions per window item at M = 4, 1-4 % on the VALU-bound M >= 4 launches).
__device__ __forceinline__ float dot2_z(uint32_t x, uint32_t c) {
    float r;
    __asm__("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(x), "v"(c));
    return r;
}

__device__ __forceinline__ u32x4 ldg16(const uint8_t* p) {
    u32x4 v;
    __builtin_memcpy(&v, p, 16);  // any alignment: global_load_dwordx4
    return v;
}
__device__ __forceinline__ uint32_t ldg_u16(const uint8_t* p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}

// ------------------------------------------------------------------------------------------
// Formats.  Each defines the lane slot of a 4096-weight window:
//   xk(lane, cj): first k (relative to the window) of activation chunk cj (8 consecutive k);
//   load(): the slot's packed bytes of one row (addresses clamped to valid bytes);
//   chunk_codes(): the 4 fp16 code pairs of chunk cj, matching activation pairs
//                  (k0,k2), (k1,k3), (k4,k6), (k5,k7) of the chunk;
//   group_scales(): per group g (chunks 8g/G .. 8(g+1)/G - 1), a_g and B_g.
// ------------------------------------------------------------------------------------------

// Q4_K: lane = (super-block sb = lane/4, qs chunk c = lane%4): 64 weights, k = 64*lane + 0..63.
// Groups: g0 = sub-block 2c (low nibbles, chunks 0-3), g1 = sub-block 2c+1 (high nibbles, 4-7).
struct GQ4K {
    static constexpr int kType = QMM_TYPE_Q4_K;
    static constexpr int kQK = kQK_K;
    static constexpr int kBlockBytes = kBytesQ4_K;
    static constexpr int kWinBytes = 16 * kBytesQ4_K;  // 2304
    static constexpr int kG = 2;
    static constexpr bool kAligned = true;
    static constexpr bool kStream = false;  // lane-slot loads measured faster than the streamed window
    struct Raw {
        u32x4 h, q0, q1;
    };
    __device__ static int xk(int lane, int cj) { return 64 * lane + 8 * cj; }
    // Only whole super-blocks exist (K % 256 == 0): a lane is valid or not as a whole.
    __device__ static bool group_valid(int lane, int, int kwin_valid) { return 64 * lane < kwin_valid; }
    __device__ static Raw load(const uint8_t* win, int lane, int kwin_valid) {
        const int sb = lane >> 2, c = lane & 3;
        const bool v = 64 * lane < kwin_valid;
        const uint8_t* p = win + (v ? sb * kBytesQ4_K : 0);
        const int qo = v ? 16 + 32 * c : 16;
        Raw r;
        r.h = *reinterpret_cast<const u32x4*>(p);
        r.q0 = *reinterpret_cast<const u32x4*>(p + qo);
        r.q1 = *reinterpret_cast<const u32x4*>(p + qo + 16);
        return r;
    }
    __device__ static void chunk_codes(const Raw& r, int cj, const Consts& K, uint32_t out[4]) {
        const int j = 2 * (cj & 3);
        const u32x4& q = j < 4 ? r.q0 : r.q1;
        const uint32_t dlo = (j & 2) ? q.z : q.x;
        const uint32_t dhi = (j & 2) ? q.w : q.y;
        const uint32_t m = cj < 4 ? K.m0f : K.mf0;
        out[0] = and_or(dlo, m, K.mg);
        out[1] = and_or(dlo >> 8, m, K.mg);
        out[2] = and_or(dhi, m, K.mg);
        out[3] = and_or(dhi >> 8, m, K.mg);
    }
    // Sub-block j's (scale, min) (reference get_scale_min_k4, src/kernels/dequantize.hip:52-65).
    __device__ static void group_scales(const Raw& r, int lane, bool valid, float a[kG], float B[kG]) {
        const int c = lane & 3;
        const float d = half_bits_to_float(r.h.x);
        const float dmin = half_bits_to_float(r.h.x >> 16);
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            // both packings are decoded and selected (no lane-divergent branch)
            const int sh = 8 * ((2 * c + g) & 3);
            const uint32_t sc_lo = (r.h.y >> sh) & 63u;
            const uint32_t mn_lo = (r.h.z >> sh) & 63u;
            const uint32_t sc_hi = ((r.h.w >> sh) & 15u) | (((r.h.y >> (sh + 6)) & 3u) << 4);
            const uint32_t mn_hi = ((r.h.w >> (sh + 4)) & 15u) | (((r.h.z >> (sh + 6)) & 3u) << 4);
            const uint32_t sc = c < 2 ? sc_lo : sc_hi;
            const uint32_t mn = c < 2 ? mn_lo : mn_hi;
            const float s = d * static_cast<float>(sc);   // exact (fp16 x 6-bit)
            const float b = dmin * static_cast<float>(mn);
            // low nibbles enter as 1024 + q, high nibbles as 1024 + 16q
            const float ag = g == 0 ? s : s * 0.0625f;
            a[g] = valid ? ag : 0.0f;
            B[g] = valid ? __fmaf_rn(1024.0f, ag, b) : 0.0f;
        }
    }
};

// Q6_K: lane = (super-block sb = lane/4, half n = (lane/2)%2, column half h = lane%2): weights
// l = 16h..16h+15 of the four 32-wide groups t of half n: k = 256sb + 128n + 32t + 16h + (0..15).
// Groups: t = 0..3 (chunks 2t, 2t+1), one int8 sub-scale each.
struct GQ6K {
    static constexpr int kType = QMM_TYPE_Q6_K;
    static constexpr int kQK = kQK_K;
    static constexpr int kBlockBytes = kBytesQ6_K;
    static constexpr int kWinBytes = 16 * kBytesQ6_K;  // 3360
    static constexpr int kG = 4;
    static constexpr bool kAligned = false;
    static constexpr bool kStream = false;
    struct Raw {
        u32x4 la, lb, qh;
        uint32_t s0, s1, d;
    };
    __device__ static int xk(int lane, int cj) {
        const int sb = lane >> 2, n = (lane >> 1) & 1, h = lane & 1;
        return 256 * sb + 128 * n + 16 * h + 32 * (cj >> 1) + 8 * (cj & 1);
    }
    __device__ static bool group_valid(int lane, int, int kwin_valid) { return 256 * (lane >> 2) < kwin_valid; }
    __device__ static Raw load(const uint8_t* win, int lane, int kwin_valid) {
        const int sb = lane >> 2, n = (lane >> 1) & 1, h = lane & 1;
        const bool v = 256 * sb < kwin_valid;
        const uint8_t* p = win + (v ? sb * kBytesQ6_K : 0);
        Raw r;
        r.la = ldg16(p + 64 * n + 16 * h);
        r.lb = ldg16(p + 64 * n + 32 + 16 * h);
        r.qh = ldg16(p + 128 + 32 * n + 16 * h);
        uint32_t s[2];
        __builtin_memcpy(s, p + 192 + 8 * n, 8);
        r.s0 = s[0];
        r.s1 = s[1];
        r.d = ldg_u16(p + 208);
        return r;
    }
    // Chunk cj: group t = cj/2 (q1..q4 of the reference), bytes 8*(cj&1) .. +7 of the slices.
    // Per dword of 4 codes: the 6-bit unsigned codes u = q + 32 are assembled byte-wise (low 4
    // bits from ql, the qh bit pair of group t masked in place), then v_perm makes the fp16
    // pairs (1024 + u) of bytes (0, 2) and (1, 3).
    __device__ static void chunk_codes(const Raw& r, int cj, const Consts& K, uint32_t out[4]) {
        const int t = cj >> 1;
        const bool second = (cj & 1) != 0;
        const u32x4& ql = (t & 1) ? r.lb : r.la;
        const uint32_t L[2] = {second ? ql.z : ql.x, second ? ql.w : ql.y};
        const uint32_t H[2] = {second ? r.qh.z : r.qh.x, second ? r.qh.w : r.qh.y};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t lo4 = (t < 2 ? L[i] : L[i] >> 4) & 0x0F0F0F0Fu;
            // bits 2t, 2t+1 of each qh byte -> bits 4, 5
            const uint32_t hs = t == 0 ? H[i] << 4 : t == 1 ? H[i] << 2 : t == 2 ? H[i] : H[i] >> 2;
            const uint32_t u = and_or(hs, 0x30303030u, lo4);
            out[2 * i] = __builtin_amdgcn_perm(K.mg, u, 0x07020500u);
            out[2 * i + 1] = __builtin_amdgcn_perm(K.mg, u, 0x07030501u);
        }
    }
    __device__ static void group_scales(const Raw& r, int lane, bool valid, float a[kG], float B[kG]) {
        const int h = lane & 1;
        const float d = half_bits_to_float(r.d);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            // sc[8n + h + 2t]: byte h + 2t of the half's 8 scale bytes (signed)
            const uint32_t w = t < 2 ? r.s0 : r.s1;
            const int sh = 8 * (h + 2 * (t & 1));
            const float s = d * static_cast<float>(static_cast<int8_t>(w >> sh));
            // codes q + 32 enter as 1024 + (q + 32)
            a[t] = valid ? s : 0.0f;
            B[t] = valid ? s * 1056.0f : 0.0f;
        }
    }
};

// Q8_0: lane = blocks 2*lane, 2*lane + 1 (64 weights, k = 64*lane + 0..63).  Groups: the blocks.
struct GQ80 {
    static constexpr int kType = QMM_TYPE_Q8_0;
    static constexpr int kQK = kQK8_0;
    static constexpr int kBlockBytes = kBytesQ8_0;
    static constexpr int kWinBytes = 128 * kBytesQ8_0;  // 4352
    static constexpr int kG = 2;
    static constexpr bool kAligned = false;
    static constexpr bool kStream = true;  // 34-byte blocks: the streamed window is 12 % faster
    struct Raw {
        u32x4 q[2][2];
        uint32_t d[2];
    };
    __device__ static int xk(int lane, int cj) { return 64 * lane + 8 * cj; }
    __device__ static bool group_valid(int lane, int g, int kwin_valid) { return 64 * lane + 32 * g < kwin_valid; }
    __device__ static Raw load(const uint8_t* win, int lane, int kwin_valid) {
        Raw r;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const bool v = 64 * lane + 32 * b < kwin_valid;
            const uint8_t* p = win + (v ? (2 * lane + b) * kBytesQ8_0 : 0);
            r.q[b][0] = ldg16(p + 2);
            r.q[b][1] = ldg16(p + 18);
            r.d[b] = ldg_u16(p);
        }
        return r;
    }
    __device__ static void chunk_codes(const Raw& r, int cj, const Consts& K, uint32_t out[4]) {
        const u32x4& q = r.q[cj >> 2][(cj >> 1) & 1];
        const bool second = (cj & 1) != 0;
        const uint32_t D[2] = {(second ? q.z : q.x) ^ 0x80808080u, (second ? q.w : q.y) ^ 0x80808080u};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            // [b0, 0x64, b2, 0x64] and [b1, 0x64, b3, 0x64]: 1024 + (q + 128)
            out[2 * i] = __builtin_amdgcn_perm(K.mg, D[i], 0x07020500u);
            out[2 * i + 1] = __builtin_amdgcn_perm(K.mg, D[i], 0x07030501u);
        }
    }
    __device__ static void group_scales(const Raw& r, int, bool, float a[kG], float B[kG]) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const float d = half_bits_to_float(r.d[g]);
            a[g] = d;
            B[g] = d * 1152.0f;
        }
    }
};

// Q4_0: lane = blocks 2*lane, 2*lane + 1.  Groups: block b low nibbles (k 32b + 0..15, chunks
// 4b, 4b+1) and high nibbles (k 32b + 16..31, chunks 4b+2, 4b+3).
struct GQ40 {
    static constexpr int kType = QMM_TYPE_Q4_0;
    static constexpr int kQK = kQK4_0;
    static constexpr int kBlockBytes = kBytesQ4_0;
    static constexpr int kWinBytes = 128 * kBytesQ4_0;  // 2304
    static constexpr int kG = 4;
    static constexpr bool kAligned = false;
    static constexpr bool kStream = false;
    struct Raw {
        u32x4 q[2];
        uint32_t d[2];
    };
    __device__ static int xk(int lane, int cj) { return 64 * lane + 8 * cj; }
    __device__ static bool group_valid(int lane, int g, int kwin_valid) { return 64 * lane + 32 * (g >> 1) < kwin_valid; }
    __device__ static Raw load(const uint8_t* win, int lane, int kwin_valid) {
        Raw r;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const bool v = 64 * lane + 32 * b < kwin_valid;
            const uint8_t* p = win + (v ? (2 * lane + b) * kBytesQ4_0 : 0);
            r.q[b] = ldg16(p + 2);
            r.d[b] = ldg_u16(p);
        }
        return r;
    }
    __device__ static void chunk_codes(const Raw& r, int cj, const Consts& K, uint32_t out[4]) {
        const u32x4& q = r.q[cj >> 2];
        const bool second = (cj & 1) != 0;   // qs bytes 8..15 of the block
        const uint32_t dlo = second ? q.z : q.x;
        const uint32_t dhi = second ? q.w : q.y;
        const uint32_t m = (cj & 2) ? K.mf0 : K.m0f;
        out[0] = and_or(dlo, m, K.mg);
        out[1] = and_or(dlo >> 8, m, K.mg);
        out[2] = and_or(dhi, m, K.mg);
        out[3] = and_or(dhi >> 8, m, K.mg);
    }
    __device__ static void group_scales(const Raw& r, int, bool, float a[kG], float B[kG]) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float d = half_bits_to_float(r.d[g >> 1]);
            if (g & 1) {           // high nibbles: 1024 + 16q, w = d (q - 8)
                a[g] = d * 0.0625f;
                B[g] = d * 72.0f;  // (1024/16 + 8) d
            } else {               // low nibbles: 1024 + q
                a[g] = d;
                B[g] = d * 1032.0f;
            }
        }
    }
};

// F16 (dense fp16 rows, the operand of the reference's matmul_nt): lane slot = 64 consecutive
// weights, eight 16-byte loads.  No scales: the dot products are the result (mac_window takes
// the dense branch).  Needs K % 16 == 0, so that a 16-value activation staging item and a
// 16-byte weight chunk are either wholly inside K or wholly outside it; chunks outside read
// the window's first bytes (a valid address) and meet zero activations.
struct GF16 {
    static constexpr int kType = QMM_TYPE_F16;
    static constexpr int kQK = 8;                      // row bytes = K / 8 * 16 = 2K
    static constexpr int kBlockBytes = 16;
    static constexpr int kWinBytes = 2 * kGemvWindow;  // 8192
    static constexpr int kG = 1;
    static constexpr bool kAligned = false;
    static constexpr bool kStream = true;
    struct Raw {
        u32x4 w[kChunks];
    };
    __device__ static int xk(int lane, int cj) { return 64 * lane + 8 * cj; }
    __device__ static bool group_valid(int lane, int, int kwin_valid) { return 64 * lane < kwin_valid; }
    __device__ static Raw load(const uint8_t* win, int lane, int kwin_valid) {
        Raw r;
#pragma unroll
        for (int c = 0; c < kChunks; ++c) {
            const int k = 64 * lane + 8 * c;
            r.w[c] = ldg16(win + (k < kwin_valid ? 2 * k : 0));
        }
        return r;
    }
    // dwords (w0,w1), (w2,w3), (w4,w5), (w6,w7) -> pairs (w0,w2), (w1,w3), (w4,w6), (w5,w7), the
    // order of the staged activation pairs
    __device__ static void chunk_codes(const Raw& r, int cj, const Consts&, uint32_t out[4]) {
        const u32x4& d = r.w[cj];
        out[0] = __builtin_amdgcn_perm(d.y, d.x, 0x05040100u);
        out[1] = __builtin_amdgcn_perm(d.y, d.x, 0x07060302u);
        out[2] = __builtin_amdgcn_perm(d.w, d.z, 0x05040100u);
        out[3] = __builtin_amdgcn_perm(d.w, d.z, 0x07060302u);
    }
    __device__ static void group_scales(const Raw&, int, bool, float a[kG], float B[kG]) {
        a[0] = 1.0f;
        B[0] = 0.0f;
    }
};

// ------------------------------------------------------------------------------------------
// Activation staging: chunk cj of lane l holds fp16 pairs (x0,x2), (x1,x3), (x4,x6), (x5,x7)
// of the 8 activations at window k = F::xk(l, cj); xsum[l][q] = sum of the 16 fp16 values of
// chunks 2q and 2q+1 (fp32, fixed order).
// ------------------------------------------------------------------------------------------
template <typename TA>
__device__ __forceinline__ void load16_act(const TA* p, bool ok, bool vec, uint32_t h[8], int sh, float& amax);

// The loads are issued whether or not the activations exist (p is always a valid address);
// missing ones (`ok` false) are replaced by zeros afterwards.  fp32 values are multiplied by 2^sh
// (0 unless the window is rescaled) before the f16 rounding; `amax` receives the largest magnitude
// of the 16 unscaled values.
template <>
__device__ __forceinline__ void load16_act<float>(const float* p, bool ok, bool vec, uint32_t h[8], int sh, float& amax) {
    float x[16];
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
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        x[i] = ok ? x[i] : 0.0f;
        mx = fmaxf(mx, fabsf(x[i]));
        x[i] = __builtin_ldexpf(x[i], sh);
    }
    amax = mx;
    // pairs (0,2), (1,3), (4,6), (5,7), ... rounded to nearest even (v_cvt_pk_f16_f32)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b = 8 * c + 4 * (i >> 1) + (i & 1);
            h16x2 v = {static_cast<_Float16>(x[b]), static_cast<_Float16>(x[b + 2])};
            __builtin_memcpy(&h[4 * c + i], &v, 4);
        }
    }
}

template <>
__device__ __forceinline__ void load16_act<__half>(const __half* p, bool ok, bool vec, uint32_t h[8], int, float& amax) {
    amax = 0.0f;
    uint32_t w[8];
    if (vec) {
        const uint4 a = reinterpret_cast<const uint4*>(p)[0];
        const uint4 b = reinterpret_cast<const uint4*>(p)[1];
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
    } else {
        const uint16_t* s = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = s[2 * i] | (static_cast<uint32_t>(s[2 * i + 1]) << 16);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = ok ? w[i] : 0u;
    // dwords (x0,x1), (x2,x3) -> (x0,x2), (x1,x3)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        h[2 * c] = __builtin_amdgcn_perm(w[2 * c + 1], w[2 * c], 0x05040100u);
        h[2 * c + 1] = __builtin_amdgcn_perm(w[2 * c + 1], w[2 * c], 0x07060302u);
    }
}

// LDS layout shared by both kernels, in u32x4 entries of the dynamic LDS array:
//   x  [slot][m][chunk][lane]  (4 fp16 pairs each)   slot = staged window
//   sx [slot][m][lane]         (float4: the 4 partial sums of the lane's 16-k pieces)
extern __shared__ u32x4 gemv_lds[];

__device__ __forceinline__ int x_index(int slot, int m, int MR, int cj, int lane) { return ((slot * MR + m) * kChunks + cj) * 64 + lane; }
__device__ __forceinline__ int sx_index(int nslots, int slot, int m, int MR, int lane) {
    return nslots * MR * kChunks * 64 + (slot * MR + m) * 64 + lane;
}

// Stages activation item idx of window w into LDS slot `slot`: item = (m, q, lane) covers the 16
// activations of chunks 2q, 2q+1 of the lane's slot.
template <class F, int MR, typename TA>
struct StageItem {
    uint32_t h[8];
    float amax;  // largest unscaled magnitude of the item (fp32 activations)
    __device__ __forceinline__ void load(const TA* __restrict__ A, int M, int K, int m0, int w, int item, bool vec,
                                         int sh = 0) {
        const int m = item >> 8, q = (item >> 6) & 3, lane = item & 63;
        const int k = w * kGemvWindow + F::xk(lane, 2 * q);
        const bool ok = m0 + m < M && k < K;
        const TA* p = A + static_cast<size_t>(ok ? m0 + m : 0) * K + (ok ? k : 0);
        load16_act<TA>(p, ok, vec, h, sh, amax);
    }
    __device__ __forceinline__ void store(int nslots, int slot, int item) const {
        const int m = item >> 8, q = (item >> 6) & 3, lane = item & 63;
        gemv_lds[x_index(slot, m, MR, 2 * q, lane)] = u32x4{h[0], h[1], h[2], h[3]};
        gemv_lds[x_index(slot, m, MR, 2 * q + 1, lane)] = u32x4{h[4], h[5], h[6], h[7]};
        const uint32_t ones = 0x3C003C00u;  // fp16 (1, 1)
        float t = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) t = dot2(h[j], ones, t);
        reinterpret_cast<float*>(&gemv_lds[sx_index(nslots, slot, m, MR, lane)])[q] = t;
    }
    // fp32 activations: the item's magnitude joins its (window, row) maximum (non-negative floats
    // order like their bit patterns).
    __device__ __forceinline__ void note_max(uint32_t* wmax) const {
        if constexpr (std::is_same<TA, float>::value) atomicMax(wmax, __float_as_uint(amax));
    }
};

// Range of fp32 activations.  f16 holds magnitudes from 2^-14 (normal) to 65504; a window (4096 k)
// of one activation row whose largest magnitude lies outside that range (at or above 65504, or in
// [2^-126, 2^-14)) is staged as x * 2^-e with e = exponent(max) - 14, which brings the maximum into
// [2^14, 2^15), and each group's net contribution (scale times dot sum minus offset times
// activation sum, formed first: its two terms can leave the fp32 range where their difference
// does not) is multiplied by 2^e.  These scalings are exact while their results are normal fp32
// numbers.  Every other window has e = 0 and is staged and multiplied exactly as fp16 activations
// are.  Infinite or NaN maxima keep e = 0 (they propagate as in fp32 arithmetic), and so do maxima
// below 2^-126 (their values round to zero in f16).  The exponent depends only on the window's own
// values, so a row's result does not depend on M.
__device__ __forceinline__ int window_exp(uint32_t maxbits) {
    const bool big = maxbits >= 0x477FE000u && maxbits < 0x7F800000u;  // [65504, inf)
    const bool tiny = maxbits >= 0x00800000u && maxbits < 0x38800000u;  // [2^-126, 2^-14)
    return big || tiny ? static_cast<int>(maxbits >> 23) - 127 - 14 : 0;
}

// (window, row) maxima of fp32 activations, in LDS: nwin * MR entries for the kernels that stage
// every window at once (at most 17 fit the LDS), 3 * MR for the windowed kernel.
constexpr int kWmaxEntries = 32;
template <typename TA>
constexpr int wmax_size(int n) { return std::is_same<TA, float>::value ? n : 1; }

__device__ __forceinline__ void lds_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// e of activation row m in staged window `w` (0 for fp16 activations).
template <int MR, typename TA>
__device__ __forceinline__ void window_factors(const uint32_t* wmax_w, int (&pe)[MR]) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        if constexpr (std::is_same<TA, float>::value) pe[m] = window_exp(wmax_w[m]);
        else pe[m] = 0;
    }
}

// After all windows of fp32 activations are staged (and a barrier): re-stages each (window, row)
// whose maximum is outside the f16 range, scaled by its power of two.  The branch is uniform and
// rare; it ends with a barrier when taken.
template <class F, int MR, int NW, typename TA>
__device__ __forceinline__ void restage_out_of_range(const TA* __restrict__ A, const uint32_t* wmax, int M, int K, int m0,
                                                     int nwin, int tid, bool vec) {
    if constexpr (std::is_same<TA, float>::value) {
        bool need = false;
        for (int i = 0; i < nwin * MR; ++i) need = need || window_exp(wmax[i]) != 0;
        if (!need) return;
        const int items = nwin * MR * 256;
        for (int it = tid; it < items; it += 64 * NW) {
            const int w = it / (MR * 256), item = it - w * (MR * 256);
            const int e = window_exp(wmax[w * MR + (item >> 8)]);
            if (e != 0) {
                StageItem<F, MR, TA> s2;
                s2.load(A, M, K, m0, w, item, vec, -e);
                s2.store(nwin, w, item);
            }
        }
        __syncthreads();
    }
}

template <typename TC>
__device__ __forceinline__ void store_out(TC* p, float v);
template <>
__device__ __forceinline__ void store_out<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_out<__half>(__half* p, float v) {
    *reinterpret_cast<uint16_t*>(p) = float_to_half_bits(v);
}

// acc[m][y] += the window's contribution of row y for activation row m.
// FULL: every lane slot of the window is inside K (no validity masks).
// SC: fp32 activations; pe[m] = e of activation row m in this window (0 unless rescaled).
template <class F, int MR, int YT, bool FULL, bool SC = false>
__device__ __forceinline__ void mac_window(const typename F::Raw (&cur)[YT], int nslots, int slot, int lane, int kv,
                                           const Consts& KC, float (&acc)[MR][YT], const int (&pe)[MR]) {
    if constexpr (F::kType == QMM_TYPE_F16) {
        // dense weights: no group scales; activations outside K are staged as zeros.  A rescaled
        // window (pe != 0) is summed on its own and added as 2^e * sum.
        float s0[MR][YT];
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int y = 0; y < YT; ++y) s0[m][y] = !SC || pe[m] == 0 ? acc[m][y] : 0.0f;
#pragma unroll
        for (int cj = 0; cj < kChunks; ++cj) {
            u32x4 xp[MR];
#pragma unroll
            for (int m = 0; m < MR; ++m) xp[m] = gemv_lds[x_index(slot, m, MR, cj, lane)];
#pragma unroll
            for (int y = 0; y < YT; ++y) {
                uint32_t w[4];
                F::chunk_codes(cur[y], cj, KC, w);
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    float s = s0[m][y];
                    s = dot2(xp[m].x, w[0], s);
                    s = dot2(xp[m].y, w[1], s);
                    s = dot2(xp[m].z, w[2], s);
                    s = dot2(xp[m].w, w[3], s);
                    s0[m][y] = s;
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int y = 0; y < YT; ++y) acc[m][y] = !SC || pe[m] == 0 ? s0[m][y] : acc[m][y] + __builtin_ldexpf(s0[m][y], pe[m]);
        return;
    }
    constexpr int G = F::kG;
    constexpr int CPG = kChunks / G;  // chunks per group
    float a[YT][G], B[YT][G];
#pragma unroll
    for (int y = 0; y < YT; ++y) {
        F::group_scales(cur[y], lane, true, a[y], B[y]);
        if constexpr (!FULL) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const bool v = F::group_valid(lane, g, kv);
                a[y][g] = v ? a[y][g] : 0.0f;
                B[y][g] = v ? B[y][g] : 0.0f;
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float S[MR][YT];
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int y = 0; y < YT; ++y) S[m][y] = 0.0f;
#pragma unroll
        for (int cc = 0; cc < CPG; ++cc) {
            const int cj = g * CPG + cc;
            u32x4 xp[MR];
#pragma unroll
            for (int m = 0; m < MR; ++m) xp[m] = gemv_lds[x_index(slot, m, MR, cj, lane)];
#pragma unroll
            for (int y = 0; y < YT; ++y) {
                uint32_t code[4];
                F::chunk_codes(cur[y], cj, KC, code);
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    // the group's first product starts from 0 (same value as 0 + product)
                    float s = cc == 0 ? dot2_z(xp[m].x, code[0]) : dot2(xp[m].x, code[0], S[m][y]);
                    s = dot2(xp[m].y, code[1], s);
                    s = dot2(xp[m].z, code[2], s);
                    s = dot2(xp[m].w, code[3], s);
                    S[m][y] = s;
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const u32x4 sv = gemv_lds[sx_index(nslots, slot, m, MR, lane)];
            float sq[4];
            __builtin_memcpy(sq, &sv, 16);
            float sxg;
            if constexpr (G == 2) sxg = sq[2 * g] + sq[2 * g + 1];
            else sxg = sq[g];
#pragma unroll
            for (int y = 0; y < YT; ++y) {
                float t = acc[m][y];
                if (SC && pe[m] != 0) {  // rescaled window: the group's net, then times 2^e
                    const float net = __fmaf_rn(a[y][g], S[m][y], -(B[y][g] * sxg));
                    t += __builtin_ldexpf(net, pe[m]);
                } else {
                    t = __fmaf_rn(a[y][g], S[m][y], t);
                    t = __fmaf_rn(-B[y][g], sxg, t);
                }
                acc[m][y] = t;
            }
        }
    }
}

// Staging with a prologue (GemvFuse kind 1 or 2; one fp16 activation row): every load of the
// thread's items (16 consecutive activations each, at most kFuseOwn) is issued first (A, R and
// the norm weights, 16-byte vectors), then v is formed, v^2 is reduced over the workgroup for the
// norm kinds, and the staged fp16 pairs and sums are written as StageItem::store does.
constexpr int kFuseOwn = 2;
// The folded staging exists for one fp16 activation row (decode) and where its registers fit
// beside the kernel's own (1024-thread workgroups have 128 per lane: one row per item there,
// and not for F16); other instantiations keep their register budget.
template <class F, int MR, int YT, int NW, typename TA>
constexpr bool kFoldable = MR == 1 && std::is_same<TA, __half>::value && (NW <= 8 || (YT == 1 && F::kType != QMM_TYPE_F16));
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));

template <class F, int MR, int NW>
__device__ __forceinline__ void stage_fused(const __half* A, const GemvFuse& fz, int M, int K, int m0, int nwin, int tid) {
    static_assert(MR == 1, "one activation row");
    __shared__ float red[NW];
    const int items = nwin * 256;
    const _Float16* a16 = reinterpret_cast<const _Float16*>(A) + static_cast<size_t>(m0) * K;
    const _Float16* r16 = static_cast<const _Float16*>(fz.R) + static_cast<size_t>(m0) * K;
    const bool two = fz.kind == 2;
    h16x8 av[kFuseOwn][2], rv[kFuseOwn][2], wv[kFuseOwn][2];
    int kk[kFuseOwn];
#pragma unroll
    for (int j = 0; j < kFuseOwn; ++j) {
        const int it = min(tid + 64 * NW * j, items - 1);
        const int w = it >> 8, q = (it >> 6) & 3, ln = it & 63;
        const int k = w * kGemvWindow + F::xk(ln, 2 * q);
        kk[j] = k;
        const int off = m0 < M && k < K ? k : 0;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            av[j][hh] = *reinterpret_cast<const h16x8*>(a16 + off + 8 * hh);
            if (two) rv[j][hh] = *reinterpret_cast<const h16x8*>(r16 + off + 8 * hh);
            {
                if (fz.w_f32) {  // an F32 norm weight is rounded to f16 first, as the reference's host does
                    const float* wf = static_cast<const float*>(fz.w) + off + 8 * hh;
                    const float4 lo = *reinterpret_cast<const float4*>(wf), hi = *reinterpret_cast<const float4*>(wf + 4);
                    wv[j][hh] = h16x8{static_cast<_Float16>(lo.x), static_cast<_Float16>(lo.y), static_cast<_Float16>(lo.z),
                                      static_cast<_Float16>(lo.w), static_cast<_Float16>(hi.x), static_cast<_Float16>(hi.y),
                                      static_cast<_Float16>(hi.z), static_cast<_Float16>(hi.w)};
                } else {
                    wv[j][hh] = *reinterpret_cast<const h16x8*>(static_cast<const _Float16*>(fz.w) + off + 8 * hh);
                }
            }
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < kFuseOwn; ++j) {
        const bool ok = tid + 64 * NW * j < items && m0 < M && kk[j] < K;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            h16x8 v = av[j][hh];
            if (two) {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    v[e] = static_cast<_Float16>(static_cast<float>(v[e]) + static_cast<float>(rv[j][hh][e]));
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                v[e] = ok ? v[e] : static_cast<_Float16>(0.0f);
                const float f = static_cast<float>(v[e]);
                ss += f * f;
            }
            av[j][hh] = v;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < NW; ++i) t += red[i];
    const float scale = rsqrtf(t / static_cast<float>(K) + fz.eps);
#pragma unroll
    for (int j = 0; j < kFuseOwn; ++j) {
        const int it = tid + 64 * NW * j;
        if (it < items) {
            uint32_t wd[8];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                h16x8 v = av[j][hh];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    v[e] = static_cast<_Float16>(static_cast<float>(v[e]) * scale * static_cast<float>(wv[j][hh][e]));
                __builtin_memcpy(&wd[4 * hh], &v, 16);
            }
            StageItem<F, MR, __half> st;
            // dwords (x0,x1), (x2,x3) -> (x0,x2), (x1,x3), the staged pair order
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                st.h[2 * c] = __builtin_amdgcn_perm(wd[2 * c + 1], wd[2 * c], 0x05040100u);
                st.h[2 * c + 1] = __builtin_amdgcn_perm(wd[2 * c + 1], wd[2 * c], 0x07060302u);
            }
            st.store(nwin, it >> 8, it & 255);
        }
    }
}

template <int MR, int YT, typename TC>
__device__ __forceinline__ void reduce_store(float (&acc)[MR][YT], TC* __restrict__ C, int M, int N, int m0, int row0,
                                             int lane, const GemvFuse& fz) {
    float v[MR][YT];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int y = 0; y < YT; ++y) v[m][y] = wave_sum_to_lane63(acc[m][y]);
    if constexpr (YT == 2 && sizeof(TC) == 2) {
        if (fz.pair) {  // row0 is the row of both matrices: C[row0] = half(silu(half(gate)) * half(up))
            if (lane == 63) {
#pragma unroll
                for (int m = 0; m < MR; ++m)
                    if (m0 + m < M && row0 < N) {
                        const float g = static_cast<float>(static_cast<_Float16>(v[m][0]));
                        const float u = static_cast<float>(static_cast<_Float16>(v[m][1]));
                        store_out<TC>(C + static_cast<size_t>(m0 + m) * N + row0, g / (1.0f + expf(-g)) * u);
                    }
            }
            return;
        }
    }
    if (lane == 63) {
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int y = 0; y < YT; ++y)
                if (m0 + m < M && row0 + y < N) {
                    const size_t o = static_cast<size_t>(m0 + m) * N + row0 + y;
                    float r = v[m][y];
                    if constexpr (sizeof(TC) == 2) {
                        if (fz.ea != nullptr) {  // residual: half(half(ea + eb) + half(acc))
                            const float h = static_cast<float>(static_cast<_Float16>(
                                static_cast<float>(static_cast<const _Float16*>(fz.ea)[o]) +
                                static_cast<float>(static_cast<const _Float16*>(fz.eb)[o])));
                            r = h + static_cast<float>(static_cast<_Float16>(r));
                        }
                    }
                    store_out<TC>(C + o, r);
                }
    }
}

// Weight matrices multiplied by the same activations in one launch (e.g. the q, k and v
// projections): their row groups are concatenated; segment s owns row groups
// [gend[s-1], gend[s]).  Unused entries have gend = INT_MAX.
constexpr int kMaxSegs = 4;
template <typename TC>
struct GemvSegs {
    const uint8_t* W[kMaxSegs];
    TC* C[kMaxSegs];
    int N[kMaxSegs];
    int gend[kMaxSegs];
};

// Segment of row group g (wave-uniform): its weights, output, rows and first row group.
template <typename TC>
struct SegRef {
    const uint8_t* W;
    TC* C;
    int N, g0;
};
template <typename TC>
__device__ __forceinline__ SegRef<TC> seg_of(const GemvSegs<TC>& sg, int g) {
    SegRef<TC> r{sg.W[0], sg.C[0], sg.N[0], 0};
#pragma unroll
    for (int j = 1; j < kMaxSegs; ++j) {
        if (g >= sg.gend[j - 1]) r = SegRef<TC>{sg.W[j], sg.C[j], sg.N[j], sg.gend[j - 1]};
    }
    return r;
}

// Resident-activation kernel: the workgroup stages all windows of its MR activation rows once,
// then every wave streams (row group, window) items (YT rows each) round-robin over the grid.
// One register buffer per item: an item's weight loads are issued as soon as the previous item
// has been multiplied (the occupancy of several waves per SIMD covers their latency).  Row and
// window arithmetic is wave-uniform (scalar).  No barrier after staging.
// Dynamic LDS: MR * nwin * 9216 bytes.
template <class F, int MR, int YT, int NW, typename TA, typename TC>
__global__ __launch_bounds__(64 * NW)
void gemv_resident_kernel(const TA* __restrict__ A, GemvSegs<TC> sg, int M, int K, int a_vec, int nrg, GemvFuse fz) {
    constexpr bool kF32 = std::is_same<TA, float>::value;
    __shared__ uint32_t wmax[wmax_size<TA>(kWmaxEntries)];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m0 = blockIdx.y * MR;
    const bool vec = a_vec != 0;
    const size_t row_bytes = static_cast<size_t>(K / F::kQK) * F::kBlockBytes;
    const int nwin = (K + kGemvWindow - 1) / kGemvWindow;
    const int stride = gridDim.x * NW;
    const Consts KC = make_consts();

    typedef typename F::Raw Raw;
    auto load_item = [&](int g, int w, Raw (&r)[YT]) {
        g = min(g, nrg - 1);  // a prefetch past the wave's last item re-reads a valid row group
        const SegRef<TC> sr = seg_of(sg, g);
        const int kv = min(K - w * kGemvWindow, kGemvWindow);
        const uint8_t* base = sr.W + static_cast<size_t>(w) * F::kWinBytes;
#pragma unroll
        for (int y = 0; y < YT; ++y) {
            // paired rows: y = 0 from the first matrix, y = 1 from the second, both row g
            const uint8_t* rp = fz.pair ? (y == 0 ? sg.W[0] : sg.W[1]) + static_cast<size_t>(w) * F::kWinBytes +
                                              static_cast<size_t>(min(g, sr.N - 1)) * row_bytes
                                        : base + static_cast<size_t>(min((g - sr.g0) * YT + y, sr.N - 1)) * row_bytes;
            r[y] = F::load(rp, lane, kv);
        }
    };
    auto next = [&](int& g, int& w) {
        if (++w == nwin) {
            w = 0;
            g += stride;
        }
    };

    // Item iterators: (gc, wc) is the next item to multiply, (gl, wl) the next to load.
    int gc = blockIdx.x * NW + wv, wc = 0;
    int gl = gc, wl = 0;
    const bool active = gc < nrg;

    // Staging order: this thread's first activation loads, then three items of weight bytes,
    // then the LDS writes; the weight loads stay in flight through the barrier.
    constexpr int kFirst = 2;  // activation items per thread issued before the weight loads
    const int items = nwin * MR * 256;
    Raw b0[YT];
    bool fused = false;
    if constexpr (kFoldable<F, MR, YT, NW, TA>) fused = fz.kind != 0;
    if (fused) {
        // weight bytes first, then the activations with their prologue
        load_item(gl, wl, b0); next(gl, wl);
        if constexpr (kFoldable<F, MR, YT, NW, TA>) stage_fused<F, MR, NW>(A, fz, M, K, m0, nwin, tid);
    } else {
        if constexpr (kF32) {
            if (tid < nwin * MR) wmax[tid] = 0u;
        }
        StageItem<F, MR, TA> st[kFirst];
#pragma unroll
        for (int j = 0; j < kFirst; ++j) {
            const int it = min(tid + 64 * NW * j, items - 1);  // loads always issued (static counts)
            const int w = it / (MR * 256);
            st[j].load(A, M, K, m0, w, it - w * (MR * 256), vec);
        }
        // issued by every wave (inactive waves re-read a valid row group) to keep counts static
        load_item(gl, wl, b0); next(gl, wl);
        if constexpr (kF32) lds_barrier();  // the maxima are cleared before any item joins them
#pragma unroll
        for (int j = 0; j < kFirst; ++j) {
            const int it = tid + 64 * NW * j;
            if (it < items) {
                const int w = it / (MR * 256), item = it - w * (MR * 256);
                st[j].store(nwin, w, item);
                st[j].note_max(&wmax[w * MR + (item >> 8)]);
            }
        }
        for (int it = tid + 64 * NW * kFirst; it < items; it += 64 * NW) {
            const int w = it / (MR * 256), item = it - w * (MR * 256);
            StageItem<F, MR, TA> s2;
            s2.load(A, M, K, m0, w, item, vec);
            s2.store(nwin, w, item);
            s2.note_max(&wmax[w * MR + (item >> 8)]);
        }
    }
    __syncthreads();
    restage_out_of_range<F, MR, NW, TA>(A, wmax, M, K, m0, nwin, tid, vec);
    if (!active) return;

    float acc[MR][YT];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int y = 0; y < YT; ++y) acc[m][y] = 0.0f;

    auto compute = [&](const Raw (&b)[YT]) {
        const int kv = min(K - wc * kGemvWindow, kGemvWindow);
        int pe[MR];
        window_factors<MR, TA>(&wmax[kF32 ? wc * MR : 0], pe);
        if (kv == kGemvWindow) mac_window<F, MR, YT, true, kF32>(b, nwin, wc, lane, kv, KC, acc, pe);
        else mac_window<F, MR, YT, false, kF32>(b, nwin, wc, lane, kv, KC, acc, pe);
        if (wc == nwin - 1) {
            const SegRef<TC> sr = seg_of(sg, gc);
            reduce_store<MR, YT, TC>(acc, sr.C, M, sr.N, m0, fz.pair ? gc : (gc - sr.g0) * YT, lane, fz);
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int y = 0; y < YT; ++y) acc[m][y] = 0.0f;
        }
        next(gc, wc);
    };

    // The next item's loads are issued right after an item's multiply (past the wave's last
    // item: a valid row group re-read).
    const int total = ((nrg - gc + stride - 1) / stride) * nwin;
    for (int i = 0;;) {
        compute(b0);
        if (++i == total) break;
        load_item(gl, wl, b0); next(gl, wl);
    }
}

// Streamed-window variant of the resident kernel: a wave copies each item's packed window
// (kWinBytes contiguous bytes of a row) into a private LDS slot with direct-to-LDS 16-byte
// loads, lanes on consecutive pieces, so every load instruction reads 1 KiB of contiguous
// memory; the lane slots are then read from LDS and multiplied exactly as in the resident kernel
// (same arithmetic, same order: results are bit-identical).  NS slots per wave: NS - 1 items are
// in flight while one is multiplied.  Needs 16-byte aligned weights and row sizes.
// Dynamic LDS: the resident kernel's activations, then NW * NS * YT window slots.
template <class F>
struct WinSlot {
    static constexpr int kPieces = (F::kWinBytes + 15) / 16;  // 16-byte pieces of a window
    static constexpr int kInstr = (kPieces + 63) / 64;        // load instructions per window row
    static constexpr int kBytes = kPieces * 16;
};

// 16 bytes at global address g -> LDS at m0 + 16 * lane (m0 = the wave-uniform `lds`, an operand
// that the compiler moves into m0).  The compiler does not track these loads: the caller waits for
// them with an explicit vmcnt.
__device__ __forceinline__ void win_direct_load16(const void* g, const void* lds) {
    const uint32_t la = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
    __asm__ volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(la) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <class F, int MR, int YT, int NW, int NS, typename TA, typename TC>
__global__ __launch_bounds__(64 * NW)
void gemv_stream_kernel(const TA* __restrict__ A, GemvSegs<TC> sg, int M, int K, int a_vec, int nrg, GemvFuse fz) {
    using WS = WinSlot<F>;
    constexpr bool kF32 = std::is_same<TA, float>::value;
    __shared__ uint32_t wmax[wmax_size<TA>(kWmaxEntries)];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m0 = blockIdx.y * MR;
    const bool vec = a_vec != 0;
    const size_t row_bytes = static_cast<size_t>(K / F::kQK) * F::kBlockBytes;
    const int nwin = (K + kGemvWindow - 1) / kGemvWindow;
    const int stride = gridDim.x * NW;
    const Consts KC = make_consts();
    const int act_u4 = nwin * MR * (kChunks * 64 + 64);  // activation entries (x and sx) of the LDS
    uint8_t* wslots = reinterpret_cast<uint8_t*>(gemv_lds + act_u4) + static_cast<size_t>(wv) * NS * YT * WS::kBytes;

    // Copies item (g, w) into slot s: YT windows of WS::kPieces pieces (past the wave's last item:
    // a valid row group is re-read, so every wave issues the same number of loads).
    auto issue = [&](int g, int w, int slot) {
        g = min(g, nrg - 1);
        const SegRef<TC> sr = seg_of(sg, g);
        const size_t woff = static_cast<size_t>(w) * F::kWinBytes;
        const int valid = static_cast<int>(min(static_cast<size_t>(F::kWinBytes), row_bytes - woff));
#pragma unroll
        for (int y = 0; y < YT; ++y) {
            const uint8_t* rp = fz.pair ? (y == 0 ? sg.W[0] : sg.W[1]) + static_cast<size_t>(min(g, sr.N - 1)) * row_bytes + woff
                                        : sr.W + static_cast<size_t>(min((g - sr.g0) * YT + y, sr.N - 1)) * row_bytes + woff;
            uint8_t* dst = wslots + (slot * YT + y) * WS::kBytes;
#pragma unroll
            for (int i = 0; i < WS::kInstr; ++i) {
                const int piece = 64 * i + lane;
                const int off = 16 * piece < valid ? 16 * piece : 0;
                if (piece < WS::kPieces) win_direct_load16(rp + off, dst + 1024 * i);
            }
        }
    };
    auto next = [&](int& g, int& w) {
        if (++w == nwin) {
            w = 0;
            g += stride;
        }
    };

    int gc = blockIdx.x * NW + wv, wc = 0;
    int gl = gc, wl = 0;
    const bool active = gc < nrg;

    // the first NS - 1 items are requested before the activations are staged
#pragma unroll
    for (int j = 0; j < NS - 1; ++j) {
        issue(gl, wl, j);
        next(gl, wl);
    }
    const int items = nwin * MR * 256;
    bool fused = false;
    if constexpr (kFoldable<F, MR, YT, NW, TA>) fused = fz.kind != 0;
    if (fused) {
        if constexpr (kFoldable<F, MR, YT, NW, TA>) stage_fused<F, MR, NW>(A, fz, M, K, m0, nwin, tid);
    } else {
        if constexpr (kF32) {
            if (tid < nwin * MR) wmax[tid] = 0u;
            lds_barrier();  // the maxima are cleared before any item joins them
        }
        for (int it = tid; it < items; it += 64 * NW) {
            const int w = it / (MR * 256), item = it - w * (MR * 256);
            StageItem<F, MR, TA> s2;
            s2.load(A, M, K, m0, w, item, vec);
            s2.store(nwin, w, item);
            s2.note_max(&wmax[w * MR + (item >> 8)]);
        }
    }
    __syncthreads();
    restage_out_of_range<F, MR, NW, TA>(A, wmax, M, K, m0, nwin, tid, vec);
    if (!active) {
        wait_vmcnt<0>();  // no LDS DMA outstanding when the wave ends
        return;
    }

    float acc[MR][YT];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int y = 0; y < YT; ++y) acc[m][y] = 0.0f;

    typedef typename F::Raw Raw;
    const int total = ((nrg - gc + stride - 1) / stride) * nwin;
    int slot = 0;
    for (int i = 0; i < total; ++i) {
        // request item i + NS - 1 into the slot item i - 1 used (its LDS reads are complete: their
        // values were consumed), then wait until item i's copies have landed
        issue(gl, wl, (slot + NS - 1) % NS);
        next(gl, wl);
        wait_vmcnt<(NS - 1) * YT * WS::kInstr>();
        const int kv = min(K - wc * kGemvWindow, kGemvWindow);
        Raw b[YT];
#pragma unroll
        for (int y = 0; y < YT; ++y) b[y] = F::load(wslots + (slot * YT + y) * WS::kBytes, lane, kv);
        int pe[MR];
        window_factors<MR, TA>(&wmax[kF32 ? wc * MR : 0], pe);
        if (kv == kGemvWindow) mac_window<F, MR, YT, true, kF32>(b, nwin, wc, lane, kv, KC, acc, pe);
        else mac_window<F, MR, YT, false, kF32>(b, nwin, wc, lane, kv, KC, acc, pe);
        if (wc == nwin - 1) {
            const SegRef<TC> sr = seg_of(sg, gc);
            reduce_store<MR, YT, TC>(acc, sr.C, M, sr.N, m0, fz.pair ? gc : (gc - sr.g0) * YT, lane, fz);
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int y = 0; y < YT; ++y) acc[m][y] = 0.0f;
        }
        next(gc, wc);
        slot = slot + 1 == NS ? 0 : slot + 1;
    }
    wait_vmcnt<0>();  // the trailing copies land before the wave ends
}

// Windowed kernel (activations too large to keep resident): one workgroup owns NW * YT rows;
// window w + 1's activations are staged into the other of two LDS slots and its weight bytes
// loaded while window w is multiplied; one barrier per window.  Dynamic LDS: MR * 2 * 9216.
template <class F, int MR, int YT, int NW, typename TA, typename TC>
__global__ __launch_bounds__(64 * NW)
void gemv_window_kernel(const TA* __restrict__ A, const uint8_t* __restrict__ W, TC* __restrict__ C,
                        int M, int N, int K, int a_vec) {
    constexpr int kItems = MR * 256;
    constexpr int kPer = (kItems + 64 * NW - 1) / (64 * NW);
    constexpr bool kF32 = std::is_same<TA, float>::value;
    // fp32 activations: maxima of window w in wmax[w % 3]; entries of window w + 2 are cleared
    // while window w is multiplied (after every read of window w - 1's, before window w + 2 is
    // staged one barrier later).
    __shared__ uint32_t wmax[wmax_size<TA>(3 * MR)];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = tid >> 6;
    const int row0 = (blockIdx.x * NW + wv) * YT;
    const int m0 = blockIdx.y * MR;
    const bool vec = a_vec != 0;
    const size_t row_bytes = static_cast<size_t>(K / F::kQK) * F::kBlockBytes;
    const Consts KC = make_consts();

    // Rows past N are computed on the last valid row and never stored.
    const uint8_t* rowp[YT];
#pragma unroll
    for (int y = 0; y < YT; ++y) rowp[y] = W + static_cast<size_t>(min(row0 + y, N - 1)) * row_bytes;

    const int nwin = (K + kGemvWindow - 1) / kGemvWindow;
    float acc[MR][YT];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int y = 0; y < YT; ++y) acc[m][y] = 0.0f;

    StageItem<F, MR, TA> st[kPer];
    typename F::Raw cur[YT], nxt[YT];

    const int kv0 = min(K, kGemvWindow);
#pragma unroll
    for (int y = 0; y < YT; ++y) cur[y] = F::load(rowp[y], lane, kv0);
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (tid + 64 * NW * i < kItems) st[i].load(A, M, K, m0, 0, tid + 64 * NW * i, vec);
    if constexpr (kF32) {
        if (tid < 2 * MR) wmax[tid] = 0u;
        lds_barrier();
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (tid + 64 * NW * i < kItems) {
            st[i].store(2, 0, tid + 64 * NW * i);
            st[i].note_max(&wmax[(tid + 64 * NW * i) >> 8]);
        }
    __syncthreads();

    for (int w = 0; w < nwin; ++w) {
        const bool more = w + 1 < nwin;
        int pe[MR];
        if constexpr (kF32) {
            const uint32_t* wm = &wmax[(w % 3) * MR];
            bool need = false;
#pragma unroll
            for (int m = 0; m < MR; ++m) need = need || window_exp(wm[m]) != 0;
            if (need) {  // rare: re-stage window w with its rows' factors
#pragma unroll
                for (int i = 0; i < kPer; ++i) {
                    const int it = tid + 64 * NW * i;
                    const int e = it < kItems ? window_exp(wm[it >> 8]) : 0;
                    if (e != 0) {
                        StageItem<F, MR, TA> s2;
                        s2.load(A, M, K, m0, w, it, vec, -e);
                        s2.store(2, w & 1, it);
                    }
                }
                __syncthreads();
            }
            window_factors<MR, TA>(wm, pe);
            if (tid < MR) wmax[((w + 2) % 3) * MR + tid] = 0u;
        } else {
            window_factors<MR, TA>(wmax, pe);
        }
        {
            // unconditional weight prefetch (the last one re-reads window w)
            const int wn = more ? w + 1 : w;
            const int kv = min(K - wn * kGemvWindow, kGemvWindow);
            const size_t wo = static_cast<size_t>(wn) * F::kWinBytes;
#pragma unroll
            for (int y = 0; y < YT; ++y) nxt[y] = F::load(rowp[y] + wo, lane, kv);
        }
        if (more) {
#pragma unroll
            for (int i = 0; i < kPer; ++i)
                if (tid + 64 * NW * i < kItems) st[i].load(A, M, K, m0, w + 1, tid + 64 * NW * i, vec);
        }
        {
            const int kv = min(K - w * kGemvWindow, kGemvWindow);
            if (kv == kGemvWindow) mac_window<F, MR, YT, true, kF32>(cur, 2, w & 1, lane, kv, KC, acc, pe);
            else mac_window<F, MR, YT, false, kF32>(cur, 2, w & 1, lane, kv, KC, acc, pe);
        }
        if (more) {
#pragma unroll
            for (int i = 0; i < kPer; ++i)
                if (tid + 64 * NW * i < kItems) {
                    st[i].store(2, (w + 1) & 1, tid + 64 * NW * i);
                    st[i].note_max(&wmax[kF32 ? ((w + 1) % 3) * MR + ((tid + 64 * NW * i) >> 8) : 0]);
                }
        }
#pragma unroll
        for (int y = 0; y < YT; ++y) cur[y] = nxt[y];
        __syncthreads();
    }
    reduce_store<MR, YT, TC>(acc, C, M, N, m0, row0, lane, GemvFuse{});
}

// Alignment-agnostic fallback: one wave per (row n, A row m), lanes over 32-weight groups,
// byte loads, fp32 FMAs.  Used when W is not 2-byte aligned (16-byte for Q4_K) or A is not
// 4-byte aligned.
template <int T, typename TA, typename TC>
__global__ __launch_bounds__(256)
void gemv_fallback_kernel(const TA* __restrict__ A, const uint8_t* __restrict__ W, TC* __restrict__ C,
                          int M, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + threadIdx.x / 64;
    const int m = blockIdx.y;
    if (n >= N || m >= M) return;
    const TA* x = A + static_cast<size_t>(m) * K;
    float acc = 0.0f;
    if constexpr (T == QMM_TYPE_F16) {  // dense fp16 rows, any K
        const uint8_t* row = W + static_cast<size_t>(n) * K * 2;
        for (int k = lane; k < K; k += 64) {
            float xv;
            if constexpr (sizeof(TA) == 4) xv = x[k];
            else xv = __half2float(x[k]);
            acc = __fmaf_rn(xv, half_bits_to_float(row[2 * k] | (row[2 * k + 1] << 8)), acc);
        }
    } else {
        const int qk = (T == QMM_TYPE_Q4_0 || T == QMM_TYPE_Q8_0) ? 32 : 256;
        const int bb = T == QMM_TYPE_Q4_0 ? kBytesQ4_0 : T == QMM_TYPE_Q8_0 ? kBytesQ8_0
                     : T == QMM_TYPE_Q4_K ? kBytesQ4_K : kBytesQ6_K;
        const uint8_t* row = W + static_cast<size_t>(n) * (K / qk) * bb;
        const int groups = K / 32;
        for (int g = lane; g < groups; g += 64) {
            float w[32];
            group_weights_bytewise<T>(row, g, w);
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                float xv;
                if constexpr (sizeof(TA) == 4) xv = x[32 * g + i];
                else xv = __half2float(x[32 * g + i]);
                acc = __fmaf_rn(xv, w[i], acc);
            }
        }
    }
    acc = wave_sum_to_lane63(acc);
    if (lane == 63) store_out<TC>(C + static_cast<size_t>(m) * N + n, acc);
}

// Per-device facts and per-(kernel, LDS size) occupancy, cached (queried once; thread-safe).
struct DevInfo {
    int cus = 0;
    size_t max_lds = 0;
};

std::mutex g_info_mutex;

hipError_t device_info(DevInfo& out) {
    static std::unordered_map<int, DevInfo> cache;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(g_info_mutex);
    auto it = cache.find(dev);
    if (it != cache.end()) {
        out = it->second;
        return hipSuccess;
    }
    DevInfo d;
    int v = 0;
    if ((e = hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    d.cus = v;
    if ((e = hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev)) != hipSuccess) return e;
    d.max_lds = static_cast<size_t>(v);
    cache[dev] = d;
    out = d;
    return hipSuccess;
}

// Workgroups of `kern` that fit on one CU with `lds` bytes of dynamic LDS (at least 1).
hipError_t occupancy(const void* kern, int threads, size_t lds, int& blocks) {
    static std::unordered_map<std::string, int> cache;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const std::string key = std::to_string(dev) + ":" + std::to_string(reinterpret_cast<uintptr_t>(kern)) + ":" +
                            std::to_string(lds);
    std::lock_guard<std::mutex> lock(g_info_mutex);
    auto it = cache.find(key);
    if (it != cache.end()) {
        blocks = it->second;
        return hipSuccess;
    }
    if (lds > 65536) {
        // raised to the largest size the device allows beside the kernel's static LDS: the attribute
        // belongs to the kernel, and setting it to this call's size would lower it for a later, larger
        // call whose occupancy is already cached
        hipFuncAttributes fa;
        if ((e = hipFuncGetAttributes(&fa, kern)) != hipSuccess) return e;
        int mx = 0;
        if ((e = hipDeviceGetAttribute(&mx, hipDeviceAttributeMaxSharedMemoryPerBlock, dev)) != hipSuccess) return e;
        e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, mx - static_cast<int>(fa.sharedSizeBytes));
        if (e != hipSuccess) return e;
    }
    int n = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, threads, lds);
    if (e != hipSuccess) return e;
    blocks = n > 0 ? n : 1;
    cache[key] = blocks;
    return hipSuccess;
}

constexpr size_t kSlotBytes = kChunks * 64 * 16 + 64 * 16;  // x + sx of one window, one A row

// One weight matrix, or several sharing the activations (segments, resident kernel only; returns
// hipErrorNotSupported when the activations do not fit in LDS and nseg > 1).
struct Seg {
    const void* W;
    void* C;
    int N;
};

// Segment table of a launch and its row-group count.  Paired rows: one segment of N row groups
// whose two rows come from the first and second matrix (W[0], W[1]).
template <typename TC, int YT>
int seg_table(const Seg* segs, int nseg, const GemvFuse& fz, GemvSegs<TC>& sg) {
    int nrg = 0;
    for (int j = 0; j < kMaxSegs; ++j) {
        if (j < nseg) {
            sg.W[j] = static_cast<const uint8_t*>(segs[j].W);
            sg.C[j] = static_cast<TC*>(segs[j].C);
            sg.N[j] = segs[j].N;
            nrg += (segs[j].N + YT - 1) / YT;
            sg.gend[j] = nrg;
        } else {
            sg.W[j] = sg.W[0];
            sg.C[j] = sg.C[0];
            sg.N[j] = sg.N[0];
            sg.gend[j] = INT_MAX;
        }
    }
    if (fz.pair) {
        nrg = segs[0].N;
        sg.gend[0] = nrg;
        for (int j = 1; j < kMaxSegs; ++j) sg.gend[j] = INT_MAX;
    }
    return nrg;
}

template <class F, int MR, int YT, int NW, typename TA, typename TC>
hipError_t launch_fast(const void* A, const Seg* segs, int nseg, int M, int K, bool a_vec, const GemvFuse& fz,
                       hipStream_t stream) {
    DevInfo di;
    hipError_t e = device_info(di);
    if (e != hipSuccess) return e;
    const int nwin = (K + kGemvWindow - 1) / kGemvWindow;
    const int mblocks = (M + MR - 1) / MR;
    const size_t res_lds = static_cast<size_t>(MR) * nwin * kSlotBytes;
    const int threads = 64 * NW;
    const bool folded = fz.kind != 0 || fz.ea != nullptr || fz.pair != 0;
    if (folded && !kFoldable<F, MR, YT, NW, TA>) return hipErrorNotSupported;
    if (fz.pair && (YT != 2 || MR != 1 || nseg != 2 || segs[0].N != segs[1].N || sizeof(TC) != 2)) return hipErrorNotSupported;
    if (fz.kind != 0 && static_cast<int64_t>(nwin) * MR * 256 > static_cast<int64_t>(kFuseOwn) * threads)
        return hipErrorNotSupported;
    // fp32 activations: one LDS maximum per staged (window, row)
    const bool wmax_fits = !std::is_same<TA, float>::value || MR * nwin <= kWmaxEntries;
    if constexpr (F::kStream) {
        auto try_stream = [&](auto nsc) -> bool {
            constexpr int NS = decltype(nsc)::value;
            const size_t row_bytes = static_cast<size_t>(K / F::kQK) * F::kBlockBytes;
            const size_t st_lds = res_lds + static_cast<size_t>(NW) * NS * YT * WinSlot<F>::kBytes;
            bool ok = row_bytes % 16 == 0 && st_lds <= di.max_lds && wmax_fits;
            for (int j = 0; j < nseg; ++j) ok = ok && (reinterpret_cast<uintptr_t>(segs[j].W) & 15u) == 0;
            if (!ok) return false;
            const void* kern = reinterpret_cast<const void*>(&gemv_stream_kernel<F, MR, YT, NW, NS, TA, TC>);
            int occ = 0;
            if ((e = occupancy(kern, threads, st_lds, occ)) != hipSuccess) return true;
            GemvSegs<TC> sg;
            const int nrg = seg_table<TC, YT>(segs, nseg, fz, sg);
            const int need = (nrg + NW - 1) / NW;
            const int fill = max(1, occ * di.cus / mblocks);
            const dim3 grid(min(need, fill), mblocks);
            hipLaunchKernelGGL((gemv_stream_kernel<F, MR, YT, NW, NS, TA, TC>), grid, dim3(threads), st_lds, stream,
                               static_cast<const TA*>(A), sg, M, K, a_vec ? 1 : 0, nrg, fz);
            e = hipGetLastError();
            return true;
        };
        // At M = 1 with one window and fewer than 16384 rows in all, lanes read their slots
        // straight from memory instead (8B Q8_0 o 4096 x 4096: 8.3 -> 6.6 us, fused q/k/v
        // 6144 x 4096: 9.9 -> 8.7 us; the fused gate + up, 28672 rows, stays streamed: 26 vs 27 us).
        int rows = 0;
        for (int j = 0; j < nseg; ++j) rows += segs[j].N;
        const bool lane_slots = MR == 1 && nwin == 1 && rows < 16384 && !folded;
        if (!lane_slots && try_stream(std::integral_constant<int, kGemvNS>{})) return e;
    }
    if (res_lds <= di.max_lds && wmax_fits) {
        const void* kern = reinterpret_cast<const void*>(&gemv_resident_kernel<F, MR, YT, NW, TA, TC>);
        int occ = 0;
        if ((e = occupancy(kern, threads, res_lds, occ)) != hipSuccess) return e;
        GemvSegs<TC> sg;
        const int nrg = seg_table<TC, YT>(segs, nseg, fz, sg);
        const int need = (nrg + NW - 1) / NW;
        const int fill = max(1, occ * di.cus / mblocks);
        const dim3 grid(min(need, fill), mblocks);
        hipLaunchKernelGGL((gemv_resident_kernel<F, MR, YT, NW, TA, TC>), grid, dim3(threads), res_lds, stream,
                           static_cast<const TA*>(A), sg, M, K, a_vec ? 1 : 0, nrg, fz);
        return hipGetLastError();
    }
    if (nseg != 1 || folded) return hipErrorNotSupported;
    const int N = segs[0].N;
    const size_t win_lds = static_cast<size_t>(MR) * 2 * kSlotBytes;
    const void* kern = reinterpret_cast<const void*>(&gemv_window_kernel<F, MR, YT, NW, TA, TC>);
    int occ = 0;
    if ((e = occupancy(kern, threads, win_lds, occ)) != hipSuccess) return e;
    constexpr int kRows = NW * YT;
    const dim3 grid((N + kRows - 1) / kRows, mblocks);
    hipLaunchKernelGGL((gemv_window_kernel<F, MR, YT, NW, TA, TC>), grid, dim3(threads), win_lds, stream,
                       static_cast<const TA*>(A), static_cast<const uint8_t*>(segs[0].W), static_cast<TC*>(segs[0].C),
                       M, N, K, a_vec ? 1 : 0);
    return hipGetLastError();
}

template <class F, int NW, typename TA, typename TC>
hipError_t dispatch_rows(const void* A, const Seg* segs, int nseg, int M, int N, int K, bool a_vec,
                         const GemvFuse& fz, hipStream_t stream) {
    // Rows per wave item by the total row count (enough items to cover the 256 CUs several times).
    if (fz.pair) {
        if (M != 1) return hipErrorNotSupported;
        return launch_fast<F, 1, 2, NW, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
    }
    if (M == 1) {
        // One weight row per wave item: more, smaller items spread short launches over more waves
        // (8B Q4_K q/k/v 6.3 -> 6.0 us, Q6_K down 4096 x 14336: 14.1 -> 12.9 us against two rows).
        // The streamed-window formats keep two rows per item on single matrices of 2048..8191
        // rows, where their window copies favour it (8B Q8_0 down 18.3 -> 16.4 us, o 8.8 -> 8.3 us).
        if constexpr (F::kStream) {
            if (nseg == 1 && N >= 2048 && N < 8192)
                return launch_fast<F, 1, 2, NW, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
        }
        // Q4_K over 16384 rows and more (gate + up in one launch), without a fused prologue or
        // epilogue: two rows per item, so that every wave holds the same number of items (70B
        // gate + up 2 x 28672 x 8192: 49.1 -> 47.5 us).
        if constexpr (F::kType == QMM_TYPE_Q4_K) {
            if (N >= 16384 && fz.kind == 0 && fz.ea == nullptr)
                return launch_fast<F, 1, 2, NW, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
        }
        return launch_fast<F, 1, 1, NW, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
    }
    if (M == 2) {
        if (N >= 8192) return launch_fast<F, 2, 1, NW, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
        if (N >= 2048) return launch_fast<F, 2, 2, NW, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
        return launch_fast<F, 2, 1, NW, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
    }
    if (M <= 4 && !fz.pair) {
        // M = 3, 4 where four staged rows exceed the LDS but two fit (70B down, K = 28672): two
        // 2-row blocks of resident activations instead of the windowed kernel's one barrier per
        // window (70B down at M = 4: 76 -> 69 us); rows keep the M = 1 arithmetic.
        DevInfo di;
        const hipError_t e = device_info(di);
        if (e != hipSuccess) return e;
        const size_t per_row = static_cast<size_t>((K + kGemvWindow - 1) / kGemvWindow) * kSlotBytes;
        if (4 * per_row > di.max_lds && 2 * per_row <= di.max_lds)
            return launch_fast<F, 2, 2, 16, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
    }
    if (N >= 4096) return launch_fast<F, 4, 2, NW, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
    return launch_fast<F, 4, 1, NW, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
}

template <class F, typename TA, typename TC>
hipError_t dispatch_fast(const void* A, const Seg* segs, int nseg, int M, int K, bool a_vec, const GemvFuse& fz,
                         hipStream_t stream) {
    int N = 0;
    for (int j = 0; j < nseg; ++j) N += segs[j].N;
    // M > 4: blocks of 8 activation rows (two weight rows per wave item) stream the weights half as
    // often as blocks of 4 (70B down at M = 8: 149 -> 110 us, gate 86 -> 79 us), where they add
    // no padded row over the 4-row tiling (M % 8 == 0 or >= 5).  F16, and fp32 activations beyond
    // two windows (resident LDS), keep 4-row blocks: their 8-row windowed kernels would spill.
    const int nwin = (K + kGemvWindow - 1) / kGemvWindow;
    if constexpr (F::kType != QMM_TYPE_F16) {
        if (M > 4 && !fz.pair && (M % 8 == 0 || M % 8 >= 5) && (std::is_same<TA, __half>::value || nwin <= 2))
            return launch_fast<F, 8, 2, 8, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
    }
    // Resident activations above 40 KB of LDS leave room for at most three workgroups per CU:
    // 16-wave workgroups then keep more waves (bytes in flight) per CU.  M = 1, 2 only (larger M
    // tiles use the windowed kernel at such K).
    const size_t res_lds = static_cast<size_t>(min(M, 4)) * nwin * kSlotBytes;
    // Q4_K at M = 1 over one window and 16384 rows or more (8B gate + up): 4-wave workgroups
    // (8B gate + up 2 x 14336 x 4096: 14.9 -> 13.8 us).
    if constexpr (F::kType == QMM_TYPE_Q4_K) {
        if (M == 1 && !fz.pair && fz.kind == 0 && fz.ea == nullptr && nwin == 1 && N >= 16384)
            return launch_fast<F, 1, 2, 4, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
    }
    if (M <= kGemvNW16MaxM && res_lds > 40 * 1024)
        return dispatch_rows<F, 16, TA, TC>(A, segs, nseg, M, N, K, a_vec, fz, stream);
    return dispatch_rows<F, kGemvNW, TA, TC>(A, segs, nseg, M, N, K, a_vec, fz, stream);
}

template <int T, typename TA, typename TC>
hipError_t launch_fallback(const void* A, const void* W, void* C, int M, int N, int K, hipStream_t stream) {
    const dim3 grid((N + 3) / 4, M);
    hipLaunchKernelGGL((gemv_fallback_kernel<T, TA, TC>), grid, dim3(256), 0, stream,
                       static_cast<const TA*>(A), static_cast<const uint8_t*>(W), static_cast<TC*>(C), M, N, K);
    return hipGetLastError();
}

// Fast-path eligibility of a weight pointer: Q4_K headers are read as 16-byte vectors, the other
// formats need 2-byte alignment (fp16 scales or values).
bool fast_weights(int t, const void* W) {
    const uintptr_t wa = reinterpret_cast<uintptr_t>(W);
    return t == QMM_TYPE_Q4_K ? (wa & 15u) == 0 : (wa & 1u) == 0;
}

template <typename TA, typename TC>
hipError_t dispatch_types(int t, const void* A, const Seg* segs, int nseg, int M, int K, const GemvFuse& fz,
                          hipStream_t stream, bool identity) {
    const bool a_ok = (reinterpret_cast<uintptr_t>(A) & (sizeof(TA) - 1)) == 0;
    const bool a_vec = (reinterpret_cast<uintptr_t>(A) & 15u) == 0;
    bool fast = a_ok && (t != QMM_TYPE_F16 || K % 16 == 0);
    for (int j = 0; j < nseg; ++j) fast = fast && fast_weights(t, segs[j].W);
    // the matrix-core GEMV from the format's smallest M (its rows are the same for every M it serves)
    if (fast && M >= gemv_mfma_min_m(t, identity) && fz.kind == 0 && fz.ea == nullptr && fz.pair == 0) {
        const void* W[kMaxSegs];
        void* C[kMaxSegs];
        int N[kMaxSegs];
        for (int j = 0; j < nseg; ++j) {
            W[j] = segs[j].W;
            C[j] = segs[j].C;
            N[j] = segs[j].N;
        }
        const int a_dt = std::is_same<TA, float>::value ? QMM_DTYPE_F32 : QMM_DTYPE_F16;
        const int c_dt = std::is_same<TC, float>::value ? QMM_DTYPE_F32 : QMM_DTYPE_F16;
        const hipError_t e = launch_gemv_mfma(t, A, a_dt, c_dt, M, K, W, C, N, nseg, stream);
        if (e != hipErrorNotSupported) return e;
    }
    if (!fast) {
        if (nseg != 1 || fz.kind != 0 || fz.ea != nullptr || fz.pair != 0) return hipErrorNotSupported;
        const void* W = segs[0].W;
        void* C = segs[0].C;
        const int N = segs[0].N;
        switch (t) {
            case QMM_TYPE_Q4_K: return launch_fallback<QMM_TYPE_Q4_K, TA, TC>(A, W, C, M, N, K, stream);
            case QMM_TYPE_Q6_K: return launch_fallback<QMM_TYPE_Q6_K, TA, TC>(A, W, C, M, N, K, stream);
            case QMM_TYPE_Q8_0: return launch_fallback<QMM_TYPE_Q8_0, TA, TC>(A, W, C, M, N, K, stream);
            case QMM_TYPE_Q4_0: return launch_fallback<QMM_TYPE_Q4_0, TA, TC>(A, W, C, M, N, K, stream);
            case QMM_TYPE_F16: return launch_fallback<QMM_TYPE_F16, TA, TC>(A, W, C, M, N, K, stream);
            default: return hipErrorInvalidValue;
        }
    }
    switch (t) {
        case QMM_TYPE_Q4_K: return dispatch_fast<GQ4K, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
        case QMM_TYPE_Q6_K: return dispatch_fast<GQ6K, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
        case QMM_TYPE_Q8_0: return dispatch_fast<GQ80, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
        case QMM_TYPE_Q4_0: return dispatch_fast<GQ40, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
        case QMM_TYPE_F16: return dispatch_fast<GF16, TA, TC>(A, segs, nseg, M, K, a_vec, fz, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t dispatch_dtypes(int t, const void* A, int a_dtype, int c_dtype, const Seg* segs, int nseg, int M, int K,
                           hipStream_t stream, bool identity, const GemvFuse& fz = GemvFuse{}) {
    if (a_dtype == QMM_DTYPE_F32) {
        if (fz.kind != 0 || fz.ea != nullptr || fz.pair != 0) return hipErrorNotSupported;
        if (c_dtype == QMM_DTYPE_F32) return dispatch_types<float, float>(t, A, segs, nseg, M, K, fz, stream, identity);
        return dispatch_types<float, __half>(t, A, segs, nseg, M, K, fz, stream, identity);
    }
    if (c_dtype == QMM_DTYPE_F32) {
        if (fz.ea != nullptr || fz.pair != 0) return hipErrorNotSupported;
        return dispatch_types<__half, float>(t, A, segs, nseg, M, K, fz, stream, identity);
    }
    return dispatch_types<__half, __half>(t, A, segs, nseg, M, K, fz, stream, identity);
}

}  // namespace

hipError_t launch_gemv(int ggml_type, const void* A, int a_dtype, const void* W, void* C,
                       int c_dtype, int M, int N, int K, hipStream_t stream, bool identity) {
    const Seg seg{W, C, N};
    return dispatch_dtypes(ggml_type, A, a_dtype, c_dtype, &seg, 1, M, K, stream, identity);
}

hipError_t launch_gemv_fused(int ggml_type, const void* A, int a_dtype, int c_dtype, int M, int K,
                             const void* const* W, void* const* C, const int* N, int count, hipStream_t stream,
                             bool identity) {
    if (count < 2 || count > kMaxSegs) return hipErrorNotSupported;
    Seg segs[kMaxSegs];
    for (int j = 0; j < count; ++j) segs[j] = Seg{W[j], C[j], N[j]};
    return dispatch_dtypes(ggml_type, A, a_dtype, c_dtype, segs, count, M, K, stream, identity);
}

int gemv_max_fused() { return kMaxSegs; }

hipError_t launch_gemv_ex(int ggml_type, const void* A, int c_dtype, int M, int K, const void* const* W, void* const* C,
                          const int* N, int count, const GemvFuse& fz, hipStream_t stream) {
    if (count < 1 || count > kMaxSegs || M != 1) return hipErrorNotSupported;
    // the folded staging reads 16-value pieces (and the norm weights) as 16-byte vectors
    const uintptr_t align = reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(fz.R) | reinterpret_cast<uintptr_t>(fz.w);
    if (fz.kind < 0 || fz.kind > 2) return hipErrorInvalidValue;
    if (fz.kind != 0 && (K % 16 != 0 || (align & 15u) != 0)) return hipErrorNotSupported;
    Seg segs[kMaxSegs];
    for (int j = 0; j < count; ++j) segs[j] = Seg{W[j], C[j], N[j]};
    return dispatch_dtypes(ggml_type, A, QMM_DTYPE_F16, c_dtype, segs, count, M, K, stream, false, fz);
}

}  // namespace qmm
