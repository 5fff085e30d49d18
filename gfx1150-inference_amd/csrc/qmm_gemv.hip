// Decode-path GEMV family (M < kGemvMaxM): C[m, n] = sum_k A[m, k] * dequant(W)[n, k].
//
// MI355X design (replaces the reference's wave32 one-output-per-wave kernels,
// src/kernels/dequantize.hip:97-148, 152-210, 232-332, 377-505, 549-685):
//   * A wave owns YT consecutive weight rows and walks K in windows of 2048 weights.
//     In every window each of the 64 lanes owns a fixed 32-weight slot (four runs of
//     8 contiguous k), so one wave-wide 16-byte load per row covers a contiguous,
//     16-byte-aligned stretch of the packed row (coalesced HBM streaming).
//   * The lane's 32 activations (per A row) are loaded once per window and reused for
//     all YT rows; per-run sums of x are hoisted so block offsets/mins cost one FMA.
//   * Q4_K rows are read straight from HBM (144-byte super-blocks are 16-byte aligned);
//     Q6_K / Q8_0 / Q4_0 windows (1680 / 2176 / 1152 bytes) are staged through a
//     wave-private LDS buffer and re-sliced per lane.
//   * fp32 accumulation with explicit FMAs in a fixed order: the result of row m does not
//     depend on M, on YT or on the grid, so every M < kGemvMaxM is bit-identical to M=1
//     (the reference's prefill-vs-M=1 invariant, tests/test_phase5_scale.py:274-310).
//   * The cross-lane reduction is a fixed DPP sequence (no atomics; deterministic).
#include <type_traits>

#include "qmm_device.h"

namespace qmm {
namespace {

constexpr int kWavesPerBlock = 4;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Decoded 32-weight slot of one row: code bytes (run r uses q[2r], q[2r+1]) and per-group
// scale a / offset b; contribution = sum_g a[g] * (sum_{runs in g} x*code) - b[g] * sum x.
template <int G>
struct Slot {
    uint32_t q[8];
    float a[G];
    float b[G];
};

// ------------------------------------------------------------------------------------
// Q4_K: 8 super-blocks per window, lane = (sb = lane/8, piece p = lane%8 of the 128 qs bytes).
// ------------------------------------------------------------------------------------
struct FmtQ4K {
    static constexpr int kType = QMM_TYPE_Q4_K;
    static constexpr int kQK = kQK_K;
    static constexpr int kBlockBytes = kBytesQ4_K;
    static constexpr int kWindowBytes = 8 * kBytesQ4_K;
    static constexpr bool kStaged = false;
    static constexpr int kGroups = 2;  // runs {0,1} lo nibbles, {2,3} hi nibbles
    static constexpr int kLoads = 2;   // header + 16 qs bytes

    __device__ static void runs(int lane, int off[4]) {
        const int sb = lane >> 3, p = lane & 7;
        const int base = 256 * sb + 64 * (p >> 1) + 16 * (p & 1);
        off[0] = base; off[1] = base + 8; off[2] = base + 32; off[3] = base + 40;
    }
    __device__ static bool lane_valid(int lane, int k0, int K) { return k0 + 256 * (lane >> 3) < K; }

    // Loads: raw[0] = 16-byte header of the lane's super-block, raw[1] = its qs bytes 16p..16p+15.

    // Every lane decodes (scale, min) of sub-block j = p; lanes p, p^1 share chunk p/2 and
    // pick sub-blocks 2c (= p&~1) and 2c+1 (= p|1) from their quad with DPP.
    __device__ static Slot<2> decode(const u32x4 raw[2], int lane) {
        const u32x4 h = raw[0];
        const u32x4 v = raw[1];
        const int p = lane & 7;
        const int s8 = 8 * (p & 3);
        const uint32_t sc_lo = (h.y >> s8) & 63u;
        const uint32_t m_lo = (h.z >> s8) & 63u;
        const uint32_t sc_hi = ((h.w >> s8) & 15u) | (((h.y >> (s8 + 6)) & 3u) << 4);
        const uint32_t m_hi = ((h.w >> (s8 + 4)) & 15u) | (((h.z >> (s8 + 6)) & 3u) << 4);
        const uint32_t sc = p < 4 ? sc_lo : sc_hi;
        const uint32_t m = p < 4 ? m_lo : m_hi;
        const float d = half_bits_to_float(h.x);
        const float dmin = half_bits_to_float(h.x >> 16);
        const float scale = d * static_cast<float>(sc);
        const float mn = dmin * static_cast<float>(m);
        Slot<2> s;
        s.a[0] = dpp_quad(scale, 0xA0);
        s.a[1] = dpp_quad(scale, 0xF5) * 0.0625f;  // hi nibbles enter as 16*q
        s.b[0] = dpp_quad(mn, 0xA0);
        s.b[1] = dpp_quad(mn, 0xF5);
        s.q[0] = v.x & 0x0F0F0F0Fu; s.q[1] = v.y & 0x0F0F0F0Fu;
        s.q[2] = v.z & 0x0F0F0F0Fu; s.q[3] = v.w & 0x0F0F0F0Fu;
        s.q[4] = v.x & 0xF0F0F0F0u; s.q[5] = v.y & 0xF0F0F0F0u;
        s.q[6] = v.z & 0xF0F0F0F0u; s.q[7] = v.w & 0xF0F0F0F0u;
        return s;
    }
};

// Reads the 8 bytes at LDS byte offset o (o even); `odd` says o % 4 == 2.
__device__ __forceinline__ void lds_read8(const uint32_t* lds32, int o, bool odd, uint32_t& lo, uint32_t& hi) {
    const int b = (o - (odd ? 2 : 0)) >> 2;
    const uint32_t d0 = lds32[b], d1 = lds32[b + 1], d2 = lds32[b + 2];
    lo = odd ? __builtin_amdgcn_alignbyte(d1, d0, 2) : d0;
    hi = odd ? __builtin_amdgcn_alignbyte(d2, d1, 2) : d1;
}

// ------------------------------------------------------------------------------------
// Q6_K: 8 super-blocks (1680 B) per window; lane = (sb = lane/8, half n, quarter qq):
// 8 values l = 8qq..8qq+7 of each of the four 32-wide groups t of half n.
// ------------------------------------------------------------------------------------
struct FmtQ6K {
    static constexpr int kType = QMM_TYPE_Q6_K;
    static constexpr int kQK = kQK_K;
    static constexpr int kBlockBytes = kBytesQ6_K;
    static constexpr int kWindowBytes = 8 * kBytesQ6_K;  // 1680 = 105 x 16
    static constexpr bool kStaged = true;
    static constexpr int kGroups = 4;
    static constexpr int kLoads = (kWindowBytes / 16 + 63) / 64;

    __device__ static void runs(int lane, int off[4]) {
        const int sb = lane >> 3, n = (lane >> 2) & 1, qq = lane & 3;
        const int base = 256 * sb + 128 * n + 8 * qq;
#pragma unroll
        for (int t = 0; t < 4; ++t) off[t] = base + 32 * t;
    }
    __device__ static bool lane_valid(int lane, int k0, int K) { return k0 + 256 * (lane >> 3) < K; }

    __device__ static Slot<4> decode(const uint32_t* lds32, int lane) {
        const int sb = lane >> 3, n = (lane >> 2) & 1, qq = lane & 3;
        const int o = 210 * sb;
        const bool odd = (sb & 1) != 0;
        uint32_t a0, a1, b0, b1, h0, h1, s0, s1;
        lds_read8(lds32, o + 64 * n + 8 * qq, odd, a0, a1);
        lds_read8(lds32, o + 64 * n + 32 + 8 * qq, odd, b0, b1);
        lds_read8(lds32, o + 128 + 32 * n + 8 * qq, odd, h0, h1);
        lds_read8(lds32, o + 192 + 8 * n, odd, s0, s1);
        const uint32_t dw = lds32[(o + 208 - (odd ? 2 : 0)) >> 2];
        const float d = half_bits_to_float(odd ? (dw >> 16) : dw);
        Slot<4> s;
        s.q[0] = (a0 & 0x0F0F0F0Fu) | ((h0 << 4) & 0x30303030u);
        s.q[1] = (a1 & 0x0F0F0F0Fu) | ((h1 << 4) & 0x30303030u);
        s.q[2] = (b0 & 0x0F0F0F0Fu) | ((h0 << 2) & 0x30303030u);
        s.q[3] = (b1 & 0x0F0F0F0Fu) | ((h1 << 2) & 0x30303030u);
        s.q[4] = ((a0 >> 4) & 0x0F0F0F0Fu) | (h0 & 0x30303030u);
        s.q[5] = ((a1 >> 4) & 0x0F0F0F0Fu) | (h1 & 0x30303030u);
        s.q[6] = ((b0 >> 4) & 0x0F0F0F0Fu) | ((h0 >> 2) & 0x30303030u);
        s.q[7] = ((b1 >> 4) & 0x0F0F0F0Fu) | ((h1 >> 2) & 0x30303030u);
        // Signed sub-scales through int8_t casts: __builtin_amdgcn_sbfe with a lane-variable
        // offset was lowered with an unsigned int->float conversion, turning negative
        // scales into ~4e9.
        const int is8 = 8 * (qq >> 1);
        const float sc0 = static_cast<float>(static_cast<int8_t>(s0 >> is8));
        const float sc1 = static_cast<float>(static_cast<int8_t>(s0 >> (is8 + 16)));
        const float sc2 = static_cast<float>(static_cast<int8_t>(s1 >> is8));
        const float sc3 = static_cast<float>(static_cast<int8_t>(s1 >> (is8 + 16)));
        s.a[0] = d * sc0; s.a[1] = d * sc1; s.a[2] = d * sc2; s.a[3] = d * sc3;
#pragma unroll
        for (int g = 0; g < 4; ++g) s.b[g] = 32.0f * s.a[g];  // codes enter unsigned (q + 32)
        return s;
    }
};

// ------------------------------------------------------------------------------------
// Q8_0: 64 blocks (2176 B) per window, lane = block.
// ------------------------------------------------------------------------------------
struct FmtQ80 {
    static constexpr int kType = QMM_TYPE_Q8_0;
    static constexpr int kQK = kQK8_0;
    static constexpr int kBlockBytes = kBytesQ8_0;
    static constexpr int kWindowBytes = 64 * kBytesQ8_0;  // 2176 = 136 x 16
    static constexpr bool kStaged = true;
    static constexpr int kGroups = 1;
    static constexpr int kLoads = (kWindowBytes / 16 + 63) / 64;

    __device__ static void runs(int lane, int off[4]) {
#pragma unroll
        for (int r = 0; r < 4; ++r) off[r] = 32 * lane + 8 * r;
    }
    __device__ static bool lane_valid(int lane, int k0, int K) { return k0 + 32 * lane < K; }

    __device__ static Slot<1> decode(const uint32_t* lds32, int lane) {
        const int o = 34 * lane;
        const bool odd = (lane & 1) != 0;
        const int b = (o - (odd ? 2 : 0)) >> 2;
        uint32_t dw[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) dw[i] = lds32[b + i];
        const float d = half_bits_to_float(odd ? (dw[0] >> 16) : dw[0]);
        Slot<1> s;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t v = odd ? dw[i + 1] : __builtin_amdgcn_alignbyte(dw[i + 1], dw[i], 2);
            s.q[i] = v ^ 0x80808080u;  // signed int8 -> unsigned q + 128
        }
        s.a[0] = d;
        s.b[0] = 128.0f * d;
        return s;
    }
};

// ------------------------------------------------------------------------------------
// Q4_0: 64 blocks (1152 B) per window, lane = block.
// ------------------------------------------------------------------------------------
struct FmtQ40 {
    static constexpr int kType = QMM_TYPE_Q4_0;
    static constexpr int kQK = kQK4_0;
    static constexpr int kBlockBytes = kBytesQ4_0;
    static constexpr int kWindowBytes = 64 * kBytesQ4_0;  // 1152 = 72 x 16
    static constexpr bool kStaged = true;
    static constexpr int kGroups = 2;
    static constexpr int kLoads = (kWindowBytes / 16 + 63) / 64;

    __device__ static void runs(int lane, int off[4]) {
#pragma unroll
        for (int r = 0; r < 4; ++r) off[r] = 32 * lane + 8 * r;
    }
    __device__ static bool lane_valid(int lane, int k0, int K) { return k0 + 32 * lane < K; }

    __device__ static Slot<2> decode(const uint32_t* lds32, int lane) {
        const int o = 18 * lane;
        const bool odd = (lane & 1) != 0;
        const int b = (o - (odd ? 2 : 0)) >> 2;
        uint32_t dw[5];
#pragma unroll
        for (int i = 0; i < 5; ++i) dw[i] = lds32[b + i];
        const float d = half_bits_to_float(odd ? (dw[0] >> 16) : dw[0]);
        uint32_t qs[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) qs[i] = odd ? dw[i + 1] : __builtin_amdgcn_alignbyte(dw[i + 1], dw[i], 2);
        Slot<2> s;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s.q[i] = qs[i] & 0x0F0F0F0Fu;      // weights 0..15
            s.q[4 + i] = qs[i] & 0xF0F0F0F0u;  // weights 16..31, entering as 16*q
        }
        s.a[0] = d;
        s.a[1] = d * 0.0625f;
        s.b[0] = 8.0f * d;
        s.b[1] = 8.0f * d;
        return s;
    }
};

template <typename TA>
__device__ __forceinline__ void load_run8(const TA* __restrict__ p, bool vec, float x[8]);

template <>
__device__ __forceinline__ void load_run8<float>(const float* __restrict__ p, bool vec, float x[8]) {
    if (vec) {
        const float4 u = reinterpret_cast<const float4*>(p)[0];
        const float4 v = reinterpret_cast<const float4*>(p)[1];
        x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w;
        x[4] = v.x; x[5] = v.y; x[6] = v.z; x[7] = v.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = p[i];
    }
}

template <>
__device__ __forceinline__ void load_run8<__half>(const __half* __restrict__ p, bool vec, float x[8]) {
    if (vec) {
        const uint4 u = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = half_bits_to_float(w[i]);
            x[2 * i + 1] = half_bits_to_float(w[i] >> 16);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = __half2float(p[i]);
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

// Weight bytes of one window for the YT rows of a wave, as loaded by one lane.
template <class F, int YT>
struct WinBuf {
    static constexpr int kRaw = F::kStaged ? F::kLoads : 2;
    u32x4 raw[YT][kRaw];
};

// Activations of one window for one lane: 4 runs of 8 consecutive k per A row.
template <int MR>
struct XBuf {
    float x[MR][32];
};

// One wave computes YT consecutive output rows over a K-slice; KS waves of a workgroup
// split the windows of the same rows round-robin (window w goes to wave w % KS) and their
// partial sums are added through LDS in wave order.  Window w + KS's weight bytes (and, for
// one A row, its activations) are loaded while window w is being multiplied.
template <class F, int MR, int YT, int KS, typename TA, typename TC>
__global__ __launch_bounds__(kWave * kWavesPerBlock)
void gemv_kernel(const TA* __restrict__ A, const uint8_t* __restrict__ W, TC* __restrict__ C,
                 int M, int N, int K, int a_vec) {
    constexpr int G = F::kGroups;
    constexpr int RPG = 4 / G;  // runs per group
    constexpr int kPieces = F::kWindowBytes / 16;
    constexpr int kRaw = WinBuf<F, YT>::kRaw;
    constexpr int kLdsWords = F::kStaged ? ((F::kWindowBytes + 16 + 15) / 16) * 4 : 4;
    constexpr int kRowGroups = kWavesPerBlock / KS;
    constexpr bool kPrefetchX = MR == 1;
    static_assert(kWavesPerBlock % KS == 0, "KS must divide the waves of a block");
    __shared__ __align__(16) uint32_t lds_all[kWavesPerBlock][kLdsWords];
    __shared__ float red[KS > 1 ? kWavesPerBlock : 1][MR * YT];

    const int lane = threadIdx.x & (kWave - 1);
    const int wv = threadIdx.x / kWave;
    const int rg = wv / KS;
    const int ks = wv - rg * KS;
    const int row0 = (blockIdx.x * kRowGroups + rg) * YT;
    const bool active = row0 < N;  // wave-uniform; idle waves still join the K-split reduction
    const int m0 = blockIdx.y * MR;
    const int mrows = min(MR, M - m0);
    const uint32_t row_bytes = static_cast<uint32_t>(K / F::kQK) * F::kBlockBytes;
    const bool vec = a_vec != 0;
    uint32_t* lds32 = lds_all[wv];

    // Rows past N and A rows past M are computed on clamped (valid) addresses and never
    // stored, so the steady-state loop carries no per-row predicates.  The host guarantees
    // N * row_bytes < 2^32, so byte offsets fit 32 bits.
    uint32_t rowoff[YT];
#pragma unroll
    for (int y = 0; y < YT; ++y) rowoff[y] = static_cast<uint32_t>(min(row0 + y, N - 1)) * row_bytes;
    const TA* xrow[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) xrow[m] = A + static_cast<size_t>(min(m0 + m, M - 1)) * K;

    int off[4];
    F::runs(lane, off);
    uint32_t loff[kRaw];  // per-lane byte offsets of the loads inside a window
    if constexpr (F::kStaged) {
#pragma unroll
        for (int j = 0; j < kRaw; ++j) loff[j] = 16u * static_cast<uint32_t>(min(lane + kWave * j, kPieces - 1));
    } else {
        loff[0] = static_cast<uint32_t>(F::kBlockBytes * (lane >> 3));
        loff[1] = loff[0] + 16u + 16u * static_cast<uint32_t>(lane & 7);
    }

    float acc[MR][YT];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int y = 0; y < YT; ++y) acc[m][y] = 0.0f;

    auto load_x = [&](XBuf<MR>& xb, int w, auto tail_tag) {
        constexpr bool kTail = decltype(tail_tag)::value;
        const int k0 = w * kWindow;
        const bool lv = kTail ? F::lane_valid(lane, k0, K) : true;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int o = kTail ? (lv ? off[r] : 0) : off[r];
                load_run8<TA>(xrow[m] + k0 + o, vec, &xb.x[m][8 * r]);
                if constexpr (kTail) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) xb.x[m][8 * r + i] = lv ? xb.x[m][8 * r + i] : 0.0f;
                }
            }
        }
    };

    // Issues the loads of window w: the weight bytes of the YT rows, then the activations.
    auto load = [&](WinBuf<F, YT>& b, XBuf<MR>& xb, int w, auto tail_tag) {
        constexpr bool kTail = decltype(tail_tag)::value;
        const int k0 = w * kWindow;
        const uint32_t wb = static_cast<uint32_t>(w) * F::kWindowBytes;
        uint32_t lo[kRaw];
#pragma unroll
        for (int j = 0; j < kRaw; ++j) lo[j] = loff[j];
        if constexpr (kTail) {
            const bool lv = F::lane_valid(lane, k0, K);
            const int valid_pieces = static_cast<int>((K - k0) / F::kQK) * F::kBlockBytes / 16;
#pragma unroll
            for (int j = 0; j < kRaw; ++j) {
                if constexpr (F::kStaged) lo[j] = 16u * static_cast<uint32_t>(min(lane + kWave * j, valid_pieces - 1));
                else lo[j] = lv ? loff[j] : (j == 0 ? 0u : 16u);
            }
        }
#pragma unroll
        for (int y = 0; y < YT; ++y)
#pragma unroll
            for (int j = 0; j < kRaw; ++j)
                b.raw[y][j] = *reinterpret_cast<const u32x4*>(W + (rowoff[y] + wb + lo[j]));
        if constexpr (kPrefetchX) load_x(xb, w, tail_tag);
    };

    auto compute = [&](const WinBuf<F, YT>& b, const XBuf<MR>& xpre, int w, auto tail_tag) {
        constexpr bool kTail = decltype(tail_tag)::value;
        const bool lv = kTail ? F::lane_valid(lane, w * kWindow, K) : true;
        XBuf<MR> xl;
        if constexpr (!kPrefetchX) load_x(xl, w, tail_tag);
        const XBuf<MR>& xb = kPrefetchX ? xpre : xl;
        float sx[MR][G];
#pragma unroll
        for (int m = 0; m < MR; ++m) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float t = xb.x[m][8 * RPG * g];
#pragma unroll
                for (int i = 1; i < 8 * RPG; ++i) t += xb.x[m][8 * RPG * g + i];
                sx[m][g] = t;
            }
        }
#pragma unroll
        for (int y = 0; y < YT; ++y) {
            Slot<G> s;
            if constexpr (F::kStaged) {
                wave_lds_sync();
#pragma unroll
                for (int j = 0; j < kRaw; ++j)
                    reinterpret_cast<u32x4*>(lds32)[min(lane + kWave * j, kPieces - 1)] = b.raw[y][j];
                wave_lds_sync();
                s = F::decode(lds32, lane);
            } else {
                s = F::decode(b.raw[y], lane);
            }
            if constexpr (kTail) {
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    s.a[g] = lv ? s.a[g] : 0.0f;
                    s.b[g] = lv ? s.b[g] : 0.0f;
                }
            }
            float c[32];
#pragma unroll
            for (int i = 0; i < 32; ++i) c[i] = ubyte_to_float(opaque(s.q[i >> 2]), i & 3);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float a = acc[m][y];
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    float t = 0.0f;
#pragma unroll
                    for (int i = 0; i < 8 * RPG; ++i) t = __fmaf_rn(xb.x[m][8 * RPG * g + i], c[8 * RPG * g + i], t);
                    a = __fmaf_rn(s.a[g], t, a);
                    a = __fmaf_rn(-s.b[g], sx[m][g], a);
                }
                acc[m][y] = a;
            }
        }
    };

    const int nfull = K / kWindow;
    if (active) {
        int w = ks;
        if (w < nfull) {
            WinBuf<F, YT> b0, b1;
            XBuf<MR> x0, x1;
            load(b0, x0, w, std::false_type{});
            while (true) {
                if (w + KS < nfull) load(b1, x1, w + KS, std::false_type{});
                compute(b0, x0, w, std::false_type{});
                w += KS;
                if (w >= nfull) break;
                if (w + KS < nfull) load(b0, x0, w + KS, std::false_type{});
                compute(b1, x1, w, std::false_type{});
                w += KS;
                if (w >= nfull) break;
            }
        }
        if (K % kWindow != 0 && nfull % KS == ks) {
            WinBuf<F, YT> bt;
            XBuf<MR> xt;
            load(bt, xt, nfull, std::true_type{});
            compute(bt, xt, nfull, std::true_type{});
        }
    }

    float v[MR][YT];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int y = 0; y < YT; ++y) v[m][y] = wave_sum_to_lane63(acc[m][y]);
    if constexpr (KS == 1) {
        if (active && lane == kWave - 1) {
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int y = 0; y < YT; ++y)
                    if (m < mrows && row0 + y < N) store_out<TC>(C + static_cast<size_t>(m0 + m) * N + row0 + y, v[m][y]);
        }
    } else {
        if (lane == kWave - 1) {
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int y = 0; y < YT; ++y) red[wv][m * YT + y] = v[m][y];
        }
        __syncthreads();
        if (active && ks == 0 && lane == kWave - 1) {
#pragma unroll
            for (int m = 0; m < MR; ++m) {
#pragma unroll
                for (int y = 0; y < YT; ++y) {
                    float t = red[wv][m * YT + y];
#pragma unroll
                    for (int j = 1; j < KS; ++j) t += red[wv + j][m * YT + y];
                    if (m < mrows && row0 + y < N) store_out<TC>(C + static_cast<size_t>(m0 + m) * N + row0 + y, t);
                }
            }
        }
    }
}

// Alignment-agnostic fallback: one wave per (row n, A row m), lanes over 32-weight groups,
// byte loads.  Used when a fast-path precondition fails (unaligned W, or K not a multiple of
// 2048 for Q6_K / of 256 for Q4_0 and Q8_0).
template <int T, typename TA, typename TC>
__global__ __launch_bounds__(kWave * kWavesPerBlock)
void gemv_fallback_kernel(const TA* __restrict__ A, const uint8_t* __restrict__ W, TC* __restrict__ C,
                          int M, int N, int K) {
    const int lane = threadIdx.x & (kWave - 1);
    const int n = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
    const int m = blockIdx.y;
    if (n >= N || m >= M) return;
    const int qk = (T == QMM_TYPE_Q4_0 || T == QMM_TYPE_Q8_0) ? 32 : 256;
    const int bb = T == QMM_TYPE_Q4_0 ? kBytesQ4_0 : T == QMM_TYPE_Q8_0 ? kBytesQ8_0
                 : T == QMM_TYPE_Q4_K ? kBytesQ4_K : kBytesQ6_K;
    const uint8_t* row = W + static_cast<size_t>(n) * (K / qk) * bb;
    const TA* x = A + static_cast<size_t>(m) * K;
    const int groups = K / 32;
    float acc = 0.0f;
    for (int g = lane; g < groups; g += kWave) {
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
    acc = wave_sum_to_lane63(acc);
    if (lane == kWave - 1) store_out<TC>(C + static_cast<size_t>(m) * N + n, acc);
}

template <class F, int MR, int YT, int KS, typename TA, typename TC>
hipError_t launch_fast(const void* A, const void* W, void* C, int M, int N, int K, bool a_vec,
                       hipStream_t stream) {
    constexpr int kRowsPerBlock = (kWavesPerBlock / KS) * YT;
    const dim3 block(kWave * kWavesPerBlock);
    const dim3 grid((N + kRowsPerBlock - 1) / kRowsPerBlock, (M + MR - 1) / MR);
    hipLaunchKernelGGL((gemv_kernel<F, MR, YT, KS, TA, TC>), grid, block, 0, stream,
                       static_cast<const TA*>(A), static_cast<const uint8_t*>(W), static_cast<TC*>(C),
                       M, N, K, a_vec ? 1 : 0);
    return hipGetLastError();
}

// Rows per wave: enough waves to cover the chip several times over.
inline int pick_yt(int N) {
    if (N >= 4 * 2048) return 4;
    if (N >= 2 * 2048) return 2;
    return 1;
}

template <class F, typename TA, typename TC>
hipError_t dispatch_fast(const void* A, const void* W, void* C, int M, int N, int K, bool a_vec,
                         hipStream_t stream) {
    const int yt = pick_yt(N);
    if (M == 1) {
        switch (yt) {
            case 4: return launch_fast<F, 1, 4, 1, TA, TC>(A, W, C, M, N, K, a_vec, stream);
            case 2: return launch_fast<F, 1, 2, 1, TA, TC>(A, W, C, M, N, K, a_vec, stream);
            default: return launch_fast<F, 1, 1, 1, TA, TC>(A, W, C, M, N, K, a_vec, stream);
        }
    }
    if (M == 2) {
        switch (yt) {
            case 4: return launch_fast<F, 2, 4, 1, TA, TC>(A, W, C, M, N, K, a_vec, stream);
            case 2: return launch_fast<F, 2, 2, 1, TA, TC>(A, W, C, M, N, K, a_vec, stream);
            default: return launch_fast<F, 2, 1, 1, TA, TC>(A, W, C, M, N, K, a_vec, stream);
        }
    }
    switch (yt) {
        case 4: return launch_fast<F, 4, 4, 1, TA, TC>(A, W, C, M, N, K, a_vec, stream);
        case 2: return launch_fast<F, 4, 2, 1, TA, TC>(A, W, C, M, N, K, a_vec, stream);
        default: return launch_fast<F, 4, 1, 1, TA, TC>(A, W, C, M, N, K, a_vec, stream);
    }
}

template <int T, typename TA, typename TC>
hipError_t launch_fallback(const void* A, const void* W, void* C, int M, int N, int K, hipStream_t stream) {
    const dim3 block(kWave * kWavesPerBlock);
    const dim3 grid((N + kWavesPerBlock - 1) / kWavesPerBlock, M);
    hipLaunchKernelGGL((gemv_fallback_kernel<T, TA, TC>), grid, block, 0, stream,
                       static_cast<const TA*>(A), static_cast<const uint8_t*>(W), static_cast<TC*>(C),
                       M, N, K);
    return hipGetLastError();
}

template <typename TA, typename TC>
hipError_t dispatch_types(int t, const void* A, const void* W, void* C, int M, int N, int K,
                          hipStream_t stream) {
    // Fast-path preconditions: 16-byte aligned packed rows, and a weight matrix below
    // 4 GiB so per-lane byte offsets fit 32 bits.
    const uint64_t total = static_cast<uint64_t>(N) * static_cast<uint64_t>(K / block_elems(t)) *
                           static_cast<uint64_t>(block_bytes(t));
    const bool w_aligned = (reinterpret_cast<uintptr_t>(W) & 15u) == 0 && total < (1ull << 32);
    const bool a_vec = (reinterpret_cast<uintptr_t>(A) & 15u) == 0;
    switch (t) {
        case QMM_TYPE_Q4_K:
            if (w_aligned) return dispatch_fast<FmtQ4K, TA, TC>(A, W, C, M, N, K, a_vec, stream);
            return launch_fallback<QMM_TYPE_Q4_K, TA, TC>(A, W, C, M, N, K, stream);
        case QMM_TYPE_Q6_K:
            if (w_aligned && K % 2048 == 0) return dispatch_fast<FmtQ6K, TA, TC>(A, W, C, M, N, K, a_vec, stream);
            return launch_fallback<QMM_TYPE_Q6_K, TA, TC>(A, W, C, M, N, K, stream);
        case QMM_TYPE_Q8_0:
            if (w_aligned && K % 256 == 0) return dispatch_fast<FmtQ80, TA, TC>(A, W, C, M, N, K, a_vec, stream);
            return launch_fallback<QMM_TYPE_Q8_0, TA, TC>(A, W, C, M, N, K, stream);
        case QMM_TYPE_Q4_0:
            if (w_aligned && K % 256 == 0) return dispatch_fast<FmtQ40, TA, TC>(A, W, C, M, N, K, a_vec, stream);
            return launch_fallback<QMM_TYPE_Q4_0, TA, TC>(A, W, C, M, N, K, stream);
        default:
            return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_gemv(int ggml_type, const void* A, int a_dtype, const void* W, void* C,
                       int c_dtype, int M, int N, int K, hipStream_t stream) {
    if (a_dtype == QMM_DTYPE_F32) {
        if (c_dtype == QMM_DTYPE_F32) return dispatch_types<float, float>(ggml_type, A, W, C, M, N, K, stream);
        return dispatch_types<float, __half>(ggml_type, A, W, C, M, N, K, stream);
    }
    if (c_dtype == QMM_DTYPE_F32) return dispatch_types<__half, float>(ggml_type, A, W, C, M, N, K, stream);
    return dispatch_types<__half, __half>(ggml_type, A, W, C, M, N, K, stream);
}

}  // namespace qmm
