// Prefill GEMM (M >= gemv_max_m(), 17 by default): C[M, N] = A[M, K] @ dequant(W)[N, K]^T on f16 MFMA with fp32
// accumulation.  Replaces the reference's TILE_M = 4 "prefill" kernels
// (src/kernels/dequantize.hip:152-210, 279-332, 440-505, 616-685), which re-read and re-decode
// every weight for each group of 4 activation rows on the vector ALUs.
//
// MI355X design:
//   * Operands are f16 (v_mfma_f32_32x32x16_f16, fp32 accumulation).  The reference's API hands
//     over fp16 activations; f16 keeps three more mantissa bits than bf16 at the same MFMA rate.
//     fp32 activations are rounded to f16 once by a conversion pass into a workspace.
//   * A workgroup (8 waves, two per SIMD, so one wave's memory stalls are covered by the other's
//     MFMAs) owns a 128 (m) x 256 (n) output tile and walks its K range in steps of 256 (one
//     Q4_K / Q6_K super-block per weight row, so each row's bytes arrive in one batch); wave w
//     owns weight rows [32w, 32w + 32) of the tile and all 128 activation rows (4 MFMA tiles of
//     32 x 32, fp32 accumulators).
//   * M <= 32 (from the default threshold of 17 up): the same kernel with a 32-row activation tile, one MFMA
//     tile per wave; its smaller register and LDS footprint fits two workgroups per CU.
//   * Activation tiles (128 x 256 f16, 64 KiB) are double-buffered in LDS: the next step's tile
//     is loaded into registers during the current step and written to the free slot near its end
//     (one barrier per step).
//     Rows are XOR-swizzled so fragment reads are bank-conflict free.
//   * Each wave dequantizes its own weight rows straight into MFMA fragments with packed f16
//     math: one v_perm makes two (1024 + code) f16 values, v_pk_add_f16 removes the offset
//     exactly, v_pk_fma_f16 applies the group's scale and min (one rounding to f16).  Raw
//     bytes are loaded one step ahead.
//   * A step is software-pipelined in sixteen sub-steps of one 16-k MFMA block: while a sub-step's
//     MFMAs run, the wave reads the next sub-step's activation fragments from LDS and
//     dequantizes its weight fragment.
//   * Narrow N (few tiles): the K range is split over workgroups; partial tiles land in a
//     workspace and a second pass adds them in a fixed order (deterministic).
//   * Tiles sharing a weight slice are placed on the same XCD (L2 reuse of the packed bytes).
#include <climits>
#include <mutex>
#include <string>
#include <type_traits>
#include <utility>
#include <unordered_map>

#include "qmm_device.h"

namespace qmm {
namespace {

// VALU operations per MFMA round of the 256 x 256 tile's schedule.
constexpr int kWideValu = 4;
// The wide tile is used while its tiles cover at least 1 / kWideMin of the CUs (K is split over
// workgroups below that).
constexpr int kWideMin = 2;
// Largest M that runs the 32-row tile (one 32-row tile per weight slice when M <= 32).
constexpr int kSmallMaxM = 32;
// Workgroups of the 32-row tile per CU that its grid is split to fill.
constexpr int kSmallFill = 1;

constexpr int kBM = 128;        // activation rows per workgroup tile
constexpr int kBN = 256;        // weight rows per workgroup tile (32 per wave)
constexpr int kHalves = 4;      // 64-k halves per step for Q4_K / Q6_K (one super-block); the
                                // 32-weight block formats and F16 take 2 (fewer raw registers:
                                // measured 2-7 % faster for Q8_0 / Q4_0, no spill for F16)
constexpr int kThreads = 512;   // 8 waves: two per SIMD, so one wave's load stalls are covered
constexpr int kSmallBM = 32;    // activation rows of the small-M tile (M <= kSmallBM)

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4p __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4p ld16(const uint8_t* p) {
    u32x4p v;
    __builtin_memcpy(&v, p, 16);  // any alignment: global_load_dwordx4
    return v;
}
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}
__device__ __forceinline__ uint32_t ld2(const uint8_t* p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}

__device__ __forceinline__ h2 as_h2(uint32_t u) {
    h2 v;
    __builtin_memcpy(&v, &u, 4);
    return v;
}
__device__ __forceinline__ uint32_t as_u32(h2 v) {
    uint32_t u;
    __builtin_memcpy(&u, &v, 4);
    return u;
}
__device__ __forceinline__ h2 splat(float f) {
    const _Float16 x = static_cast<_Float16>(f);
    return h2{x, x};
}

// Four byte codes q (bytes of `x`) -> two f16 pairs (q0, q1), (q2, q3) with value (q + off), exact:
// v_perm builds (1024 + q) and v_pk_add_f16 subtracts 1024 - off.
__device__ __forceinline__ void bytes_to_h2(uint32_t x, h2 sub, h2& lo, h2& hi) {
    const uint32_t mg = 0x64006400u;
    lo = as_h2(__builtin_amdgcn_perm(mg, x, 0x07010500u)) - sub;
    hi = as_h2(__builtin_amdgcn_perm(mg, x, 0x07030502u)) - sub;
}

// fragment dword from two f16 pairs: (w0, w1) = c * a + b, one rounding (v_pk_fma_f16)
__device__ __forceinline__ uint32_t affine(h2 c, h2 a, h2 b) { return as_u32(__builtin_elementwise_fma(c, a, b)); }

// ---------------------------------------------------------------------------------------------
// Weight producers, for steps of H halves of 64 k (H = 4: one Q4_K / Q6_K super-block or eight
// Q4_0 / Q8_0 blocks per step; H = 2: half of that).  A step runs 4H sub-steps (U, S), U < H,
// S = 0..3, of one MFMA k-block (16 k) each; in sub-step (U, S), lane half h covers
// k = 64U + 32*(S>>1) + 16*h + 8*(S&1) + (0..7) of the step.
//   load()        one weight row's raw bytes for the whole step (issued a step ahead);
//   scales<U>()   the f16 scale (and offset) pairs of half U's two 32-weight groups;
//   frag<U, S>()  the MFMA fragment (8 f16, natural k order) of sub-step (U, S).
// kv = K - k0 lets the 32-weight formats zero a K tail; the zeroing happens in scales(), so no
// prefetched value is consumed before its sub-step.
// ---------------------------------------------------------------------------------------------
template <int H>
struct PQ4K {
    static constexpr int kH = H;
    static_assert(H == 2 || H == 4, "steps of 128 or 256 k");
    static constexpr int kQK = kQK_K, kBytes = kBytesQ4_K;
    struct Raw { u32x4p hd, q[H]; };
    struct Sc { h2 a0, b0, a1, b1; };
    // step at k0 (multiple of 64H): super-block k0/256, qs chunks c = c0 + U with c0 = (k0/64)%4
    // (always 0 when H = 4); lane half h takes qs bytes 16h..16h+15 of chunk c (low nibbles:
    // sub-block 2c, high: 2c+1).
    __device__ static void prep(Raw&, int) {}
    __device__ static Raw load(const uint8_t* row, int k0, int h, int, int) {
        const uint8_t* sb = row + static_cast<size_t>(k0 >> 8) * kBytes;
        const int c0 = H == 4 ? 0 : ((k0 >> 6) & 2);
        Raw r;
        r.hd = *reinterpret_cast<const u32x4p*>(sb);
#pragma unroll
        for (int c = 0; c < H; ++c) r.q[c] = *reinterpret_cast<const u32x4p*>(sb + 16 + 32 * (c0 + c) + 16 * h);
        return r;
    }
    template <int U>
    __device__ static Sc scales(const Raw& r, int k0, int, int) {
        // 6-bit scales/mins of sub-blocks 2c and 2c + 1: bytes 2(c&1), 2(c&1)+1 of the packed
        // scale words; sub-blocks 4..7 (c >= 2) take their top bits from words 0/1.  With H = 2
        // the choice is uniform over the step, so it is a select, not a branch.
        constexpr int sh = 16 * (U & 1);
        const uint32_t u0 = r.hd.y >> sh, u1 = r.hd.z >> sh, u2 = r.hd.w >> sh;
        const uint32_t sc_lo = u0 & 0x3F3Fu, m_lo = u1 & 0x3F3Fu;
        const uint32_t sc_hi = (u2 & 0x0F0Fu) | ((u0 >> 2) & 0x3030u);
        const uint32_t m_hi = ((u2 >> 4) & 0x0F0Fu) | ((u1 >> 2) & 0x3030u);
        uint32_t scp, mp;
        if constexpr (H == 4) {
            scp = U < 2 ? sc_lo : sc_hi;
            mp = U < 2 ? m_lo : m_hi;
        } else {
            const bool upper = ((k0 >> 6) & 2) != 0;
            scp = upper ? sc_hi : sc_lo;
            mp = upper ? m_hi : m_lo;
        }
        const float d = half_bits_to_float(r.hd.x), dmin = half_bits_to_float(r.hd.x >> 16);
        Sc s;
        s.a0 = splat(d * static_cast<float>(scp & 0xFFu));
        s.b0 = splat(-(dmin * static_cast<float>(mp & 0xFFu)));
        s.a1 = splat(d * static_cast<float>((scp >> 8) & 0xFFu));
        s.b1 = splat(-(dmin * static_cast<float>((mp >> 8) & 0xFFu)));
        return s;
    }
    template <int U, int S>
    __device__ static void frag(const Raw& r, const Sc& sc, int, uint32_t f[4]) {
        constexpr bool hi = S >= 2;  // high nibbles: sub-block 2c + 1
        const u32x4p q = r.q[U];
        const uint32_t w[2] = {(S & 1) ? q.z : q.x, (S & 1) ? q.w : q.y};
        const h2 off = splat(1024.0f);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t codes = hi ? ((w[j] >> 4) & 0x0F0F0F0Fu) : (w[j] & 0x0F0F0F0Fu);
            h2 p, qq;
            bytes_to_h2(codes, off, p, qq);
            f[2 * j] = affine(p, hi ? sc.a1 : sc.a0, hi ? sc.b1 : sc.b0);
            f[2 * j + 1] = affine(qq, hi ? sc.a1 : sc.a0, hi ? sc.b1 : sc.b0);
        }
    }
};

template <int H>
struct PQ6K {
    static constexpr int kH = H;
    static_assert(H == 2 || H == 4, "steps of 128 or 256 k");
    static constexpr int kQK = kQK_K, kBytes = kBytesQ6_K;
    struct Raw {
        u32x4p la[H / 2], lb[H / 2], qh[H / 2], s;  // ql / qh slices, sub-scales (H = 2: s.x, s.y)
        uint32_t tail, d;                          // the dword after s (f = 2), d
        int f;                                     // byte shift: 0 or 2, uniform over the wave
    };
    struct Sc { h2 a0, a1; };
    // step at k0 (multiple of 64H): super-block k0/256.  Half U covers the block's 64-weight
    // quarter 2*n2 + (U&1) of 128-weight half n2 = U>>1 (H = 4) or (k0/128)%2 (H = 2), groups
    // t = 2(U&1) + (S>>1).  Lane half h takes l = 16h..16h+15 of ql (groups t even: ql[64n2 + l],
    // odd: ql[64n2 + 32 + l]; U&1 picks the nibble) and of qh[32n2 + l]; sub-scale word U holds
    // sc[8n2 + 4(U&1) + (0..3)].
    //
    // Alignment (256-k steps): a 210-byte block starts 2 bytes off a 4-byte boundary when its
    // index is odd (with 4-aligned rows), and 16-byte loads at such addresses measured 16 %
    // slower over a whole launch (8B down at M = 512).  For those blocks every slice is loaded
    // from 2 bytes lower (f = 2, 4-aligned) and prep() shifts it back: dword k of a slice is
    // bytes 2..3 of loaded dword k and bytes 0..1 of dword k + 1, the last one taken from the
    // slice that follows in memory (the other lane half's register, fetched with
    // v_permlane32_swap, or `tail`).  With al == 0 (rows not 4-aligned) blocks are read as they lie.
    __device__ static Raw load(const uint8_t* row, int k0, int h, int, int al) {
        const uint8_t* sb = row + static_cast<size_t>(k0 >> 8) * kBytes;
        Raw r;
        if constexpr (H == 2) {
            // 128-k steps (256 x 256 tile): blocks are read as they lie; the realignment's extra
            // loads and shifts measured 7 % slower in this one-wave-per-SIMD tile.
            const int nb = (k0 >> 7) & 1;
            r.la[0] = ld16(sb + 64 * nb + 16 * h);
            r.lb[0] = ld16(sb + 64 * nb + 32 + 16 * h);
            r.qh[0] = ld16(sb + 128 + 32 * nb + 16 * h);
            r.s.x = ld4(sb + 192 + 8 * nb);
            r.s.y = ld4(sb + 196 + 8 * nb);
            r.s.z = r.s.w = r.tail = 0u;
            r.f = 0;
        } else {
            const int f = al && ((k0 >> 8) & 1) ? 2 : 0;
            const uint8_t* sf = sb - f;  // in bounds: f = 2 only for blocks with an odd index
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                r.la[j] = ld16(sf + 64 * j + 16 * h);
                r.lb[j] = ld16(sf + 64 * j + 32 + 16 * h);
                r.qh[j] = ld16(sf + 128 + 32 * j + 16 * h);
            }
            r.s = ld16(sf + 192);
            r.tail = ld4(sb + 204 + f);  // f = 2: bytes 206..209 (after s); f = 0: unused
            r.f = f;
        }
        r.d = ld2(sb + 208);
        return r;
    }
    // Realigns a 256-k step's slices (f = 2) once its loads have landed; f is uniform over the
    // wave, so this is a branch, not a select.
    __device__ static void prep(Raw& r, int h) {
        if constexpr (H == 4) {
            if (r.f != 0) {
                // nx(R): the dword after slice R in memory.  Lane half 0's slice R is followed by
                // half 1's R; half 1's by half 0's next slice (la0 lb0 la1 lb1 qh0 qh1 s, s
                // loaded by both halves).  swap(a, b) gives lanes 0..31 lane l + 32's a and lanes
                // 32..63 lane l - 32's b.
                auto nextof = [&](uint32_t a, uint32_t b) {
                    const auto sw = __builtin_amdgcn_permlane32_swap(a, b, false, false);
                    return h ? static_cast<uint32_t>(sw[0]) : static_cast<uint32_t>(sw[1]);
                };
                auto fix = [](u32x4p& v, uint32_t nx) {
                    const u32x4p o = v;
                    v.x = __builtin_amdgcn_alignbyte(o.y, o.x, 2);
                    v.y = __builtin_amdgcn_alignbyte(o.z, o.y, 2);
                    v.z = __builtin_amdgcn_alignbyte(o.w, o.z, 2);
                    v.w = __builtin_amdgcn_alignbyte(nx, o.w, 2);
                };
                const uint32_t n0 = nextof(r.la[0].x, r.lb[0].x), n1 = nextof(r.lb[0].x, r.la[1].x);
                const uint32_t n2 = nextof(r.la[1].x, r.lb[1].x), n3 = nextof(r.lb[1].x, r.qh[0].x);
                const uint32_t n4 = nextof(r.qh[0].x, r.qh[1].x), n5 = nextof(r.qh[1].x, r.s.x);
                fix(r.la[0], n0);
                fix(r.lb[0], n1);
                fix(r.la[1], n2);
                fix(r.lb[1], n3);
                fix(r.qh[0], n4);
                fix(r.qh[1], n5);
                fix(r.s, r.tail);
            }
        }
    }
    template <int U>
    __device__ static Sc scales(const Raw& r, int, int h, int) {
        // sub-scales of word U, bytes h and h + 2
        const uint32_t sc = U == 0 ? r.s.x : U == 1 ? r.s.y : U == 2 ? r.s.z : r.s.w;
        const float d = half_bits_to_float(r.d);
        Sc s;
        s.a0 = splat(d * static_cast<float>(static_cast<int8_t>(sc >> (8 * h))));
        s.a1 = splat(d * static_cast<float>(static_cast<int8_t>(sc >> (8 * h + 16))));
        return s;
    }
    template <int U, int S>
    __device__ static void frag(const Raw& r, const Sc& sc, int, uint32_t f[4]) {
        constexpr int j = U >> 1, nib = 4 * (U & 1), u = S >> 1;  // group t = 2(U&1) + u
        constexpr int hs = nib + 2 * u;                             // qh bit pair of the group
        const u32x4p l = u ? r.lb[j] : r.la[j];
        const u32x4p qh = r.qh[j];
        const uint32_t lw[2] = {(S & 1) ? l.z : l.x, (S & 1) ? l.w : l.y};
        const uint32_t hw[2] = {(S & 1) ? qh.z : qh.x, (S & 1) ? qh.w : qh.y};
        const h2 off = splat(1056.0f);  // 1024 + 32: codes q enter as 1024 + q, weight is a (q - 32)
        const h2 a = u ? sc.a1 : sc.a0;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const uint32_t lo4 = (lw[jj] >> nib) & 0x0F0F0F0Fu;
            const uint32_t hi2 = ((hw[jj] >> hs) & 0x03030303u) << 4;
            h2 p, q;
            bytes_to_h2(lo4 | hi2, off, p, q);
            f[2 * jj] = as_u32(p * a);
            f[2 * jj + 1] = as_u32(q * a);
        }
    }
};

// 32-weight block formats: a step covers blocks k0/32 + b, b < 2H (block b absent when
// kv <= 32b: load() clamps its address to block 0 and scales() zeroes its scale).  Half U
// holds blocks 2U (S = 0, 1) and 2U + 1 (S = 2, 3).
template <int H>
struct PQ80 {
    static constexpr int kH = H;
    static constexpr int kQK = kQK8_0, kBytes = kBytesQ8_0;
    struct Raw { u32x4p q[2 * H]; uint32_t d[2 * H]; };
    struct Sc { h2 a0, a1; };
    __device__ static void prep(Raw&, int) {}
    __device__ static Raw load(const uint8_t* row, int k0, int h, int kv, int) {
        const uint8_t* b0 = row + static_cast<size_t>(k0 >> 5) * kBytes;
        Raw r;
#pragma unroll
        for (int b = 0; b < 2 * H; ++b) {
            const uint8_t* bb = kv > 32 * b ? b0 + b * kBytes : b0;
            r.q[b] = ld16(bb + 2 + 16 * h);
            r.d[b] = ld2(bb);  // always issued (static load count)
        }
        return r;
    }
    template <int U>
    __device__ static Sc scales(const Raw& r, int, int, int kv) {
        Sc s;
        s.a0 = splat(half_bits_to_float(kv > 64 * U ? r.d[2 * U] : 0u));
        s.a1 = splat(half_bits_to_float(kv > 64 * U + 32 ? r.d[2 * U + 1] : 0u));
        return s;
    }
    template <int U, int S>
    __device__ static void frag(const Raw& r, const Sc& sc, int, uint32_t f[4]) {
        constexpr int u = S >> 1;
        const u32x4p q = r.q[2 * U + u];
        const uint32_t w[2] = {(S & 1) ? q.z : q.x, (S & 1) ? q.w : q.y};
        const h2 off = splat(1152.0f);  // signed codes enter as 1024 + (q + 128)
        const h2 a = u ? sc.a1 : sc.a0;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            h2 p, qq;
            bytes_to_h2(w[j] ^ 0x80808080u, off, p, qq);
            f[2 * j] = as_u32(p * a);
            f[2 * j + 1] = as_u32(qq * a);
        }
    }
};

template <int H>
struct PQ40 {
    static constexpr int kH = H;
    static constexpr int kQK = kQK4_0, kBytes = kBytesQ4_0;
    struct Raw { u32x4p q[2 * H]; uint32_t d[2 * H]; };
    struct Sc { h2 a0, a1; };
    // lane half h takes the block's low (h = 0, k 0..15) or high (h = 1, k 16..31) nibbles.
    __device__ static void prep(Raw&, int) {}
    __device__ static Raw load(const uint8_t* row, int k0, int, int kv, int) {
        const uint8_t* b0 = row + static_cast<size_t>(k0 >> 5) * kBytes;
        Raw r;
#pragma unroll
        for (int b = 0; b < 2 * H; ++b) {
            const uint8_t* bb = kv > 32 * b ? b0 + b * kBytes : b0;
            r.q[b] = ld16(bb + 2);
            r.d[b] = ld2(bb);  // always issued (static load count)
        }
        return r;
    }
    template <int U>
    __device__ static Sc scales(const Raw& r, int, int, int kv) {
        Sc s;
        s.a0 = splat(half_bits_to_float(kv > 64 * U ? r.d[2 * U] : 0u));
        s.a1 = splat(half_bits_to_float(kv > 64 * U + 32 ? r.d[2 * U + 1] : 0u));
        return s;
    }
    template <int U, int S>
    __device__ static void frag(const Raw& r, const Sc& sc, int h, uint32_t f[4]) {
        constexpr int u = S >> 1;
        const u32x4p q = r.q[2 * U + u];
        const uint32_t w[2] = {(S & 1) ? q.z : q.x, (S & 1) ? q.w : q.y};
        const h2 off = splat(1032.0f);  // codes enter as 1024 + q, weight is d (q - 8)
        const h2 a = u ? sc.a1 : sc.a0;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            h2 p, qq;
            bytes_to_h2((w[j] >> (4 * h)) & 0x0F0F0F0Fu, off, p, qq);
            f[2 * j] = as_u32(p * a);
            f[2 * j + 1] = as_u32(qq * a);
        }
    }
};

// F16 (dense fp16 rows, the operand of the reference's matmul_nt): a lane loads the 8 weights
// of each of its sub-steps straight into the fragment (natural k order, no conversion).  Needs
// K % 8 == 0: a chunk is wholly inside K or wholly outside it; one outside reads the row's first
// bytes (a valid address) and is zeroed in scales(), when its sub-step comes.
template <int H>
struct PF16 {
    static constexpr int kH = H;
    static constexpr int kQK = 8, kBytes = 16;  // row bytes = K / 8 * 16 = 2K
    struct Raw { u32x4p w[H][4]; };
    struct Sc { uint32_t keep[4]; };
    __device__ static constexpr int off(int U, int S, int h) { return 64 * U + 32 * (S >> 1) + 16 * h + 8 * (S & 1); }
    __device__ static void prep(Raw&, int) {}
    __device__ static Raw load(const uint8_t* row, int k0, int h, int kv, int) {
        Raw r;
#pragma unroll
        for (int U = 0; U < H; ++U)
#pragma unroll
            for (int S = 0; S < 4; ++S) {
                const int o = off(U, S, h);
                r.w[U][S] = ld16(row + 2 * static_cast<size_t>(o < kv ? k0 + o : 0));
            }
        return r;
    }
    template <int U>
    __device__ static Sc scales(const Raw&, int, int h, int kv) {
        Sc s;
#pragma unroll
        for (int S = 0; S < 4; ++S) s.keep[S] = off(U, S, h) < kv ? 0xFFFFFFFFu : 0u;
        return s;
    }
    template <int U, int S>
    __device__ static void frag(const Raw& r, const Sc& sc, int, uint32_t f[4]) {
        const u32x4p w = r.w[U][S];
        f[0] = w.x & sc.keep[S];
        f[1] = w.y & sc.keep[S];
        f[2] = w.z & sc.keep[S];
        f[3] = w.w & sc.keep[S];
    }
};

// Output segments of one launch: consecutive weight matrices that multiply the same activations
// (q/k/v, gate/up).  Their n-tiles are concatenated; tile_end[s] is the cumulative n-tile count
// through segment s (INT_MAX for unused entries), part_off[s] the offset of segment s's split-K
// partial block ([ksplit][M][N_s] fp32) in the partial workspace.  Segment s computes columns
// [0, N_s) of a C block whose rows are ldc[s] elements apart (a column range of a wider C when
// a launch covers only some of a matrix's rows).
constexpr int kPfMaxSegs = 4;
template <typename TC>
struct PfSegs {
    const uint8_t* W[kPfMaxSegs];
    TC* C[kPfMaxSegs];
    int N[kPfMaxSegs];
    int ldc[kPfMaxSegs];
    int tile_end[kPfMaxSegs];
    size_t part_off[kPfMaxSegs];
    const float* rs;  // per activation row output factor (a power of two), or nullptr
};

// Segment of the workgroup's n-tile tn (uniform), and tn's index inside that segment.
template <typename TC>
__device__ __forceinline__ int pf_seg_of(const PfSegs<TC>& sg, int& tn) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < kPfMaxSegs - 1; ++i) s += tn >= sg.tile_end[i] ? 1 : 0;
    if (s > 0) tn -= sg.tile_end[s - 1];
    return s;
}

// Activation chunk (row r, chunk c = 8 f16) position inside a 1024-chunk half stage: rows are
// XOR-swizzled so that 16 consecutive rows read at one chunk hit 16 different bank groups.
__device__ __forceinline__ int a_slot(int r, int c) { return 8 * r + (c ^ ((r >> 1) & 7)); }

// Sub-step S, lane half h -> activation chunk of the half stage.
__device__ __forceinline__ int a_chunk(int s, int h) { return 4 * (s >> 1) + 2 * h + (s & 1); }

// Four consecutive outputs n..n+3 of row m (n a multiple of 4) from a wave's accumulators: one
// 16-byte (fp32) or 8-byte (fp16) store when all four exist and the address is aligned for it,
// element stores otherwise.  With K split, the fp32 partial tile `ksplit` block kz instead.
template <typename TC>
__device__ __forceinline__ void store_quad(TC* __restrict__ C, float* __restrict__ part, int ksplit, int kz, int M, int N,
                                           int ldc, int m, int n, const float (&vs)[4]) {
    if (ksplit > 1) {
        float* dst = part + (static_cast<size_t>(kz) * M + m) * N + n;
        if (n + 3 < N && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
            *reinterpret_cast<float4*>(dst) = make_float4(vs[0], vs[1], vs[2], vs[3]);
            return;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (n + e < N) dst[e] = vs[e];
        return;
    }
    TC* dst = C + static_cast<size_t>(m) * ldc + n;
    if constexpr (sizeof(TC) == 4) {
        if (n + 3 < N && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
            *reinterpret_cast<float4*>(dst) = make_float4(vs[0], vs[1], vs[2], vs[3]);
            return;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (n + e < N) reinterpret_cast<float*>(dst)[e] = vs[e];
    } else {
        if (n + 3 < N && (reinterpret_cast<uintptr_t>(dst) & 7u) == 0) {
            *reinterpret_cast<uint2*>(dst) = make_uint2(float_to_half_bits(vs[0]) | (float_to_half_bits(vs[1]) << 16),
                                                        float_to_half_bits(vs[2]) | (float_to_half_bits(vs[3]) << 16));
            return;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (n + e < N) reinterpret_cast<uint16_t*>(dst)[e] = float_to_half_bits(vs[e]);
    }
}

// Workgroup barrier for LDS traffic only: this wave's LDS operations are complete, then
// s_barrier.  Unlike __syncthreads() it does not wait for outstanding global loads (the
// prefetches stay in flight); the empty asm statements keep the compiler from moving memory
// operations across it.
__device__ __forceinline__ void lds_barrier() {
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

// Instruction interleave of one sub-step for the scheduler: four rounds of one MFMA, one LDS read
// and a few VALU operations, so the dequantization of the next sub-step runs while the matrix
// core works on this one.
template <int V>
__device__ __forceinline__ void interleave_substep() {
#define QMM_PF_ROUND                                   \
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); \
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); \
    __builtin_amdgcn_sched_group_barrier(0x002, V, 0);
    QMM_PF_ROUND QMM_PF_ROUND QMM_PF_ROUND QMM_PF_ROUND
#undef QMM_PF_ROUND
}

// f(integral_constant<int, Q>) for Q = 0, 1, ... in order (compile-time sub-step indices).
template <class F, int... Q>
__device__ __forceinline__ void for_each_index(F& f, std::integer_sequence<int, Q...>) {
    (f(std::integral_constant<int, Q>{}), ...);
}

// BM = 128 (kBM) or 32 (kSmallBM: one MFMA tile of activation rows per wave, for M <= 32, where
// the 128-row tile would spend three quarters of its matrix-core work on padding rows; the
// smaller tile's registers and LDS let two workgroups share a CU).
template <class P, typename TC, int BM>
__global__ __launch_bounds__(kThreads, BM == kBM ? 1 : 2)
void prefill_kernel(const _Float16* __restrict__ A16, int lda, PfSegs<TC> sg, float* __restrict__ part_base, int M, int K,
                    int klen, int tiles_m, int tiles_n, int ksplit) {
    constexpr int kH = P::kH;      // 64-k halves per step
    constexpr int kBK = 64 * kH;   // k per step
    constexpr int NI = BM / 32;    // 32 x 32 MFMA tiles of activation rows per wave
    constexpr int CPH = BM * 8;    // 16-byte chunks (8 f16) per 64-k half stage
    constexpr int NJ = CPH >= kThreads ? CPH / kThreads : 1;  // chunks per thread and half
    constexpr int kAThreads = CPH >= kThreads ? kThreads : CPH;  // threads that stage chunks
    static_assert(BM % 32 == 0 && (CPH % kThreads == 0 || kThreads % CPH == 0), "tile shape");
    __shared__ __align__(16) u32x4p sA[2][kH * CPH];

    // Tile order: m fastest, then n-tile, then k split; blocks sharing a weight slice (same
    // n-tile and k range, different m) are consecutive and dealt to one XCD.
    const int tiles = tiles_m * tiles_n * ksplit;
    int b = blockIdx.x;
    if (tiles % 8 == 0) b = (b % 8) * (tiles / 8) + b / 8;
    const int tm = b % tiles_m;
    int tn = (b / tiles_m) % tiles_n;
    const int kz = b / (tiles_m * tiles_n);
    const int sgi = pf_seg_of(sg, tn);
    const uint8_t* __restrict__ W = sg.W[sgi];
    TC* __restrict__ C = sg.C[sgi];
    const int N = sg.N[sgi];
    const int ldc = sg.ldc[sgi];
    float* __restrict__ part = part_base + sg.part_off[sgi];
    const int m0 = tm * BM, n0 = tn * kBN;
    const int kb = kz * klen;
    const int kend = min(K, kb + klen);
    const int nsteps = (kend - kb + kBK - 1) / kBK;

    const int tid = threadIdx.x;
    // threads past the chunk count (small tile) load a copy of another thread's chunks, store nothing
    const bool a_owner = kAThreads == kThreads || tid < kAThreads;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const int l32 = lane & 31;

    const size_t row_bytes = static_cast<size_t>(K / P::kQK) * P::kBytes;
    const int wal = ((reinterpret_cast<uintptr_t>(W) | row_bytes) & 3) == 0;  // 4-aligned rows
    const uint8_t* wrow = W + static_cast<size_t>(min(n0 + 32 * wv + l32, N - 1)) * row_bytes;

    // Thread tid copies half-stage chunks p = tid + 512 j (j < NJ) of every half: row p >> 3,
    // chunk (p & 7) ^ swizzle, so each thread's global reads are 16-byte aligned f16 runs and
    // its LDS writes are in place.
    const _Float16* arow[NJ];
    int apos[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int p = (kAThreads == kThreads ? tid : tid % kAThreads) + kThreads * j;
        const int r = p >> 3;
        const int c = (p & 7) ^ ((r >> 1) & 7);
        arow[j] = A16 + static_cast<size_t>(min(m0 + r, M - 1)) * lda + kb + 8 * c;
        apos[j] = p;
    }
    auto load_a = [&](int t, u32x4p (&ar)[NJ * kH]) {
        const int kk = min(t, nsteps - 1) * kBK;  // past the end: re-read the last step
#pragma unroll
        for (int u = 0; u < kH; ++u)
#pragma unroll
            for (int j = 0; j < NJ; ++j) ar[NJ * u + j] = *reinterpret_cast<const u32x4p*>(arow[j] + kk + 64 * u);
    };
    auto store_a = [&](int slot, const u32x4p (&ar)[NJ * kH]) {
        if (!a_owner) return;
#pragma unroll
        for (int u = 0; u < kH; ++u)
#pragma unroll
            for (int j = 0; j < NJ; ++j) sA[slot][CPH * u + apos[j]] = ar[NJ * u + j];
    };
    auto load_raw = [&](int t, typename P::Raw& raw) {
        const int k0 = kb + min(t, nsteps - 1) * kBK;
        raw = P::load(wrow, k0, h, kend - k0, wal);
    };
    // activation fragments of sub-step (U, S) of the step held in `slot`
    auto read_a = [&](int slot, int U, int S, f16x8 (&af)[NI]) {
        const u32x4p* sa = sA[slot] + CPH * U;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const u32x4p av = sa[a_slot(32 * i + l32, a_chunk(S, h))];
            __builtin_memcpy(&af[i], &av, 16);
        }
    };

    f32x16 acc[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;

    // Software pipeline.  Step t (k0 = kb + kBK t) runs sub-steps q = 0..Q-1 (Q = 4 kH: 16 for
    // the quantized formats, 8 for F16; U = q/4, S = q%4).  While the 4 MFMAs of sub-step q run
    // on wf[q&1] / af[q&1], the wave reads the activation fragments of q+1 from LDS and
    // dequantizes its weight fragment into the other buffers.
    //   q = 0: the raw bytes of step t+1 (into `nxt`) and A(t+1) (into `an`) are requested;
    //   q = 4U+1 (U < kH-1): scales of half U+1 (from `cur`) into sc[(U+1)&1];
    //   q = Q-3: scales of the next step's half 0 (from `nxt`) into sc[0] (its last use in this
    //           step, by half kH-2's fragments, is at q = Q-6);
    //   q = Q-2: after the reads for q = Q-1, A(t+1) goes to the free LDS slot, then the barrier
    //           (after it, q = Q-1 reads the next step's first fragments from that slot);
    //   q = Q-1: fragment of the next step's (0, 0) from `nxt`; at the end `cur` takes `nxt`.
    // The LDS slot (t+1)%2 last served step t-1, whose reads all precede step t-1's barrier, so
    // one barrier per step covers both the write-after-read and the read-after-write order.
    using Raw = typename P::Raw;
    using Sc = typename P::Sc;
    u32x4p an[NJ * kH];
    Raw cur, nxt;
    Sc sc[2];          // [half]
    uint32_t wf[2][4]; // [buffer][dword]
    f16x8 af[2][NI];   // [buffer][i]

    load_raw(0, cur);
    load_a(0, an);
    store_a(0, an);
    lds_barrier();
    P::prep(cur, h);
    sc[0] = P::template scales<0>(cur, kb, h, kend - kb);
    P::template frag<0, 0>(cur, sc[0], h, wf[0]);
    read_a(0, 0, 0, af[0]);

    for (int t = 0; t < nsteps; ++t) {
        const int k0 = kb + t * kBK;
        const int slot = t & 1;
        // raw bytes first: they are consumed (q = 13) before A(t+1) is (q = 14)
        load_raw(t + 1, nxt);
        load_a(t + 1, an);
        __builtin_amdgcn_sched_barrier(0);

        constexpr int kQ = 4 * kH;  // sub-steps per step
        auto sub = [&](auto qc) {
            constexpr int q = decltype(qc)::value;
            constexpr int U = q >> 2, B = q & 1;
            constexpr int qn = q + 1, Un = qn >> 2, Sn = qn & 3;
            if constexpr (qn < kQ) read_a(slot, Un, Sn, af[B ^ 1]);
            if constexpr (q == kQ - 2) {
                // free slot <- A(t+1).  The barrier comes after the last reads of this step's slot
                // (those of the last sub-step, just issued), so the next step may overwrite it.
                store_a(slot ^ 1, an);
                lds_barrier();
            }
            if constexpr (qn == kQ) read_a(slot ^ 1, 0, 0, af[B ^ 1]);
            if constexpr ((q & 3) == 1 && U + 1 < kH)
                sc[(U + 1) & 1] = P::template scales<(U + 1) % kH>(cur, k0, h, kend - k0);
            if constexpr (q == kQ - 3) {
                P::prep(nxt, h);
                sc[0] = P::template scales<0>(nxt, k0 + kBK, h, kend - k0 - kBK);
            }
            if constexpr (qn < kQ) P::template frag<Un % kH, Sn>(cur, sc[Un & 1], h, wf[B ^ 1]);
            else P::template frag<0, 0>(nxt, sc[0], h, wf[B ^ 1]);
            f16x8 bw;
            __builtin_memcpy(&bw, wf[B], 16);
#pragma unroll
            for (int i = 0; i < NI; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bw, af[B][i], acc[i], 0, 0, 0);
            if constexpr (NI == 4) interleave_substep<5>();
            __builtin_amdgcn_sched_barrier(0);
        };
        for_each_index(sub, std::make_integer_sequence<int, kQ>{});
        cur = nxt;
    }

    // Output tile through LDS (both activation stages: 256 x kH x BM bytes), so that every store
    // instruction writes whole row segments: fp16 rows of 512 bytes (fp16 C), or fp32 rows of
    // 1 KiB (fp32 C; with 256-k steps only, where they fit).  Without a K split only: the split's
    // fp32 partial tiles measured no faster this way.  16-byte chunks are XOR-swizzled by row so
    // that the 32 rows one write instruction touches fall in different banks.
    constexpr bool kLdsF16 = sizeof(TC) == 2;
    constexpr bool kLdsF32 = sizeof(TC) == 4 && kH == 4;
    if ((kLdsF16 || kLdsF32) && ksplit == 1) {
        constexpr bool f16 = kLdsF16;
        __syncthreads();  // every wave is done with the activation stages
        uint8_t* const st = reinterpret_cast<uint8_t*>(&sA[0][0]);
        constexpr int rowb = f16 ? 512 : 1024;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int m = 32 * i + l32;
            const float sm = sg.rs != nullptr && m0 + m < M ? sg.rs[m0 + m] : 1.0f;
            uint8_t* const row = st + m * rowb;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = 32 * wv + 8 * g + 4 * h;  // tile-local, multiple of 4
                const float v0 = acc[i][4 * g] * sm, v1 = acc[i][4 * g + 1] * sm;
                const float v2 = acc[i][4 * g + 2] * sm, v3 = acc[i][4 * g + 3] * sm;
                if constexpr (f16) {
                    const uint32_t w0 = float_to_half_bits(v0) | (static_cast<uint32_t>(float_to_half_bits(v1)) << 16);
                    const uint32_t w1 = float_to_half_bits(v2) | (static_cast<uint32_t>(float_to_half_bits(v3)) << 16);
                    *reinterpret_cast<uint2*>(row + (((n >> 3) ^ (m & 31)) << 4) + ((n >> 2) & 1) * 8) = make_uint2(w0, w1);
                } else {
                    *reinterpret_cast<float4*>(row + (((n >> 2) ^ (m & 31)) << 4)) = make_float4(v0, v1, v2, v3);
                }
            }
        }
        __syncthreads();
        if constexpr (f16) {
            const int c = lane & 31;  // 16-byte chunk: columns 8c .. 8c + 7
#pragma unroll
            for (int k = 0; k < BM / 16; ++k) {  // two rows per instruction, BM / 8 rows per wave
                const int m = (BM / 8) * wv + 2 * k + (lane >> 5);
                const uint4 v = *reinterpret_cast<const uint4*>(st + m * 512 + ((c ^ (m & 31)) << 4));
                const int gm = m0 + m, gn = n0 + 8 * c;
                if (gm >= M || gn >= N) continue;
                uint16_t* dst = reinterpret_cast<uint16_t*>(C) + static_cast<size_t>(gm) * ldc + gn;
                if (gn + 7 < N && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
                    *reinterpret_cast<uint4*>(dst) = v;
                } else {
                    const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (gn + e < N) dst[e] = static_cast<uint16_t>(vw[e >> 1] >> (16 * (e & 1)));
                }
            }
        } else {
            const int c = lane;  // 16-byte chunk: columns 4c .. 4c + 3
#pragma unroll
            for (int k = 0; k < BM / 8; ++k) {  // one row per instruction
                const int m = (BM / 8) * wv + k;
                const float4 v = *reinterpret_cast<const float4*>(st + m * 1024 + ((c ^ (m & 31)) << 4));
                const int gm = m0 + m, gn = n0 + 4 * c;
                if (gm >= M || gn >= N) continue;
                float* dst = reinterpret_cast<float*>(C) + static_cast<size_t>(gm) * ldc + gn;
                if (gn + 3 < N && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
                    *reinterpret_cast<float4*>(dst) = v;
                } else {
                    const float vf[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (gn + e < N) dst[e] = vf[e];
                }
            }
        }
        return;
    }

    // D element v of tile i: weight row n = n0 + 32wv + 8(v/4) + 4h + v%4, activation row
    // m = m0 + 32i + l32.
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int m = m0 + 32 * i + l32;
        if (m >= M) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n = n0 + 32 * wv + 8 * g + 4 * h;
            const float sm = sg.rs != nullptr ? sg.rs[m] : 1.0f;
            const float vs[4] = {acc[i][4 * g] * sm, acc[i][4 * g + 1] * sm, acc[i][4 * g + 2] * sm, acc[i][4 * g + 3] * sm};
            store_quad<TC>(C, part, ksplit, kz, M, N, ldc, m, n, vs);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Wide tile for M >= 256: one wave per SIMD, each wave owns 64 weight rows x 256 activation rows
// (16 MFMA tiles of 32 x 32, 256 fp32 accumulators in the AGPR file).  Every dequantized weight
// fragment feeds 8 MFMAs and every activation fragment read from LDS feeds 2, so a sub-step
// issues 16 MFMAs (512 matrix-core cycles) against ~40 VALU and 8 LDS reads: the dequantization
// and the LDS traffic hide under the matrix core within one wave instead of depending on two
// waves interleaving.
//   * Workgroup: 4 waves, tile 256 (m) x 256 (n); steps of 128 k (H = 2 producer halves).
//   * Activation tile of a step: 256 x 128 f16 = 64 KiB, double-buffered in LDS (128 KiB).  The
//     next step's tile is requested at the start of the current step with direct global -> LDS
//     loads (no staging registers, no LDS write instructions); one barrier per step.
//   * Raw weight bytes of the next step (two rows per lane) are loaded at the start of a step.
// ---------------------------------------------------------------------------------------------
constexpr int kWBM = 256;       // activation rows per workgroup tile
constexpr int kWBN = 256;       // weight rows per workgroup tile (64 per wave)
constexpr int kWH = 2;          // 64-k halves per step
constexpr int kWBK = 64 * kWH;  // k per step
constexpr int kWThreads = 256;  // 4 waves, one per SIMD
constexpr int kWChunksPerHalf = kWBM * 64 / 8;  // 16-byte chunks per 64-k half stage = 2048

// Direct global -> LDS load of 16 bytes per lane (global_load_lds_dwordx4): lane l's bytes land
// at the wave-uniform LDS address of `lds` (passed in m0 through an operand, so the compiler sets
// m0) plus 16 l.  Issued as inline assembly, so the compiler's wait counting covers only the
// ordinary loads and LDS reads; the caller waits for these with an explicit vmcnt(0) before the
// barrier that publishes the stage.  (Memory operations unknown to the compiler can only make its
// own vmcnt / lgkmcnt waits wait longer.)
__device__ __forceinline__ void lds_direct_load16(const void* g, const u32x4p* lds) {
    const uint32_t la = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));  // LDS offset
    __asm__ volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(la) : "memory");
}

// Instruction interleave of one wide sub-step: sixteen rounds of one MFMA, one LDS read (eight
// exist) and V VALU operations.
template <int V>
__device__ __forceinline__ void interleave_wide() {
#define QMM_PF_ROUND                                   \
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); \
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); \
    __builtin_amdgcn_sched_group_barrier(0x002, V, 0);
    QMM_PF_ROUND QMM_PF_ROUND QMM_PF_ROUND QMM_PF_ROUND QMM_PF_ROUND QMM_PF_ROUND QMM_PF_ROUND QMM_PF_ROUND
    QMM_PF_ROUND QMM_PF_ROUND QMM_PF_ROUND QMM_PF_ROUND QMM_PF_ROUND QMM_PF_ROUND QMM_PF_ROUND QMM_PF_ROUND
#undef QMM_PF_ROUND
}

template <class P, typename TC>
__global__ __launch_bounds__(kWThreads, 1) __attribute__((amdgpu_waves_per_eu(1, 1)))
void prefill_wide_kernel(const _Float16* __restrict__ A16, int lda, PfSegs<TC> sg, float* __restrict__ part_base, int M,
                         int K, int klen, int tiles_m, int tiles_n, int ksplit) {
    // one array per stage (not one [2][...] array); the step body is instantiated per stage, so each
    // of its LDS addresses is a fixed offset into one array
    __shared__ __align__(16) u32x4p sA0[kWH * kWChunksPerHalf];
    __shared__ __align__(16) u32x4p sA1[kWH * kWChunksPerHalf];

    // Tile order as in prefill_kernel: m fastest, then n-tile, then k split, dealt to XCDs in runs.
    const int tiles = tiles_m * tiles_n * ksplit;
    int b = blockIdx.x;
    if (tiles % 8 == 0) b = (b % 8) * (tiles / 8) + b / 8;
    const int tm = b % tiles_m;
    int tn = (b / tiles_m) % tiles_n;
    const int kz = b / (tiles_m * tiles_n);
    const int sgi = pf_seg_of(sg, tn);
    const uint8_t* __restrict__ W = sg.W[sgi];
    TC* __restrict__ C = sg.C[sgi];
    const int N = sg.N[sgi];
    const int ldc = sg.ldc[sgi];
    float* __restrict__ part = part_base + sg.part_off[sgi];
    const int m0 = tm * kWBM, n0 = tn * kWBN;
    const int kb = kz * klen;
    const int kend = min(K, kb + klen);
    const int nsteps = (kend - kb + kWBK - 1) / kWBK;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const int l32 = lane & 31;

    const size_t row_bytes = static_cast<size_t>(K / P::kQK) * P::kBytes;
    const int wal = ((reinterpret_cast<uintptr_t>(W) | row_bytes) & 3) == 0;  // 4-aligned rows
    const uint8_t* wrow[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
        wrow[nb] = W + static_cast<size_t>(min(n0 + 64 * wv + 32 * nb + l32, N - 1)) * row_bytes;

    // Thread tid copies chunks p = tid + 256j (j = 0..7) of each half stage: row (tid >> 3) + 32j,
    // stored in place at p, holding logical chunk c = (tid & 7) ^ swizzle(row) (the swizzle of
    // a_slot() is the same for all eight rows).  aoff[j]: element offset of the row's chunk c.
    // The copy is a direct global -> LDS load (global_load_lds_dwordx4): lane l of wave wv
    // writes 16 bytes at the wave-uniform base chunk 2048u + 256j + 64wv plus l, i.e. at p.
    const int ac = (tid & 7) ^ ((tid >> 4) & 7);
    uint32_t aoff[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        aoff[j] = static_cast<uint32_t>(min(m0 + (tid >> 3) + 32 * j, M - 1)) * static_cast<uint32_t>(lda) +
                  static_cast<uint32_t>(kb + 8 * ac);
    auto copy_a = [&](int t, u32x4p* dst) {
        const int kk = min(t, nsteps - 1) * kWBK;  // past the end: re-read the last step
#pragma unroll
        for (int u = 0; u < kWH; ++u)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                lds_direct_load16(A16 + aoff[j] + kk + 64 * u, dst + kWChunksPerHalf * u + 256 * j + 64 * wv);
    };
    using Raw = typename P::Raw;
    using Sc = typename P::Sc;
    auto load_raw = [&](int t, Raw (&raw)[2]) {
        const int k0 = kb + min(t, nsteps - 1) * kWBK;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) raw[nb] = P::load(wrow[nb], k0, h, kend - k0, wal);
    };
    auto read_a = [&](const u32x4p* stage, int U, int S, f16x8 (&af)[8]) {
        const u32x4p* sa = stage + kWChunksPerHalf * U;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const u32x4p av = sa[a_slot(32 * i + l32, a_chunk(S, h))];
            __builtin_memcpy(&af[i], &av, 16);
        }
    };

    f32x16 acc[2][8];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[nb][i][v] = 0.0f;

    // Software pipeline.  Step t (k0 = kb + 128t) runs sub-steps q = 0..7 (U = q/4, S = q%4) on
    // the stage held in sA0 (t even) or sA1 (t odd).  While the 16 MFMAs of sub-step q run on
    // wf[q&1] / af[q&1], the wave reads the activation fragments of q+1 from LDS and dequantizes
    // its two weight fragments into the other buffers.
    //   q = 0: the direct loads of A(t+1) into the other stage, then the raw bytes of step t+1
    //          (into `nxt`), are issued;
    //   q = 1: scales of half 1 (from `cur`);
    //   q = 5: scales of the next step's half 0 (from `nxt`);
    //   q = 7: first this wave's loads (A(t+1), `nxt`) and LDS reads (issued a sub-step earlier)
    //          complete, then the barrier; then the fragments of the next step's (0, 0):
    //          activations from the other stage, weights from `nxt`; at the end `cur` takes `nxt`.
    // The other stage last served step t-1, whose reads all precede step t-1's barrier, so one
    // barrier per step covers both the write-after-read and the read-after-write order.
    Raw cur[2], nxt[2];
    Sc sc[2][2];          // [weight block][half]
    uint32_t wf[2][2][4]; // [buffer][weight block][dword]
    f16x8 af[2][8];       // [buffer][activation block]

    load_raw(0, cur);
    copy_a(0, sA0);
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
    lds_barrier();
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        P::prep(cur[nb], h);
        sc[nb][0] = P::template scales<0>(cur[nb], kb, h, kend - kb);
        P::template frag<0, 0>(cur[nb], sc[nb][0], h, wf[0][nb]);
    }
    read_a(sA0, 0, 0, af[0]);

    auto step = [&](auto stage_c, int t) {
        constexpr bool odd = decltype(stage_c)::value != 0;
        const u32x4p* const s_cur = odd ? sA1 : sA0;
        u32x4p* const s_nxt = odd ? sA0 : sA1;
        const int k0 = kb + t * kWBK;
        copy_a(t + 1, s_nxt);
        load_raw(t + 1, nxt);
        __builtin_amdgcn_sched_barrier(0);

        constexpr int kQ = 4 * kWH;  // sub-steps per step
        auto sub = [&](auto qc) {
            constexpr int q = decltype(qc)::value;
            constexpr int B = q & 1;
            constexpr int qn = q + 1, Un = qn >> 2, Sn = qn & 3;
            if constexpr (qn == kQ) {
                __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0): A(t+1) is in LDS
                lds_barrier();
                read_a(s_nxt, 0, 0, af[B ^ 1]);
            } else {
                read_a(s_cur, Un, Sn, af[B ^ 1]);
            }
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                if constexpr (q == 1) sc[nb][1] = P::template scales<1>(cur[nb], k0, h, kend - k0);
                if constexpr (q == kQ - 3) {
                    P::prep(nxt[nb], h);
                    sc[nb][0] = P::template scales<0>(nxt[nb], k0 + kWBK, h, kend - k0 - kWBK);
                }
                if constexpr (qn < kQ) P::template frag<Un, Sn>(cur[nb], sc[nb][Un], h, wf[B ^ 1][nb]);
                else P::template frag<0, 0>(nxt[nb], sc[nb][0], h, wf[B ^ 1][nb]);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    f16x8 bw;
                    __builtin_memcpy(&bw, wf[B][nb], 16);
                    acc[nb][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bw, af[B][i], acc[nb][i], 0, 0, 0);
                }
            interleave_wide<kWideValu>();
            __builtin_amdgcn_sched_barrier(0);
        };
        for_each_index(sub, std::make_integer_sequence<int, kQ>{});
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) cur[nb] = nxt[nb];
    };
    int t = 0;
    for (; t + 1 < nsteps; t += 2) {
        step(std::integral_constant<int, 0>{}, t);
        step(std::integral_constant<int, 1>{}, t + 1);
    }
    if (t < nsteps) step(std::integral_constant<int, 0>{}, t);

    if constexpr (sizeof(TC) == 2) {
        if (ksplit == 1) {
            // fp16 tile through LDS, so that every store instruction writes whole row segments:
            // the 256 x 256 tile (128 KiB) goes into the two activation stages (rows 0..127 and
            // 128..255, 512 bytes each, 16-byte chunks XOR-swizzled by row so that the 32 rows a
            // write instruction touches fall in different banks), then each wave stores 64 rows,
            // two 512-byte row segments per instruction.
            __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // trailing stage copies have landed
            __syncthreads();
            uint8_t* const st0 = reinterpret_cast<uint8_t*>(sA0);
            uint8_t* const st1 = reinterpret_cast<uint8_t*>(sA1);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int m = 32 * i + l32;
                const float sm = sg.rs != nullptr && m0 + m < M ? sg.rs[m0 + m] : 1.0f;
                uint8_t* const row = (m < 128 ? st0 : st1) + (m & 127) * 512;
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const int n = 64 * wv + 32 * nb + 8 * g + 4 * h;  // tile-local, multiple of 4
                        const uint32_t w0 = float_to_half_bits(acc[nb][i][4 * g] * sm) |
                                            (static_cast<uint32_t>(float_to_half_bits(acc[nb][i][4 * g + 1] * sm)) << 16);
                        const uint32_t w1 = float_to_half_bits(acc[nb][i][4 * g + 2] * sm) |
                                            (static_cast<uint32_t>(float_to_half_bits(acc[nb][i][4 * g + 3] * sm)) << 16);
                        *reinterpret_cast<uint2*>(row + (((n >> 3) ^ (m & 31)) << 4) + ((n >> 2) & 1) * 8) = make_uint2(w0, w1);
                    }
            }
            __syncthreads();
            const int c = lane & 31;  // 16-byte chunk of the row: columns 8c .. 8c + 7
#pragma unroll 4
            for (int k = 0; k < 32; ++k) {
                const int m = 64 * wv + 2 * k + (lane >> 5);
                const uint8_t* row = (m < 128 ? st0 : st1) + (m & 127) * 512;
                const uint4 v = *reinterpret_cast<const uint4*>(row + ((c ^ (m & 31)) << 4));
                const int gm = m0 + m, gn = n0 + 8 * c;
                if (gm >= M || gn >= N) continue;
                uint16_t* dst = reinterpret_cast<uint16_t*>(C) + static_cast<size_t>(gm) * ldc + gn;
                if (gn + 7 < N && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
                    *reinterpret_cast<uint4*>(dst) = v;
                } else {
                    const uint32_t wv4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (gn + e < N) dst[e] = static_cast<uint16_t>(wv4[e >> 1] >> (16 * (e & 1)));
                }
            }
            return;
        }
    }
    if constexpr (sizeof(TC) == 4) {
        if (ksplit == 1) {
            // fp32 tile through LDS in two passes of 128 rows (128 KiB each: a pass's rows 0..63 in
            // the first activation stage, 64..127 in the second, 1 KiB per row, 16-byte chunks
            // XOR-swizzled by row), then each wave stores 32 rows, one 1 KiB row segment per
            // instruction.
            __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // trailing stage copies have landed
            uint8_t* const st0 = reinterpret_cast<uint8_t*>(sA0);
            uint8_t* const st1 = reinterpret_cast<uint8_t*>(sA1);
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                __syncthreads();  // the stages are idle: past the last step (p = 0), or pass 0 is stored
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    const int i = 4 * p + ii;
                    const int r = 32 * ii + l32;  // row within the pass; tile row 128p + r
                    const float sm = sg.rs != nullptr && m0 + 128 * p + r < M ? sg.rs[m0 + 128 * p + r] : 1.0f;
                    uint8_t* const row = (r < 64 ? st0 : st1) + (r & 63) * 1024;
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            const int n = 64 * wv + 32 * nb + 8 * g + 4 * h;  // tile-local, multiple of 4
                            *reinterpret_cast<float4*>(row + (((n >> 2) ^ (r & 31)) << 4)) =
                                make_float4(acc[nb][i][4 * g] * sm, acc[nb][i][4 * g + 1] * sm,
                                            acc[nb][i][4 * g + 2] * sm, acc[nb][i][4 * g + 3] * sm);
                        }
                }
                __syncthreads();
#pragma unroll 4
                for (int k = 0; k < 32; ++k) {
                    const int r = 32 * wv + k;
                    const uint8_t* row = (r < 64 ? st0 : st1) + (r & 63) * 1024;
                    const float4 v = *reinterpret_cast<const float4*>(row + ((lane ^ (r & 31)) << 4));
                    const int gm = m0 + 128 * p + r, gn = n0 + 4 * lane;  // columns 4 lane .. + 3
                    if (gm >= M || gn >= N) continue;
                    float* dst = reinterpret_cast<float*>(C) + static_cast<size_t>(gm) * ldc + gn;
                    if (gn + 3 < N && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
                        *reinterpret_cast<float4*>(dst) = v;
                    } else {
                        const float vf[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (gn + e < N) dst[e] = vf[e];
                    }
                }
            }
            return;
        }
    }

    // D element v of tile (nb, i): weight row n = n0 + 64wv + 32nb + 8(v/4) + 4h + v%4,
    // activation row m = m0 + 32i + l32.
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int m = m0 + 32 * i + l32;
        if (m >= M) continue;
        const float sm = sg.rs != nullptr ? sg.rs[m] : 1.0f;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = n0 + 64 * wv + 32 * nb + 8 * g + 4 * h;
                const float vs[4] = {acc[nb][i][4 * g] * sm, acc[nb][i][4 * g + 1] * sm, acc[nb][i][4 * g + 2] * sm,
                                     acc[nb][i][4 * g + 3] * sm};
                store_quad<TC>(C, part, ksplit, kz, M, N, ldc, m, n, vs);
            }
    }
}

// fp32 / fp16 activations [M, K] -> f16 [M, lda] (round to nearest even; columns K..lda-1 zero).
template <typename TA>
__global__ __launch_bounds__(256) void to_f16_kernel(const TA* __restrict__ A, _Float16* __restrict__ out, int M, int K,
                                                     int lda) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // 8 outputs per thread
    const int64_t per_row = lda / 8;
    if (i >= static_cast<int64_t>(M) * per_row) return;
    const int m = static_cast<int>(i / per_row);
    const int k = static_cast<int>(i - static_cast<int64_t>(m) * per_row) * 8;
    _Float16 v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int kk = k + e;
        float x = 0.0f;
        if (kk < K) {
            if constexpr (sizeof(TA) == 4) x = A[static_cast<size_t>(m) * K + kk];
            else x = __half2float(A[static_cast<size_t>(m) * K + kk]);
        }
        v[e] = static_cast<_Float16>(x);
    }
    __builtin_memcpy(out + static_cast<size_t>(m) * lda + k, v, 16);
}

// fp32 activations [M, K] -> f16 [M, lda], one workgroup per row.  A row whose largest magnitude
// lies outside the f16 range (at or above 65504, or in [2^-126, 2^-14)) is rounded as x * 2^-e
// with e = exponent(max) - 14 (its maximum lands in [2^14, 2^15)), and rs[m] = 2^e (a subnormal
// fp32 number below 2^-126) multiplies the row's outputs: a product of the scaled row is the
// original one times 2^-e, and both scalings are exact while their results are normal fp32
// numbers.  Other rows are rounded unchanged and rs[m] = 1.  Infinite or NaN values keep e = 0
// and propagate, and so does a row whose maximum is below 2^-126 (it rounds to zero in f16).
__global__ __launch_bounds__(256) void to_f16_rows_kernel(const float* __restrict__ A, _Float16* __restrict__ out,
                                                          float* __restrict__ rs, int K, int lda) {
    __shared__ float red[4];
    const int m = blockIdx.x;
    const int tid = threadIdx.x;
    const float* row = A + static_cast<size_t>(m) * K;
    // 16-byte loads where the row allows them, several in flight per thread (the maximum does not
    // depend on the order)
    const bool vec = (K & 7) == 0 && (reinterpret_cast<uintptr_t>(row) & 15u) == 0;
    // Rows of up to 16384 values (padded) are read once: each thread keeps its eight-value units
    // in registers between the maximum and the conversion, all its loads in flight at once.
    constexpr int kU = 8;
    const bool cached = vec && lda <= 8 * 256 * kU;
    float4 va[kU], vb[kU];
    float mx = 0.0f;
    if (cached) {
        const float4* r4 = reinterpret_cast<const float4*>(row);
#pragma unroll
        for (int i = 0; i < kU; ++i) {
            const int k = 8 * (tid + 256 * i);
            const bool in = k < K;  // K % 8 == 0: a unit is inside the row or past it
            va[i] = in ? r4[k / 4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            vb[i] = in ? r4[k / 4 + 1] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int i = 0; i < kU; ++i) {
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(va[i].x), fabsf(va[i].y)), fmaxf(fabsf(va[i].z), fabsf(va[i].w))));
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(vb[i].x), fabsf(vb[i].y)), fmaxf(fabsf(vb[i].z), fabsf(vb[i].w))));
        }
    } else if (vec) {
        const float4* r4 = reinterpret_cast<const float4*>(row);
#pragma unroll 4
        for (int k = tid; k < K / 4; k += 256) {
            const float4 v = r4[k];
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    } else {
        for (int k = tid; k < K; k += 256) mx = fmaxf(mx, fabsf(row[k]));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const uint32_t mb = __float_as_uint(mx);
    const bool big = mb >= 0x477FE000u && mb < 0x7F800000u;
    const bool tiny = mb >= 0x00800000u && mb < 0x38800000u;
    const int e = big || tiny ? static_cast<int>(mb >> 23) - 127 - 14 : 0;
    if (tid == 0) rs[m] = __builtin_ldexpf(1.0f, e);
    if (cached) {
#pragma unroll
        for (int i = 0; i < kU; ++i) {
            const int k = 8 * (tid + 256 * i);
            if (k >= lda) break;
            const float x[8] = {va[i].x, va[i].y, va[i].z, va[i].w, vb[i].x, vb[i].y, vb[i].z, vb[i].w};
            _Float16 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = static_cast<_Float16>(__builtin_ldexpf(x[j], -e));
            __builtin_memcpy(out + static_cast<size_t>(m) * lda + k, v, 16);
        }
        return;
    }
#pragma unroll 2
    for (int k = 8 * tid; k < lda; k += 8 * 256) {
        float x[8];
        if (vec && k + 8 <= K) {
            const float4 a = *reinterpret_cast<const float4*>(row + k);
            const float4 b = *reinterpret_cast<const float4*>(row + k + 4);
            x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = k + j < K ? row[k + j] : 0.0f;
        }
        _Float16 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = static_cast<_Float16>(__builtin_ldexpf(x[j], -e));
        __builtin_memcpy(out + static_cast<size_t>(m) * lda + k, v, 16);
    }
}

// C[m, n] (rows ldc apart) = sum_z part[z][m][n] in a fixed order, for part blocks [ksplit][M][N].
// Four consecutive elements per thread: with N % 4 == 0 (no quad crosses a row) and 16-byte
// aligned partials, 16-byte loads, the partial blocks requested four at a time before they are
// added (in z order), and one 8- or 16-byte store where C's row allows it; element by element
// otherwise.
template <typename TC>
__global__ __launch_bounds__(256) void reduce_kernel(const float* __restrict__ part, TC* __restrict__ C, int M, int N,
                                                     int ldc, int ksplit) {
    const int64_t mn = static_cast<int64_t>(M) * N;
    const int64_t i0 = 4 * (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x);
    if (i0 >= mn) return;
    const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(part) & 15u) == 0 && (mn & 3) == 0;
    if (!vec) {
        for (int64_t i = i0; i < min(i0 + 4, mn); ++i) {
            float s = part[i];
            for (int z = 1; z < ksplit; ++z) s += part[static_cast<size_t>(z) * mn + i];
            const int64_t m = i / N;
            const size_t o = static_cast<size_t>(m) * ldc + static_cast<size_t>(i - m * N);
            if constexpr (sizeof(TC) == 4) C[o] = s;
            else reinterpret_cast<uint16_t*>(C)[o] = float_to_half_bits(s);
        }
        return;
    }
    const float4* p4 = reinterpret_cast<const float4*>(part) + i0 / 4;
    const int64_t zs = mn / 4;  // float4 stride between partial blocks
    float4 s = p4[0];
    for (int z = 1; z < ksplit; z += 4) {
        float4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = p4[static_cast<size_t>(min(z + j, ksplit - 1)) * zs];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (z + j < ksplit) {
                s.x += v[j].x;
                s.y += v[j].y;
                s.z += v[j].z;
                s.w += v[j].w;
            }
        }
    }
    const int64_t m = i0 / N;
    const int64_t n = i0 - m * N;
    TC* dst = C + static_cast<size_t>(m) * ldc + n;
    if constexpr (sizeof(TC) == 4) {
        if ((reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
            *reinterpret_cast<float4*>(dst) = s;
        } else {
            dst[0] = s.x;
            dst[1] = s.y;
            dst[2] = s.z;
            dst[3] = s.w;
        }
    } else {
        const uint32_t lo = float_to_half_bits(s.x) | (static_cast<uint32_t>(float_to_half_bits(s.y)) << 16);
        const uint32_t hi = float_to_half_bits(s.z) | (static_cast<uint32_t>(float_to_half_bits(s.w)) << 16);
        if ((reinterpret_cast<uintptr_t>(dst) & 7u) == 0) {
            *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
        } else {
            uint16_t* d16 = reinterpret_cast<uint16_t*>(dst);
            d16[0] = static_cast<uint16_t>(lo);
            d16[1] = static_cast<uint16_t>(lo >> 16);
            d16[2] = static_cast<uint16_t>(hi);
            d16[3] = static_cast<uint16_t>(hi >> 16);
        }
    }
}

// Grow-only device workspace per (device, stream): the f16 copy of the activations and the
// split-K partial tiles.  Calls on one stream are ordered, so they may share it.
struct Workspace {
    void* buf = nullptr;
    size_t cap = 0;
};
std::mutex g_ws_mutex;
std::unordered_map<std::string, Workspace> g_ws;

hipError_t workspace(hipStream_t stream, size_t bytes, void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const std::string key = std::to_string(dev) + ":" + std::to_string(reinterpret_cast<uintptr_t>(stream));
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    Workspace& ws = g_ws[key];
    if (ws.cap < bytes) {
        if (ws.buf) {
            // the previous buffer may still be read by queued work on this stream
            if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
            if ((e = hipFree(ws.buf)) != hipSuccess) return e;
            ws.buf = nullptr;
            ws.cap = 0;
        }
        if ((e = hipMalloc(&ws.buf, bytes)) != hipSuccess) return e;
        ws.cap = bytes;
    }
    *out = ws.buf;
    return hipSuccess;
}

}  // namespace

hipError_t release_prefill_workspaces() {
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    for (auto& kv : g_ws) {
        if (!kv.second.buf) continue;
        const int dev = std::stoi(kv.first.substr(0, kv.first.find(':')));
        // queued kernels on any stream of the device may still read the buffer
        if ((e = hipSetDevice(dev)) != hipSuccess) return e;
        if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
        if ((e = hipFree(kv.second.buf)) != hipSuccess) return e;
        kv.second.buf = nullptr;
        kv.second.cap = 0;
    }
    g_ws.clear();
    return hipSetDevice(cur);
}

namespace {

int g_cus = 0;

hipError_t cu_count(int& cus) {
    if (g_cus > 0) {
        cus = g_cus;
        return hipSuccess;
    }
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
    g_cus = cus;
    return hipSuccess;
}

// The wide tile pays off once a 256-row activation tile is mostly filled (M >= 256, and padding M
// to 256 costs at most 64 rows more than padding it to 128) and its tiles cover at least half the
// CUs without splitting K (one workgroup per CU; a split costs a partial-sum pass).  Its element
// offsets are 32-bit.
bool use_wide(int M, int64_t wide_tiles_n, int K, int cus) {
    const int64_t pad256 = (static_cast<int64_t>(M) + kWBM - 1) / kWBM * kWBM;
    const int64_t pad128 = (static_cast<int64_t>(M) + kBM - 1) / kBM * kBM;
    const int64_t lda = (static_cast<int64_t>(K) + kWBK - 1) / kWBK * kWBK;
    const int64_t tiles = (pad256 / kWBM) * wide_tiles_n;
    return M >= kWBM && pad256 <= pad128 + 64 && kWideMin * tiles >= cus && static_cast<int64_t>(M) * lda < (int64_t{1} << 31);
}

struct PfSeg {
    const void* W;
    void* C;
    int N;
    int ldc;  // elements between rows of C (N for a whole matrix)
};

// A caller-provided workspace (the allocation-free entry point): `need` receives the bytes the
// launch plan uses; a plan needing more than `cap` launches nothing.
struct PfWs {
    void* buf;
    size_t cap;
    size_t need;
};

// Tile kinds: 128 x 256, 256 x 256 (wide) and 32 x 256 (small M).
enum PfTile { kTileStd = 0, kTileWide = 1, kTileSmall = 2 };
template <class P, int Tile>
struct PfShape {
    static constexpr bool kWide = Tile == kTileWide;
    static constexpr int BM = kWide ? kWBM : Tile == kTileSmall ? kSmallBM : kBM;
    static constexpr int BN = kWide ? kWBN : kBN;
    static constexpr int BK = kWide ? kWBK : 64 * P::kH;
    static constexpr int threads = kWide ? kWThreads : kThreads;
};

// One launch of the tile kernel `Tile` over `segs` with K split `ksplit` ways (at most; the split
// length is a whole number of steps), then, for a split, the pass that adds the partial tiles (at
// `part`) into C.
template <class P, typename TC, int Tile>
hipError_t launch_grid(const _Float16* a16, int lda, const PfSeg* segs, int nseg, int M, int K, int ksplit,
                       float* part, const float* rs, hipStream_t stream) {
    using Sh = PfShape<P, Tile>;
    constexpr int BM = Sh::BM, BN = Sh::BN, BK = Sh::BK;
    constexpr int threads = Sh::threads;
    const int tiles_m = (M + BM - 1) / BM;
    const int steps = (K + BK - 1) / BK;
    const int klen = ((steps + ksplit - 1) / ksplit) * BK;
    ksplit = (steps * BK + klen - 1) / klen;
    PfSegs<TC> sg;
    sg.rs = rs;
    size_t off = 0;
    int tiles_n = 0;
    for (int i = 0; i < kPfMaxSegs; ++i) {
        const bool used = i < nseg;
        sg.W[i] = used ? static_cast<const uint8_t*>(segs[i].W) : nullptr;
        sg.C[i] = used ? static_cast<TC*>(segs[i].C) : nullptr;
        sg.N[i] = used ? segs[i].N : 0;
        sg.ldc[i] = used ? segs[i].ldc : 0;
        if (used) tiles_n += (segs[i].N + BN - 1) / BN;
        sg.tile_end[i] = used ? tiles_n : INT_MAX;
        sg.part_off[i] = off;
        if (used && ksplit > 1) off += static_cast<size_t>(ksplit) * M * segs[i].N;
    }
    const int tiles = tiles_m * tiles_n * ksplit;
    if constexpr (Sh::kWide)
        hipLaunchKernelGGL((prefill_wide_kernel<P, TC>), dim3(tiles), dim3(threads), 0, stream, a16, lda, sg,
                           ksplit > 1 ? part : nullptr, M, K, klen, tiles_m, tiles_n, ksplit);
    else
        hipLaunchKernelGGL((prefill_kernel<P, TC, BM>), dim3(tiles), dim3(threads), 0, stream, a16, lda, sg,
                           ksplit > 1 ? part : nullptr, M, K, klen, tiles_m, tiles_n, ksplit);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (ksplit > 1) {
        for (int i = 0; i < nseg; ++i) {
            const int64_t mn = static_cast<int64_t>(M) * segs[i].N;
            hipLaunchKernelGGL((reduce_kernel<TC>), dim3(static_cast<unsigned>((mn + 1023) / 1024)), dim3(256), 0, stream,
                               part + sg.part_off[i], sg.C[i], M, segs[i].N, segs[i].ldc, ksplit);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

// Launch plan.  While the tiles cover at most half the CUs, K is split over the whole grid
// (doubling, keeping at least 1024 k per split).  Otherwise, when the tiles fill the CUs at
// least once and leave a last round of at most half the CUs (e.g. 896 tiles on 256 CUs), the
// last `tail_n` n-tiles (all m) run as a second launch with K split `tail_ks` ways, so that
// round's work is spread over all CUs: whole rounds first, then the split tail and its
// partial-sum pass over those columns only.  Wide tile only, for K of at least 32 steps (a
// shorter split saves less than its partial sums cost).
struct PfPlan {
    int ksplit = 1;
    int tail_n = 0;
    int tail_ks = 1;
};

PfPlan plan_prefill(bool wide, int tiles_m, int tiles_n, int steps, int bk, int cus, int fill = 1) {
    PfPlan p;
    while (tiles_m * tiles_n * p.ksplit * 2 <= fill * cus && steps / (p.ksplit * 2) >= 1024 / bk) p.ksplit *= 2;
    if (!wide || p.ksplit > 1 || steps < 32) return p;
    const int64_t T = static_cast<int64_t>(tiles_m) * tiles_n;
    const int64_t r = T % cus;
    if (T <= cus || r == 0 || 2 * r > cus) return p;
    const int tail_n = static_cast<int>((r + tiles_m - 1) / tiles_m);
    if (tail_n >= tiles_n) return p;
    int ks = static_cast<int>(cus / (static_cast<int64_t>(tiles_m) * tail_n));
    while (ks > 1 && steps / ks < 1024 / bk) --ks;
    if (ks < 2) return p;
    p.tail_n = tail_n;
    p.tail_ks = ks;
    return p;
}

template <class P, typename TA, typename TC, int Tile>
hipError_t launch_p(const void* A, const PfSeg* segs, int nseg, int M, int K, hipStream_t stream, PfWs* ext) {
    using Sh = PfShape<P, Tile>;
    constexpr int BM = Sh::BM, BN = Sh::BN, BK = Sh::BK;
    int cus = 0;
    hipError_t e = cu_count(cus);
    if (e != hipSuccess) return e;
    const int tiles_m = (M + BM - 1) / BM;
    int tiles_n = 0;
    int64_t n_total = 0;
    for (int i = 0; i < nseg; ++i) {
        tiles_n += (segs[i].N + BN - 1) / BN;
        n_total += segs[i].N;
    }
    const int steps = (K + BK - 1) / BK;
    // the small tile's grid is split to fill kSmallFill of its workgroups per CU
    const PfPlan plan = plan_prefill(Sh::kWide, tiles_m, tiles_n, steps, BK, cus, Tile == kTileSmall ? kSmallFill : 1);

    // the tail launch's segments: rows from n-tile ns on, as column ranges of the callers' C
    PfSeg main_segs[kPfMaxSegs], tail_segs[kPfMaxSegs];
    int n_main = 0, n_tail = 0;
    int64_t n_tail_total = 0;
    if (plan.tail_n > 0) {
        const int ns = tiles_n - plan.tail_n;
        const size_t row_bytes = static_cast<size_t>(K / P::kQK) * P::kBytes;
        int a = 0;
        for (int i = 0; i < nseg; ++i) {
            const int t = (segs[i].N + BN - 1) / BN;
            if (a < ns) main_segs[n_main++] = PfSeg{segs[i].W, segs[i].C, min(segs[i].N, (ns - a) * BN), segs[i].ldc};
            if (a + t > ns) {
                const int r0 = max(0, ns - a) * BN;
                tail_segs[n_tail++] = PfSeg{static_cast<const uint8_t*>(segs[i].W) + static_cast<size_t>(r0) * row_bytes,
                                            static_cast<TC*>(segs[i].C) + r0, segs[i].N - r0, segs[i].ldc};
                n_tail_total += segs[i].N - r0;
            }
            a += t;
        }
    }

    const bool direct = sizeof(TA) == 2 && K % BK == 0 && (reinterpret_cast<uintptr_t>(A) & 15u) == 0;
    const int lda = direct ? K : steps * BK;
    // f16 copy of the activations, then (fp32 activations) the rows' output factors
    const size_t a16_bytes = direct ? 0 : ((static_cast<size_t>(M) * lda * 2 + 255) / 256) * 256;
    const size_t a_bytes = a16_bytes + (sizeof(TA) == 4 ? static_cast<size_t>(M) * 4 : 0);
    size_t p_bytes = 0;
    if (plan.ksplit > 1) p_bytes = static_cast<size_t>(plan.ksplit) * M * n_total * 4;
    if (plan.tail_n > 0) p_bytes = static_cast<size_t>(plan.tail_ks) * M * n_tail_total * 4;
    void* ws = nullptr;
    if (ext != nullptr) {
        // caller-provided scratch: checked before anything is launched
        ext->need = a_bytes + p_bytes > 0 ? a_bytes + p_bytes + 256 : 0;
        if (ext->need > ext->cap) return hipErrorOutOfMemory;
        ws = ext->buf;
    } else if (a_bytes + p_bytes > 0 && (e = workspace(stream, a_bytes + p_bytes + 256, &ws)) != hipSuccess) {
        return e;
    }
    const _Float16* a16 = static_cast<const _Float16*>(A);
    float* rs = nullptr;
    if (!direct) {
        _Float16* dst = static_cast<_Float16*>(ws);
        if constexpr (sizeof(TA) == 4) {
            rs = reinterpret_cast<float*>(static_cast<char*>(ws) + a16_bytes);
            hipLaunchKernelGGL(to_f16_rows_kernel, dim3(static_cast<unsigned>(M)), dim3(256), 0, stream,
                               static_cast<const float*>(A), dst, rs, K, lda);
        } else {
            const int64_t n8 = static_cast<int64_t>(M) * (lda / 8);
            hipLaunchKernelGGL((to_f16_kernel<TA>), dim3(static_cast<unsigned>((n8 + 255) / 256)), dim3(256), 0, stream,
                               static_cast<const TA*>(A), dst, M, K, lda);
        }
        if ((e = hipGetLastError()) != hipSuccess) return e;
        a16 = dst;
    }
    float* part = p_bytes > 0 ? reinterpret_cast<float*>(static_cast<char*>(ws) + ((a_bytes + 255) / 256) * 256) : nullptr;
    if (plan.tail_n == 0) return launch_grid<P, TC, Tile>(a16, lda, segs, nseg, M, K, plan.ksplit, part, rs, stream);
    if ((e = launch_grid<P, TC, Tile>(a16, lda, main_segs, n_main, M, K, 1, nullptr, rs, stream)) != hipSuccess) return e;
    return launch_grid<P, TC, Tile>(a16, lda, tail_segs, n_tail, M, K, plan.tail_ks, part, rs, stream);
}

// HN: 64-k halves per step of the 128 x 256 kernel for this format.
template <template <int> class PF, int HN, typename TA, typename TC>
hipError_t launch_family(const void* A, const PfSeg* segs, int nseg, int M, int K, hipStream_t stream, PfWs* ext) {
    int cus = 0;
    hipError_t e = cu_count(cus);
    if (e != hipSuccess) return e;
    int64_t wide_tiles_n = 0;
    for (int i = 0; i < nseg; ++i) wide_tiles_n += (segs[i].N + kWBN - 1) / kWBN;
    if (use_wide(M, wide_tiles_n, K, cus)) return launch_p<PF<kWH>, TA, TC, kTileWide>(A, segs, nseg, M, K, stream, ext);
    if (M <= kSmallMaxM) return launch_p<PF<HN>, TA, TC, kTileSmall>(A, segs, nseg, M, K, stream, ext);
    return launch_p<PF<HN>, TA, TC, kTileStd>(A, segs, nseg, M, K, stream, ext);
}

template <typename TA, typename TC>
hipError_t dispatch_p(int t, const void* A, const PfSeg* segs, int nseg, int M, int K, hipStream_t stream, PfWs* ext) {
    switch (t) {
        case QMM_TYPE_Q4_K: return launch_family<PQ4K, kHalves, TA, TC>(A, segs, nseg, M, K, stream, ext);
        case QMM_TYPE_Q6_K: return launch_family<PQ6K, kHalves, TA, TC>(A, segs, nseg, M, K, stream, ext);
        case QMM_TYPE_Q8_0: return launch_family<PQ80, 2, TA, TC>(A, segs, nseg, M, K, stream, ext);
        case QMM_TYPE_Q4_0: return launch_family<PQ40, 2, TA, TC>(A, segs, nseg, M, K, stream, ext);
        case QMM_TYPE_F16: return launch_family<PF16, 2, TA, TC>(A, segs, nseg, M, K, stream, ext);
        default: return hipErrorInvalidValue;
    }
}

hipError_t dispatch_dtypes(int t, const void* A, int a_dtype, int c_dtype, const PfSeg* segs, int nseg, int M, int K,
                           hipStream_t stream, PfWs* ext = nullptr) {
    if (a_dtype == QMM_DTYPE_F32) {
        if (c_dtype == QMM_DTYPE_F32) return dispatch_p<float, float>(t, A, segs, nseg, M, K, stream, ext);
        return dispatch_p<float, __half>(t, A, segs, nseg, M, K, stream, ext);
    }
    if (c_dtype == QMM_DTYPE_F32) return dispatch_p<__half, float>(t, A, segs, nseg, M, K, stream, ext);
    return dispatch_p<__half, __half>(t, A, segs, nseg, M, K, stream, ext);
}

}  // namespace

bool gemm_prefill_supported(int ggml_type, int a_dtype, int c_dtype, int M, int N, int K, const void*, const void* W,
                            const void*) {
    (void)a_dtype; (void)c_dtype;
    // Q4_K headers and qs pieces are read with 16-byte aligned loads; other formats need 2-byte
    // alignment (fp16 scales or values); F16 rows are read in 8-value chunks.
    const uintptr_t wa = reinterpret_cast<uintptr_t>(W);
    if (ggml_type == QMM_TYPE_Q4_K && (wa & 15u) != 0) return false;
    if ((wa & 1u) != 0) return false;
    if (ggml_type == QMM_TYPE_F16 && K % 8 != 0) return false;
    return M > 0 && N > 0 && K > 0;
}

hipError_t launch_gemm_prefill(int ggml_type, const void* A, int a_dtype, const void* W, void* C, int c_dtype, int M,
                               int N, int K, hipStream_t stream) {
    const PfSeg seg{W, C, N, N};
    return dispatch_dtypes(ggml_type, A, a_dtype, c_dtype, &seg, 1, M, K, stream);
}

int prefill_max_fused() { return kPfMaxSegs; }

// ---- allocation-free prefill: the workspace is a file-scope device array ------------------------
// Each device the library runs on holds its own copy of `scratch` until the process ends.  In host
// code `scratch` names a host-side stand-in, never the device memory: kernels get the per-device
// address that hipGetSymbolAddress returns (looked up once per device, with that device current).
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
// Per device: the scratch address, and an event recorded after the last eager call that used the
// scratch, with that call's stream.  An eager call on another stream waits for the event first, so
// calls on different streams take turns on the array instead of racing.  Calls under stream
// capture neither wait nor record (the caller orders graph replays against other work).
struct ScratchDev {
    void* ptr = nullptr;
    hipEvent_t done = nullptr;
    hipStream_t last = nullptr;
    bool pending = false;
};
std::mutex g_scratch_mutex;
std::unordered_map<int, ScratchDev> g_scratch;
}  // namespace

hipError_t launch_gemm_prefill_noalloc(int ggml_type, const void* A, int a_dtype, const void* W, void* C, int c_dtype,
                                       int M, int N, int K, hipStream_t stream, size_t* need) {
    *need = 0;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);  // held through the launches: calls take turns
    ScratchDev& sd = g_scratch[dev];
    if (sd.ptr == nullptr) {
        void* ptr = nullptr;
        if ((e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch))) != hipSuccess) return e;
        if (ptr == nullptr) return hipErrorInvalidSymbol;
        if ((e = hipEventCreateWithFlags(&sd.done, hipEventDisableTiming)) != hipSuccess) return e;
        sd.ptr = ptr;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if ((e = hipStreamIsCapturing(stream, &cs)) != hipSuccess) return e;
    const bool eager = cs == hipStreamCaptureStatusNone;
    if (eager && sd.pending && stream != sd.last && (e = hipStreamWaitEvent(stream, sd.done, 0)) != hipSuccess) return e;
    PfWs ext{sd.ptr, kNoAllocScratchBytes, 0};
    const PfSeg seg{W, C, N, N};
    e = dispatch_dtypes(ggml_type, A, a_dtype, c_dtype, &seg, 1, M, K, stream, &ext);
    *need = ext.need;
    if (e == hipSuccess && eager && ext.need > 0) {
        if ((e = hipEventRecord(sd.done, stream)) != hipSuccess) return e;
        sd.last = stream;
        sd.pending = true;
    }
    return e;
}

hipError_t launch_gemm_prefill_fused(int ggml_type, const void* A, int a_dtype, int c_dtype, int M, int K,
                                     const void* const* W, void* const* C, const int* N, int count, hipStream_t stream) {
    if (count < 1 || count > kPfMaxSegs) return hipErrorInvalidValue;
    PfSeg segs[kPfMaxSegs];
    for (int i = 0; i < count; ++i) segs[i] = PfSeg{W[i], C[i], N[i], N[i]};
    return dispatch_dtypes(ggml_type, A, a_dtype, c_dtype, segs, count, M, K, stream);
}

}  // namespace qmm
