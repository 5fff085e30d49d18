// Prefill GEMM (M >= kGemvMaxM): C[M, N] = A[M, K] @ dequant(W)[N, K]^T on f16 MFMA with fp32
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
#include <mutex>
#include <string>
#include <type_traits>
#include <utility>
#include <unordered_map>

#include "qmm_device.h"

namespace qmm {
namespace {

constexpr int kBM = 128;        // activation rows per workgroup tile
constexpr int kBN = 256;        // weight rows per workgroup tile (32 per wave)
constexpr int kHalves = 4;      // 64-k halves per step
constexpr int kBK = 64 * kHalves;  // k per step (one Q4_K / Q6_K super-block)
constexpr int kThreads = 512;   // 8 waves: two per SIMD, so one wave's load stalls are covered
constexpr int kChunksPerHalf = kBM * 64 / 8;  // 16-byte chunks (8 f16) per 64-k half stage = 1024

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
// Weight producers.  A step covers 256 k (one Q4_K / Q6_K super-block per row, eight Q4_0 /
// Q8_0 blocks) as four halves U = 0..3 of 64 and sixteen sub-steps (U, S), S = 0..3, of one MFMA
// k-block (16 k) each.  In sub-step (U, S), lane half h covers
// k = 64U + 32*(S>>1) + 16*h + 8*(S&1) + (0..7) of the step.
//   load()        one weight row's raw bytes for the whole step (issued a step ahead);
//   scales<U>()   the f16 scale (and offset) pairs of half U's two 32-weight groups;
//   frag<U, S>()  the MFMA fragment (8 f16, natural k order) of sub-step (U, S).
// kv = K - k0 lets the 32-weight formats zero a K tail; the zeroing happens in scales(), so no
// prefetched value is consumed before its sub-step.
// ---------------------------------------------------------------------------------------------
struct PQ4K {
    static constexpr int kQK = kQK_K, kBytes = kBytesQ4_K;
    struct Raw { u32x4p hd, q[4]; };
    struct Sc { h2 a0, b0, a1, b1; };
    // step at k0 (multiple of 256): super-block k0/256; half U is qs chunk c = U (low nibbles:
    // sub-block 2c, high: 2c+1); lane half h takes qs bytes 16h..16h+15 of each chunk.
    __device__ static Raw load(const uint8_t* row, int k0, int h, int) {
        const uint8_t* sb = row + static_cast<size_t>(k0 >> 8) * kBytes;
        Raw r;
        r.hd = *reinterpret_cast<const u32x4p*>(sb);
#pragma unroll
        for (int c = 0; c < 4; ++c) r.q[c] = *reinterpret_cast<const u32x4p*>(sb + 16 + 32 * c + 16 * h);
        return r;
    }
    template <int U>
    __device__ static Sc scales(const Raw& r, int, int, int) {
        // 6-bit scales/mins of sub-blocks 2U and 2U + 1: bytes 2(U&1), 2(U&1)+1 of the packed
        // scale words; sub-blocks 4..7 (U >= 2) take their top bits from words 0/1.
        constexpr int sh = 16 * (U & 1);
        const uint32_t u0 = r.hd.y >> sh, u1 = r.hd.z >> sh, u2 = r.hd.w >> sh;
        uint32_t scp, mp;
        if constexpr (U < 2) {
            scp = u0 & 0x3F3Fu;
            mp = u1 & 0x3F3Fu;
        } else {
            scp = (u2 & 0x0F0Fu) | ((u0 >> 2) & 0x3030u);
            mp = ((u2 >> 4) & 0x0F0Fu) | ((u1 >> 2) & 0x3030u);
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
        constexpr bool hi = S >= 2;  // high nibbles: sub-block 2U + 1
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

struct PQ6K {
    static constexpr int kQK = kQK_K, kBytes = kBytesQ6_K;
    struct Raw { u32x4p la[2], lb[2], qh[2], sc; uint32_t d; };
    struct Sc { h2 a0, a1; };
    // step at k0 (multiple of 256): super-block k0/256; half U is quarter qt = U of the block:
    // half n2 = U>>1 of 128 weights, groups t = 2(U&1) + (S>>1).  Lane half h takes l = 16h..16h+15
    // of ql (groups t even: ql[64n2 + l], odd: ql[64n2 + 32 + l]; U&1 picks the nibble) and of
    // qh[32n2 + l]; the sixteen int8 sub-scales arrive as one 16-byte load.
    __device__ static Raw load(const uint8_t* row, int k0, int h, int) {
        const uint8_t* sb = row + static_cast<size_t>(k0 >> 8) * kBytes;
        Raw r;
#pragma unroll
        for (int n2 = 0; n2 < 2; ++n2) {
            r.la[n2] = ld16(sb + 64 * n2 + 16 * h);
            r.lb[n2] = ld16(sb + 64 * n2 + 32 + 16 * h);
            r.qh[n2] = ld16(sb + 128 + 32 * n2 + 16 * h);
        }
        r.sc = ld16(sb + 192);
        r.d = ld2(sb + 208);
        return r;
    }
    template <int U>
    __device__ static Sc scales(const Raw& r, int, int h, int) {
        // sub-scales sc[4U + h + {0, 2}]
        const uint32_t sc = U == 0 ? r.sc.x : U == 1 ? r.sc.y : U == 2 ? r.sc.z : r.sc.w;
        const float d = half_bits_to_float(r.d);
        Sc s;
        s.a0 = splat(d * static_cast<float>(static_cast<int8_t>(sc >> (8 * h))));
        s.a1 = splat(d * static_cast<float>(static_cast<int8_t>(sc >> (8 * h + 16))));
        return s;
    }
    template <int U, int S>
    __device__ static void frag(const Raw& r, const Sc& sc, int, uint32_t f[4]) {
        constexpr int n2 = U >> 1, nib = 4 * (U & 1), u = S >> 1;  // group t = 2(U&1) + u
        constexpr int hs = nib + 2 * u;                              // qh bit pair of the group
        const u32x4p l = u ? r.lb[n2] : r.la[n2];
        const u32x4p qh = r.qh[n2];
        const uint32_t lw[2] = {(S & 1) ? l.z : l.x, (S & 1) ? l.w : l.y};
        const uint32_t hw[2] = {(S & 1) ? qh.z : qh.x, (S & 1) ? qh.w : qh.y};
        const h2 off = splat(1056.0f);  // 1024 + 32: codes q enter as 1024 + q, weight is a (q - 32)
        const h2 a = u ? sc.a1 : sc.a0;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t lo4 = (lw[j] >> nib) & 0x0F0F0F0Fu;
            const uint32_t hi2 = ((hw[j] >> hs) & 0x03030303u) << 4;
            h2 p, q;
            bytes_to_h2(lo4 | hi2, off, p, q);
            f[2 * j] = as_u32(p * a);
            f[2 * j + 1] = as_u32(q * a);
        }
    }
};

// 32-weight block formats: a step covers blocks k0/32 + b, b = 0..7 (block b absent when
// kv <= 32b: load() clamps its address to block 0 and scales() zeroes its scale).  Half U
// holds blocks 2U (S = 0, 1) and 2U + 1 (S = 2, 3).
struct PQ80 {
    static constexpr int kQK = kQK8_0, kBytes = kBytesQ8_0;
    struct Raw { u32x4p q[8]; uint32_t d[8]; };
    struct Sc { h2 a0, a1; };
    __device__ static Raw load(const uint8_t* row, int k0, int h, int kv) {
        const uint8_t* b0 = row + static_cast<size_t>(k0 >> 5) * kBytes;
        Raw r;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
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

struct PQ40 {
    static constexpr int kQK = kQK4_0, kBytes = kBytesQ4_0;
    struct Raw { u32x4p q[8]; uint32_t d[8]; };
    struct Sc { h2 a0, a1; };
    // lane half h takes the block's low (h = 0, k 0..15) or high (h = 1, k 16..31) nibbles.
    __device__ static Raw load(const uint8_t* row, int k0, int, int kv) {
        const uint8_t* b0 = row + static_cast<size_t>(k0 >> 5) * kBytes;
        Raw r;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
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

// Activation chunk (row r, chunk c = 8 f16) position inside a 1024-chunk half stage: rows are
// XOR-swizzled so that 16 consecutive rows read at one chunk hit 16 different bank groups.
__device__ __forceinline__ int a_slot(int r, int c) { return 8 * r + (c ^ ((r >> 1) & 7)); }

// Sub-step S, lane half h -> activation chunk of the half stage.
__device__ __forceinline__ int a_chunk(int s, int h) { return 4 * (s >> 1) + 2 * h + (s & 1); }

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

template <class P, typename TC>
__global__ __launch_bounds__(kThreads, 1)
void prefill_kernel(const _Float16* __restrict__ A16, int lda, const uint8_t* __restrict__ W, TC* __restrict__ C,
                    float* __restrict__ part, int M, int N, int K, int klen, int tiles_m, int tiles_n, int ksplit) {
    __shared__ __align__(16) u32x4p sA[2][kHalves * kChunksPerHalf];

    // Tile order: m fastest, then n-tile, then k split; blocks sharing a weight slice (same
    // n-tile and k range, different m) are consecutive and dealt to one XCD.
    const int tiles = tiles_m * tiles_n * ksplit;
    int b = blockIdx.x;
    if (tiles % 8 == 0) b = (b % 8) * (tiles / 8) + b / 8;
    const int tm = b % tiles_m;
    const int tn = (b / tiles_m) % tiles_n;
    const int kz = b / (tiles_m * tiles_n);
    const int m0 = tm * kBM, n0 = tn * kBN;
    const int kb = kz * klen;
    const int kend = min(K, kb + klen);
    const int nsteps = (kend - kb + kBK - 1) / kBK;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const int l32 = lane & 31;

    const size_t row_bytes = static_cast<size_t>(K / P::kQK) * P::kBytes;
    const uint8_t* wrow = W + static_cast<size_t>(min(n0 + 32 * wv + l32, N - 1)) * row_bytes;

    // Thread tid copies half-stage chunks p = tid + 512 j (j = 0..1) of both halves: row p >> 3,
    // chunk (p & 7) ^ swizzle, so each thread's 4 global reads are 16-byte aligned f16 runs and
    // its LDS writes are in place.
    const _Float16* arow[2];
    int apos[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int p = tid + 512 * j;
        const int r = p >> 3;
        const int c = (p & 7) ^ ((r >> 1) & 7);
        arow[j] = A16 + static_cast<size_t>(min(m0 + r, M - 1)) * lda + kb + 8 * c;
        apos[j] = p;
    }
    auto load_a = [&](int t, u32x4p (&ar)[2 * kHalves]) {
        const int kk = min(t, nsteps - 1) * kBK;  // past the end: re-read the last step
#pragma unroll
        for (int u = 0; u < kHalves; ++u)
#pragma unroll
            for (int j = 0; j < 2; ++j) ar[2 * u + j] = *reinterpret_cast<const u32x4p*>(arow[j] + kk + 64 * u);
    };
    auto store_a = [&](int slot, const u32x4p (&ar)[2 * kHalves]) {
#pragma unroll
        for (int u = 0; u < kHalves; ++u)
#pragma unroll
            for (int j = 0; j < 2; ++j) sA[slot][kChunksPerHalf * u + apos[j]] = ar[2 * u + j];
    };
    auto load_raw = [&](int t, typename P::Raw& raw) {
        const int k0 = kb + min(t, nsteps - 1) * kBK;
        raw = P::load(wrow, k0, h, kend - k0);
    };
    // activation fragments of sub-step (U, S) of the step held in `slot`
    auto read_a = [&](int slot, int U, int S, f16x8 (&af)[4]) {
        const u32x4p* sa = sA[slot] + kChunksPerHalf * U;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4p av = sa[a_slot(32 * i + l32, a_chunk(S, h))];
            __builtin_memcpy(&af[i], &av, 16);
        }
    };

    f32x16 acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][v] = 0.0f;

    // Software pipeline.  Step t (k0 = kb + 256t) runs sub-steps q = 0..15 (U = q/4, S = q%4).
    // While the 4 MFMAs of sub-step q run on wf[q&1] / af[q&1], the wave reads the activation
    // fragments of q+1 from LDS and dequantizes its weight fragment into the other buffers.
    //   q = 0: the raw bytes of step t+1 (into `nxt`) and A(t+1) (into `an`) are requested;
    //   q = 4U+1 (U < 3): scales of half U+1 (from `cur`) into sc[(U+1)&1];
    //   q = 13: scales of the next step's half 0 (from `nxt`) into sc[0];
    //   q = 14: after the reads for q = 15, A(t+1) goes to the free LDS slot, then the barrier
    //           (after it, q = 15 reads the next step's first fragments from that slot);
    //   q = 15: fragment of the next step's (0, 0) from `nxt`; at the end `cur` takes `nxt`.
    // The LDS slot (t+1)%2 last served step t-1, whose reads all precede step t-1's barrier, so
    // one barrier per step covers both the write-after-read and the read-after-write order.
    using Raw = typename P::Raw;
    using Sc = typename P::Sc;
    u32x4p an[2 * kHalves];
    Raw cur, nxt;
    Sc sc[2];          // [half]
    uint32_t wf[2][4]; // [buffer][dword]
    f16x8 af[2][4];    // [buffer][i]

    load_raw(0, cur);
    load_a(0, an);
    store_a(0, an);
    lds_barrier();
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

        constexpr int kQ = 4 * kHalves;  // sub-steps per step
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
            if constexpr ((q & 3) == 1 && U + 1 < kHalves)
                sc[(U + 1) & 1] = P::template scales<(U + 1) % kHalves>(cur, k0, h, kend - k0);
            if constexpr (q == kQ - 3) sc[0] = P::template scales<0>(nxt, k0 + kBK, h, kend - k0 - kBK);
            if constexpr (qn < kQ) P::template frag<Un % kHalves, Sn>(cur, sc[Un & 1], h, wf[B ^ 1]);
            else P::template frag<0, 0>(nxt, sc[0], h, wf[B ^ 1]);
            f16x8 bw;
            __builtin_memcpy(&bw, wf[B], 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bw, af[B][i], acc[i], 0, 0, 0);
            interleave_substep<5>();
            __builtin_amdgcn_sched_barrier(0);
        };
        for_each_index(sub, std::make_integer_sequence<int, kQ>{});
        cur = nxt;
    }

    // D element v of tile i: weight row n = n0 + 32wv + 8(v/4) + 4h + v%4, activation row
    // m = m0 + 32i + l32.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 32 * i + l32;
        if (m >= M) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n = n0 + 32 * wv + 8 * g + 4 * h;
            const float vs[4] = {acc[i][4 * g], acc[i][4 * g + 1], acc[i][4 * g + 2], acc[i][4 * g + 3]};
            if (ksplit > 1) {
                float* dst = part + (static_cast<size_t>(kz) * M + m) * N;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (n + e < N) dst[n + e] = vs[e];
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (n + e < N) {
                        if constexpr (sizeof(TC) == 4) reinterpret_cast<float*>(C)[static_cast<size_t>(m) * N + n + e] = vs[e];
                        else reinterpret_cast<uint16_t*>(C)[static_cast<size_t>(m) * N + n + e] = float_to_half_bits(vs[e]);
                    }
                }
            }
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

// C = sum_z part[z] in a fixed order.
template <typename TC>
__global__ __launch_bounds__(256) void reduce_kernel(const float* __restrict__ part, TC* __restrict__ C, int64_t mn,
                                                     int ksplit) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= mn) return;
    float s = part[i];
    for (int z = 1; z < ksplit; ++z) s += part[static_cast<size_t>(z) * mn + i];
    if constexpr (sizeof(TC) == 4) C[i] = s;
    else reinterpret_cast<uint16_t*>(C)[i] = float_to_half_bits(s);
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

template <class P, typename TA, typename TC>
hipError_t launch_p(const void* A, const void* W, void* C, int M, int N, int K, hipStream_t stream) {
    int cus = 0;
    hipError_t e = cu_count(cus);
    if (e != hipSuccess) return e;
    const int tiles_m = (M + kBM - 1) / kBM;
    const int tiles_n = (N + kBN - 1) / kBN;
    const int steps = (K + kBK - 1) / kBK;
    // split K while the grid would still cover at most half the CUs (the partial-sum pass costs
    // 4 * (ksplit + 1) * M * N bytes), keeping at least 4 steps (1024 k) per split
    int ksplit = 1;
    while (tiles_m * tiles_n * ksplit * 2 <= cus && steps / (ksplit * 2) >= 4) ksplit *= 2;
    const int klen = ((steps + ksplit - 1) / ksplit) * kBK;
    ksplit = (steps * kBK + klen - 1) / klen;

    const bool direct = sizeof(TA) == 2 && K % kBK == 0 && (reinterpret_cast<uintptr_t>(A) & 15u) == 0;
    const int lda = direct ? K : steps * kBK;
    const size_t a_bytes = direct ? 0 : static_cast<size_t>(M) * lda * 2;
    const size_t p_bytes = ksplit > 1 ? static_cast<size_t>(ksplit) * M * N * 4 : 0;
    void* ws = nullptr;
    if (a_bytes + p_bytes > 0 && (e = workspace(stream, a_bytes + p_bytes + 256, &ws)) != hipSuccess) return e;
    const _Float16* a16 = static_cast<const _Float16*>(A);
    if (!direct) {
        _Float16* dst = static_cast<_Float16*>(ws);
        const int64_t n8 = static_cast<int64_t>(M) * (lda / 8);
        hipLaunchKernelGGL((to_f16_kernel<TA>), dim3(static_cast<unsigned>((n8 + 255) / 256)), dim3(256), 0, stream,
                           static_cast<const TA*>(A), dst, M, K, lda);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        a16 = dst;
    }
    float* part = ksplit > 1 ? reinterpret_cast<float*>(static_cast<char*>(ws) + ((a_bytes + 255) / 256) * 256) : nullptr;
    const int tiles = tiles_m * tiles_n * ksplit;
    hipLaunchKernelGGL((prefill_kernel<P, TC>), dim3(tiles), dim3(kThreads), 0, stream, a16, lda,
                       static_cast<const uint8_t*>(W), static_cast<TC*>(C), part, M, N, K, klen, tiles_m, tiles_n, ksplit);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (ksplit > 1) {
        const int64_t mn = static_cast<int64_t>(M) * N;
        hipLaunchKernelGGL((reduce_kernel<TC>), dim3(static_cast<unsigned>((mn + 255) / 256)), dim3(256), 0, stream, part,
                           static_cast<TC*>(C), mn, ksplit);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return hipSuccess;
}

template <typename TA, typename TC>
hipError_t dispatch_p(int t, const void* A, const void* W, void* C, int M, int N, int K, hipStream_t stream) {
    switch (t) {
        case QMM_TYPE_Q4_K: return launch_p<PQ4K, TA, TC>(A, W, C, M, N, K, stream);
        case QMM_TYPE_Q6_K: return launch_p<PQ6K, TA, TC>(A, W, C, M, N, K, stream);
        case QMM_TYPE_Q8_0: return launch_p<PQ80, TA, TC>(A, W, C, M, N, K, stream);
        case QMM_TYPE_Q4_0: return launch_p<PQ40, TA, TC>(A, W, C, M, N, K, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool gemm_prefill_supported(int ggml_type, int a_dtype, int c_dtype, int M, int N, int K, const void*, const void* W,
                            const void*) {
    (void)a_dtype; (void)c_dtype;
    // Q4_K headers and qs pieces are read with 16-byte aligned loads; other formats need 2-byte
    // alignment (fp16 scales).
    const uintptr_t wa = reinterpret_cast<uintptr_t>(W);
    if (ggml_type == QMM_TYPE_Q4_K && (wa & 15u) != 0) return false;
    if ((wa & 1u) != 0) return false;
    return M > 0 && N > 0 && K > 0;
}

hipError_t launch_gemm_prefill(int ggml_type, const void* A, int a_dtype, const void* W, void* C, int c_dtype, int M,
                               int N, int K, hipStream_t stream) {
    if (a_dtype == QMM_DTYPE_F32) {
        if (c_dtype == QMM_DTYPE_F32) return dispatch_p<float, float>(ggml_type, A, W, C, M, N, K, stream);
        return dispatch_p<float, __half>(ggml_type, A, W, C, M, N, K, stream);
    }
    if (c_dtype == QMM_DTYPE_F32) return dispatch_p<__half, float>(ggml_type, A, W, C, M, N, K, stream);
    return dispatch_p<__half, __half>(ggml_type, A, W, C, M, N, K, stream);
}

}  // namespace qmm
