// Prefill GEMM (M >= kGemvMaxM): C[M, N] = A[M, K] @ dequant(W)[N, K]^T on f16 MFMA with fp32
// accumulation.  Replaces the reference's TILE_M = 4 "prefill" kernels
// (src/kernels/dequantize.hip:152-210, 279-332, 440-505, 616-685), which re-read and re-decode
// every weight for each group of 4 activation rows on the vector ALUs.
//
// MI355X design:
//   * Operands are f16 (v_mfma_f32_32x32x16_f16, fp32 accumulation).  The reference's API hands
//     over fp16 activations; f16 keeps three more mantissa bits than bf16 at the same MFMA rate.
//     fp32 activations are rounded to f16 once by a conversion pass into a workspace.
//   * A workgroup (4 waves) owns a 128 (m) x 256 (n) output tile and walks its K range in steps of
//     64; wave w owns weight rows [64w, 64w + 64) of the tile and all 128 activation rows (4 x 2
//     MFMA tiles of 32 x 32).
//   * Activation tiles are double-buffered in LDS: the next step's tile is loaded into registers
//     while the current one is multiplied and written to the free slot at the end of the step
//     (one barrier per step).  Rows are XOR-swizzled so fragment reads are bank-conflict free;
//     each fragment is read once per step and feeds both of the wave's weight tiles.
//   * Each wave dequantizes its own weight rows straight into MFMA fragments with packed f16
//     math: one v_perm makes two (1024 + code) f16 values, v_pk_add_f16 removes the offset
//     exactly, v_pk_fma_f16 applies the group's scale and min (one rounding to f16).  Raw
//     bytes are loaded one step ahead.
//   * Narrow N (few tiles): the K range is split over workgroups; partial tiles land in a
//     workspace and a second pass adds them in a fixed order (deterministic).
//   * Tiles sharing a weight slice are placed on the same XCD (L2 reuse of the packed bytes).
#include <mutex>
#include <string>
#include <type_traits>
#include <unordered_map>

#include "qmm_device.h"

namespace qmm {
namespace {

constexpr int kBM = 128;        // activation rows per workgroup tile
constexpr int kBN = 256;        // weight rows per workgroup tile (64 per wave)
constexpr int kBK = 64;         // k per step
constexpr int kThreads = 256;
constexpr int kChunksPerStage = kBM * kBK / 8;  // 16-byte chunks (8 f16) per stage = 1024

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
// Weight producers.  MFMA s (0..3) of a step and lane half h cover step-relative
// k = 32*(s>>1) + 16*h + 8*(s&1) + (0..7); make() writes the 4 fragments (8 f16 each, natural k
// order) of one weight row.
// ---------------------------------------------------------------------------------------------
struct PQ4K {
    static constexpr int kQK = kQK_K, kBytes = kBytesQ4_K;
    struct Raw { u32x4p hd, q; };
    // step at k0 (multiple of 64): super-block k0/256, qs chunk c = (k0/64)%4; lane half h takes
    // qs bytes 16h..16h+15 of the chunk (low nibbles: sub-block 2c, high: 2c+1).
    __device__ static Raw load(const uint8_t* row, int k0, int h, int) {
        const uint8_t* sb = row + static_cast<size_t>(k0 >> 8) * kBytes;
        Raw r;
        r.hd = *reinterpret_cast<const u32x4p*>(sb);
        r.q = *reinterpret_cast<const u32x4p*>(sb + 16 + 32 * ((k0 >> 6) & 3) + 16 * h);
        return r;
    }
    __device__ static void make(const Raw& r, int k0, int, uint32_t f[4][4]) {
        // 6-bit scales/mins of sub-blocks 2c and 2c + 1 (bytes 2(c&1), 2(c&1)+1 of the packed
        // scale words; sub-blocks 4..7 take their top bits from words 0/1).  c is uniform, so the
        // choice is a select, not a branch.
        const int c = (k0 >> 6) & 3;
        const int sh = 16 * (c & 1);
        const uint32_t u0 = r.hd.y >> sh, u1 = r.hd.z >> sh, u2 = r.hd.w >> sh;
        const uint32_t sc_lo = u0 & 0x3F3Fu, m_lo = u1 & 0x3F3Fu;
        const uint32_t sc_hi = (u2 & 0x0F0Fu) | ((u0 >> 2) & 0x3030u);
        const uint32_t m_hi = ((u2 >> 4) & 0x0F0Fu) | ((u1 >> 2) & 0x3030u);
        const uint32_t scp = c >= 2 ? sc_hi : sc_lo, mp = c >= 2 ? m_hi : m_lo;
        const uint32_t sc0 = scp & 0xFFu, sc1 = (scp >> 8) & 0xFFu, m0 = mp & 0xFFu, m1 = (mp >> 8) & 0xFFu;
        const float d = half_bits_to_float(r.hd.x), dmin = half_bits_to_float(r.hd.x >> 16);
        const h2 a0 = splat(d * static_cast<float>(sc0)), b0 = splat(-(dmin * static_cast<float>(m0)));
        const h2 a1 = splat(d * static_cast<float>(sc1)), b1 = splat(-(dmin * static_cast<float>(m1)));
        const h2 off = splat(1024.0f);
        const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const bool hi = s >= 2;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t x = w[2 * (s & 1) + j];
                const uint32_t codes = hi ? ((x >> 4) & 0x0F0F0F0Fu) : (x & 0x0F0F0F0Fu);
                h2 p, q;
                bytes_to_h2(codes, off, p, q);
                f[s][2 * j] = affine(p, hi ? a1 : a0, hi ? b1 : b0);
                f[s][2 * j + 1] = affine(q, hi ? a1 : a0, hi ? b1 : b0);
            }
        }
    }
};

struct PQ6K {
    static constexpr int kQK = kQK_K, kBytes = kBytesQ6_K;
    struct Raw { u32x4p la, lb, qh; uint32_t sc, d; };
    // step at k0: super-block k0/256, quarter qt = (k0/64)%4 -> half n2 = qt/2, groups t = 2(qt&1) + (s>>1);
    // lane half h takes l = 16h..16h+15 of ql (groups t even: ql[64n2 + l], odd: ql[64n2 + 32 + l]) and qh.
    __device__ static Raw load(const uint8_t* row, int k0, int h, int) {
        const uint8_t* sb = row + static_cast<size_t>(k0 >> 8) * kBytes;
        const int qt = (k0 >> 6) & 3, n2 = qt >> 1;
        Raw r;
        r.la = ld16(sb + 64 * n2 + 16 * h);
        r.lb = ld16(sb + 64 * n2 + 32 + 16 * h);
        r.qh = ld16(sb + 128 + 32 * n2 + 16 * h);
        r.sc = ld4(sb + 192 + 8 * n2 + 4 * (qt & 1));  // sc[.. + h + {0, 2}]
        r.d = ld2(sb + 208);
        return r;
    }
    __device__ static void make(const Raw& r, int k0, int h, uint32_t f[4][4]) {
        const int qt = (k0 >> 6) & 3;
        const int nib = 4 * (qt & 1);
        const float d = half_bits_to_float(r.d);
        const h2 a0 = splat(d * static_cast<float>(static_cast<int8_t>(r.sc >> (8 * h))));
        const h2 a1 = splat(d * static_cast<float>(static_cast<int8_t>(r.sc >> (8 * h + 16))));
        const h2 off = splat(1056.0f);  // 1024 + 32: codes q enter as 1024 + q, weight is a (q - 32)
        const uint32_t la[4] = {r.la.x, r.la.y, r.la.z, r.la.w};
        const uint32_t lb[4] = {r.lb.x, r.lb.y, r.lb.z, r.lb.w};
        const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int u = s >> 1;  // group t = 2(qt&1) + u
            const int hs = nib + 2 * u;  // qh bit pair of the group
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int i = 2 * (s & 1) + j;
                const uint32_t lo4 = ((u ? lb[i] : la[i]) >> nib) & 0x0F0F0F0Fu;
                const uint32_t hi2 = ((qh[i] >> hs) & 0x03030303u) << 4;
                h2 p, q;
                bytes_to_h2(lo4 | hi2, off, p, q);
                const h2 a = u ? a1 : a0;
                f[s][2 * j] = as_u32(p * a);
                f[s][2 * j + 1] = as_u32(q * a);
            }
        }
    }
};

struct PQ80 {
    static constexpr int kQK = kQK8_0, kBytes = kBytesQ8_0;
    struct Raw { u32x4p q0, q1; uint32_t d0, d1; };
    // step at k0: blocks k0/32 (k 0..31) and k0/32 + 1 (k 32..63, absent on a K tail)
    __device__ static Raw load(const uint8_t* row, int k0, int h, int kv) {
        const uint8_t* b0 = row + static_cast<size_t>(k0 >> 5) * kBytes;
        const uint8_t* b1 = kv > 32 ? b0 + kBytes : b0;
        Raw r;
        r.q0 = ld16(b0 + 2 + 16 * h);
        r.q1 = ld16(b1 + 2 + 16 * h);
        r.d0 = ld2(b0);
        const uint32_t d1 = ld2(b1);  // always issued (static load count); zero scale on a K tail
        r.d1 = kv > 32 ? d1 : 0u;
        return r;
    }
    __device__ static void make(const Raw& r, int, int, uint32_t f[4][4]) {
        const h2 a0 = splat(half_bits_to_float(r.d0)), a1 = splat(half_bits_to_float(r.d1));
        const h2 off = splat(1152.0f);  // signed codes enter as 1024 + (q + 128)
        const uint32_t q0[4] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w};
        const uint32_t q1[4] = {r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int u = s >> 1;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int i = 2 * (s & 1) + j;
                h2 p, q;
                bytes_to_h2((u ? q1[i] : q0[i]) ^ 0x80808080u, off, p, q);
                const h2 a = u ? a1 : a0;
                f[s][2 * j] = as_u32(p * a);
                f[s][2 * j + 1] = as_u32(q * a);
            }
        }
    }
};

struct PQ40 {
    static constexpr int kQK = kQK4_0, kBytes = kBytesQ4_0;
    struct Raw { u32x4p q0, q1; uint32_t d0, d1; };
    // step at k0: blocks k0/32 and k0/32 + 1; lane half h takes the block's low (h = 0, k 0..15)
    // or high (h = 1, k 16..31) nibbles.
    __device__ static Raw load(const uint8_t* row, int k0, int, int kv) {
        const uint8_t* b0 = row + static_cast<size_t>(k0 >> 5) * kBytes;
        const uint8_t* b1 = kv > 32 ? b0 + kBytes : b0;
        Raw r;
        r.q0 = ld16(b0 + 2);
        r.q1 = ld16(b1 + 2);
        r.d0 = ld2(b0);
        const uint32_t d1 = ld2(b1);  // always issued (static load count); zero scale on a K tail
        r.d1 = kv > 32 ? d1 : 0u;
        return r;
    }
    __device__ static void make(const Raw& r, int, int h, uint32_t f[4][4]) {
        const h2 a0 = splat(half_bits_to_float(r.d0)), a1 = splat(half_bits_to_float(r.d1));
        const h2 off = splat(1032.0f);  // codes enter as 1024 + q, weight is d (q - 8)
        const uint32_t q0[4] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w};
        const uint32_t q1[4] = {r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int u = s >> 1;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int i = 2 * (s & 1) + j;
                h2 p, q;
                bytes_to_h2(((u ? q1[i] : q0[i]) >> (4 * h)) & 0x0F0F0F0Fu, off, p, q);
                const h2 a = u ? a1 : a0;
                f[s][2 * j] = as_u32(p * a);
                f[s][2 * j + 1] = as_u32(q * a);
            }
        }
    }
};

template <class P>
constexpr int raw_loads() {
    return std::is_same<P, PQ4K>::value ? 2 : std::is_same<P, PQ6K>::value ? 5 : 4;
}

// Activation chunk (row r, chunk c = 8 f16) position inside a 1024-chunk stage: rows are
// XOR-swizzled so that 16 consecutive rows read at one chunk hit 16 different bank groups.
__device__ __forceinline__ int a_slot(int r, int c) { return 8 * r + (c ^ ((r >> 1) & 7)); }

// MFMA s, lane half h -> activation chunk of the step.
__device__ __forceinline__ int a_chunk(int s, int h) { return 4 * (s >> 1) + 2 * h + (s & 1); }

// Workgroup barrier for LDS traffic only: this wave's LDS writes are complete, then s_barrier.
// Unlike __syncthreads() it does not wait for outstanding global loads (the prefetches stay in
// flight); the empty asm statements keep the compiler from moving memory operations across it.
__device__ __forceinline__ void lds_barrier() {
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

template <class P, typename TC>
__global__ __launch_bounds__(kThreads, 1)
void prefill_kernel(const _Float16* __restrict__ A16, int lda, const uint8_t* __restrict__ W, TC* __restrict__ C,
                    float* __restrict__ part, int M, int N, int K, int klen, int tiles_m, int tiles_n, int ksplit) {
    __shared__ __align__(16) u32x4p sA[2][kChunksPerStage];

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
    const uint8_t* wrow[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) wrow[r] = W + static_cast<size_t>(min(n0 + 64 * wv + 32 * r + l32, N - 1)) * row_bytes;

    // Thread tid copies stage chunks p = tid + 256 j (j = 0..3): row p >> 3, chunk (p & 7) ^ swizzle,
    // so each thread's 4 global reads are 16-byte aligned f16 runs and its LDS writes are in place.
    const _Float16* arow[4];
    int apos[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int p = tid + 256 * j;
        const int r = p >> 3;
        const int c = (p & 7) ^ ((r >> 1) & 7);
        arow[j] = A16 + static_cast<size_t>(min(m0 + r, M - 1)) * lda + kb + 8 * c;
        apos[j] = p;
    }
    auto load_a = [&](int t, u32x4p (&ar)[4]) {
        const int kk = min(t, nsteps - 1) * kBK;  // past the end: re-read the last step
#pragma unroll
        for (int j = 0; j < 4; ++j) ar[j] = *reinterpret_cast<const u32x4p*>(arow[j] + kk);
    };
    auto store_a = [&](int slot, const u32x4p (&ar)[4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) sA[slot][apos[j]] = ar[j];
    };
    auto load_raw = [&](int t, typename P::Raw (&raw)[2]) {
        const int k0 = kb + min(t, nsteps - 1) * kBK;
#pragma unroll
        for (int r = 0; r < 2; ++r) raw[r] = P::load(wrow[r], k0, h, kend - k0);
    };

    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][r][v] = 0.0f;

    // Pipeline: at step t the LDS slot t%2 holds A(t); A(t+1) and the raw weight bytes of step t+1
    // are in flight in registers while step t is multiplied.  At the end of the step A(t+1) goes
    // to the other slot and the raw bytes move into `cur`.  One loop body keeps the accumulators
    // in place (no register renaming across unrolled copies).
    u32x4p an[4];
    typename P::Raw cur[2], nxt[2];
    load_a(0, an);
    load_raw(0, cur);
    store_a(0, an);
    lds_barrier();

    for (int t = 0; t < nsteps; ++t) {
        load_a(t + 1, an);
        load_raw(t + 1, nxt);
        // Keep the prefetches at the top of the step: left alone, the scheduler sinks them next
        // to their uses at the end of the step and their latency is no longer hidden.
        __builtin_amdgcn_sched_barrier(0);
        const int k0 = kb + t * kBK;
        uint32_t wf[2][4][4];
#pragma unroll
        for (int r = 0; r < 2; ++r) P::make(cur[r], k0, h, wf[r]);
        const u32x4p* sa = sA[t & 1];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            f16x8 af[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const u32x4p av = sa[a_slot(32 * i + l32, a_chunk(s, h))];
                __builtin_memcpy(&af[i], &av, 16);
            }
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                f16x8 bw;
                __builtin_memcpy(&bw, wf[r][s], 16);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[i][r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bw, af[i], acc[i][r], 0, 0, 0);
            }
        }
        store_a((t + 1) & 1, an);
        lds_barrier();
#pragma unroll
        for (int r = 0; r < 2; ++r) cur[r] = nxt[r];
    }

    // D element v of tile (i, r): weight row n = n0 + 64wv + 32r + 8(v/4) + 4h + v%4,
    // activation row m = m0 + 32i + l32.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 32 * i + l32;
        if (m >= M) continue;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = n0 + 64 * wv + 32 * r + 8 * g + 4 * h;
                const float vs[4] = {acc[i][r][4 * g], acc[i][r][4 * g + 1], acc[i][r][4 * g + 2], acc[i][r][4 * g + 3]};
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
    // 4 * (ksplit + 1) * M * N bytes), keeping at least 16 steps per split
    int ksplit = 1;
    while (tiles_m * tiles_n * ksplit * 2 <= cus && steps / (ksplit * 2) >= 16) ksplit *= 2;
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
