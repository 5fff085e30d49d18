// Prefill GEMM (M >= kGemvMaxM): C[M, N] = A[M, K] @ dequant(W)[N, K]^T on bf16 MFMA with fp32
// accumulation.  Replaces the reference's TILE_M = 4 "prefill" kernels
// (src/kernels/dequantize.hip:152-210, 279-332, 440-505, 616-685), which re-read and re-decode
// every weight for each group of 4 activation rows on the vector ALUs.
//
// MI355X design:
//   * A workgroup (4 waves) owns a 128 (m) x 256 (n) output tile; wave w owns weight rows
//     [64w, 64w + 64) of the tile and all 128 activation rows, as 4 x 2 tiles of
//     v_mfma_f32_32x32x16_bf16 (MFMA A operand = weights, B operand = activations).
//   * K advances in steps of 64.  Each wave dequantizes its own 64 weight rows for the step
//     straight into MFMA fragments (registers, no LDS round trip): a lane reads one
//     contiguous 16-byte piece of code bytes per row and per stream, decodes scales in
//     registers, computes w = a*q - b in fp32 exactly as the reference CPU dequantizer does,
//     and rounds to bf16.  The 64 k of a step are permuted so that every lane's piece is
//     contiguous: MFMA s (0..3), lane half h = lane/32 covers k = kBase[s] + 16h + (0..7).
//   * Activations (fp32 or fp16) are converted to bf16 once per tile and staged in a
//     double-buffered LDS tile (row pitch 72 bf16 = 144 bytes), read with the same permutation.
//   * The next step's activations and weight bytes are loaded while the current step's 32
//     MFMAs run; one barrier per step.
//   * Tiles sharing a weight slice are placed on the same XCD (L2 reuse of the packed bytes).
#include "qmm_device.h"

namespace qmm {
namespace {

constexpr int kPM = 128;        // activation rows per workgroup tile
constexpr int kPN = 256;        // weight rows per workgroup tile (64 per wave)
constexpr int kPK = 64;         // k per step
constexpr int kPitch = 72;      // LDS row pitch of the activation tile, in bf16
constexpr int kPThreads = 256;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4p __attribute__((ext_vector_type(4)));

// k offset (within a 64-k step) of MFMA s's first 8-k chunk for lane half h = 0.
__device__ __forceinline__ int kbase(int s) { return (s & 1) * 8 + (s >> 1) * 32; }

__device__ __forceinline__ u32x4p load16(const uint8_t* p) {
    // Packed GGUF blocks are only 2-byte aligned; global loads accept any alignment.
    u32x4p v;
    __builtin_memcpy(&v, p, 16);
    return v;
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    bf16x2 r;
    r[0] = static_cast<__bf16>(lo);
    r[1] = static_cast<__bf16>(hi);
    uint32_t u;
    __builtin_memcpy(&u, &r, 4);
    return u;
}

// Eight weights a*code - b (one fp32 rounding, as the reference CPU dequantizer) from the
// eight code bytes lo = bytes 0..3, hi = bytes 4..7, rounded to bf16 and packed in pairs.
__device__ __forceinline__ void frag_affine(uint32_t lo, uint32_t hi, float a, float b, uint32_t out[4]) {
    float w[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        w[i] = __fmaf_rn(a, ubyte_to_float(opaque(lo), i), -b);
        w[4 + i] = __fmaf_rn(a, ubyte_to_float(opaque(hi), i), -b);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = pack_bf16(w[2 * i], w[2 * i + 1]);
}

// ----------------------------------------------------------------------------------------
// Per-format weight producers.  raw[] holds the lane's bytes of one row for one step;
// make() writes the 4 fragments (MFMA s = 0..3) of that row.
// ----------------------------------------------------------------------------------------
struct PQ4K {
    static constexpr int kQK = kQK_K, kBytes = kBytesQ4_K, kRaw = 2;
    // step t: super-block t/4, qs chunk c = t%4 (sub-blocks 2c: low nibbles, 2c+1: high).
    __device__ static void load(const uint8_t* row, int t, int h, bool, u32x4p raw[kRaw]) {
        const uint8_t* sb = row + static_cast<size_t>(t >> 2) * kBytes;
        raw[0] = *reinterpret_cast<const u32x4p*>(sb);                            // d, dmin, scales
        raw[1] = *reinterpret_cast<const u32x4p*>(sb + 16 + 32 * (t & 3) + 16 * h);  // 16 qs bytes
    }
    __device__ static void make(const u32x4p raw[kRaw], int t, bool, uint32_t f[4][4], int) {
        const u32x4p hd = raw[0];
        const int c = t & 3;
        uint32_t sc0, m0, sc1, m1;
        q4k_scale_min(2 * c, hd.y, hd.z, hd.w, sc0, m0);
        q4k_scale_min(2 * c + 1, hd.y, hd.z, hd.w, sc1, m1);
        const float d = half_bits_to_float(hd.x), dmin = half_bits_to_float(hd.x >> 16);
        const float a0 = d * static_cast<float>(sc0), b0 = dmin * static_cast<float>(m0);
        const float a1 = d * static_cast<float>(sc1), b1 = dmin * static_cast<float>(m1);
        const u32x4p q = raw[1];
        frag_affine(q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, a0, b0, f[0]);
        frag_affine(q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu, a0, b0, f[1]);
        frag_affine((q.x >> 4) & 0x0F0F0F0Fu, (q.y >> 4) & 0x0F0F0F0Fu, a1, b1, f[2]);
        frag_affine((q.z >> 4) & 0x0F0F0F0Fu, (q.w >> 4) & 0x0F0F0F0Fu, a1, b1, f[3]);
    }
};

struct PQ6K {
    static constexpr int kQK = kQK_K, kBytes = kBytesQ6_K, kRaw = 4;
    // step t: super-block t/4, half n = (t/2)%2, part p = t%2 (p = 0: q1/q2, p = 1: q3/q4).
    __device__ static void load(const uint8_t* row, int t, int h, bool, u32x4p raw[kRaw]) {
        const uint8_t* sb = row + static_cast<size_t>(t >> 2) * kBytes;
        const int n = (t >> 1) & 1;
        raw[0] = load16(sb + 64 * n + 16 * h);           // ql, groups 2p
        raw[1] = load16(sb + 64 * n + 32 + 16 * h);      // ql, groups 2p + 1
        raw[2] = load16(sb + 128 + 32 * n + 16 * h);     // qh
        u32x4p s;                                         // scales 8n..8n+7, then d
        __builtin_memcpy(&s, sb + 192 + 8 * n, 8);
        uint16_t dbits;
        __builtin_memcpy(&dbits, sb + 208, 2);
        s.z = dbits;
        s.w = 0;
        raw[3] = s;
    }
    __device__ static void make(const u32x4p raw[kRaw], int t, bool, uint32_t f[4][4], int h) {
        const int p = t & 1;
        const u32x4p la = raw[0], lb = raw[1], qh = raw[2], sd = raw[3];
        const float d = half_bits_to_float(sd.z);
        // sc[8n + h + 4p] for groups 2p, sc[8n + h + 4p + 2] for groups 2p + 1
        const int sh = 8 * h;
        const uint32_t sw = p ? sd.y : sd.x;
        const float a0 = d * static_cast<float>(static_cast<int8_t>(sw >> sh));
        const float a1 = d * static_cast<float>(static_cast<int8_t>(sw >> (sh + 16)));
        const int ns = 4 * p;             // nibble of ql
        const int hs0 = 4 * p, hs1 = 4 * p + 2;  // qh bit pairs of groups 2p, 2p + 1
        auto codes = [&](uint32_t ql, uint32_t h4, int hs) {
            return ((ql >> ns) & 0x0F0F0F0Fu) | (((h4 >> hs) & 0x03030303u) << 4);
        };
        // codes are unsigned 0..63; w = a * (code - 32) = a*code - 32a (exact: a*code fits fp32).
        frag_affine(codes(la.x, qh.x, hs0), codes(la.y, qh.y, hs0), a0, 32.0f * a0, f[0]);
        frag_affine(codes(la.z, qh.z, hs0), codes(la.w, qh.w, hs0), a0, 32.0f * a0, f[1]);
        frag_affine(codes(lb.x, qh.x, hs1), codes(lb.y, qh.y, hs1), a1, 32.0f * a1, f[2]);
        frag_affine(codes(lb.z, qh.z, hs1), codes(lb.w, qh.w, hs1), a1, 32.0f * a1, f[3]);
    }
};

struct PQ80 {
    static constexpr int kQK = kQK8_0, kBytes = kBytesQ8_0, kRaw = 3;
    // step t: blocks 2t (k 0..31) and 2t + 1 (k 32..63); the second is absent on a K tail.
    __device__ static void load(const uint8_t* row, int t, int h, bool has2, u32x4p raw[kRaw]) {
        const uint8_t* b0 = row + static_cast<size_t>(2 * t) * kBytes;
        const uint8_t* b1 = has2 ? b0 + kBytes : b0;
        raw[0] = load16(b0 + 2 + 16 * h);
        raw[1] = load16(b1 + 2 + 16 * h);
        uint16_t d0, d1;
        __builtin_memcpy(&d0, b0, 2);
        __builtin_memcpy(&d1, b1, 2);
        raw[2] = u32x4p{d0, d1, 0u, 0u};
    }
    __device__ static void make(const u32x4p raw[kRaw], int, bool has2, uint32_t f[4][4], int) {
        const float d0 = half_bits_to_float(raw[2].x);
        const float d1 = has2 ? half_bits_to_float(raw[2].y) : 0.0f;
        // int8 codes enter unsigned (q + 128): w = d*(q+128) - 128d, exact before the subtraction.
        const u32x4p c0 = raw[0] ^ u32x4p{0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
        const u32x4p c1 = raw[1] ^ u32x4p{0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
        frag_affine(c0.x, c0.y, d0, 128.0f * d0, f[0]);
        frag_affine(c0.z, c0.w, d0, 128.0f * d0, f[1]);
        frag_affine(c1.x, c1.y, d1, 128.0f * d1, f[2]);
        frag_affine(c1.z, c1.w, d1, 128.0f * d1, f[3]);
    }
};

struct PQ40 {
    static constexpr int kQK = kQK4_0, kBytes = kBytesQ4_0, kRaw = 3;
    __device__ static void load(const uint8_t* row, int t, int, bool has2, u32x4p raw[kRaw]) {
        const uint8_t* b0 = row + static_cast<size_t>(2 * t) * kBytes;
        const uint8_t* b1 = has2 ? b0 + kBytes : b0;
        raw[0] = load16(b0 + 2);
        raw[1] = load16(b1 + 2);
        uint16_t d0, d1;
        __builtin_memcpy(&d0, b0, 2);
        __builtin_memcpy(&d1, b1, 2);
        raw[2] = u32x4p{d0, d1, 0u, 0u};
    }
    // lane half h takes weights 16h..16h+15 of each block: low nibbles (h = 0) or high (h = 1).
    __device__ static void make(const u32x4p raw[kRaw], int, bool has2, uint32_t f[4][4], int h) {
        const float d0 = half_bits_to_float(raw[2].x);
        const float d1 = has2 ? half_bits_to_float(raw[2].y) : 0.0f;
        const int sh = 4 * h;
        const u32x4p q0 = raw[0], q1 = raw[1];
        frag_affine((q0.x >> sh) & 0x0F0F0F0Fu, (q0.y >> sh) & 0x0F0F0F0Fu, d0, 8.0f * d0, f[0]);
        frag_affine((q0.z >> sh) & 0x0F0F0F0Fu, (q0.w >> sh) & 0x0F0F0F0Fu, d0, 8.0f * d0, f[1]);
        frag_affine((q1.x >> sh) & 0x0F0F0F0Fu, (q1.y >> sh) & 0x0F0F0F0Fu, d1, 8.0f * d1, f[2]);
        frag_affine((q1.z >> sh) & 0x0F0F0F0Fu, (q1.w >> sh) & 0x0F0F0F0Fu, d1, 8.0f * d1, f[3]);
    }
};

// Activation tile staging: thread `tid` converts 32 consecutive k of one row.
template <typename TA>
struct ARegs {
    float v[32];
};

template <typename TA>
__device__ __forceinline__ void load_a(const TA* __restrict__ A, int M, int K, int m0, int k0, int tid, bool vec,
                                       ARegs<TA>& r) {
    const int m = m0 + (tid >> 1);
    const int kk = k0 + 32 * (tid & 1);
    const bool rv = m < M;
    const TA* p = A + static_cast<size_t>(rv ? m : M - 1) * K;
    if (vec && kk + 32 <= K) {
        if constexpr (sizeof(TA) == 4) {
            const float4* q = reinterpret_cast<const float4*>(p + kk);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 u = q[i];
                r.v[4 * i] = u.x; r.v[4 * i + 1] = u.y; r.v[4 * i + 2] = u.z; r.v[4 * i + 3] = u.w;
            }
        } else {
            const uint4* q = reinterpret_cast<const uint4*>(p + kk);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 u = q[i];
                const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    r.v[8 * i + 2 * j] = half_bits_to_float(w[j]);
                    r.v[8 * i + 2 * j + 1] = half_bits_to_float(w[j] >> 16);
                }
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const int k = kk + i;
            float x = 0.0f;
            if (k < K) {
                if constexpr (sizeof(TA) == 4) x = p[k];
                else x = __half2float(p[k]);
            }
            r.v[i] = x;
        }
    }
    if (!rv) {
#pragma unroll
        for (int i = 0; i < 32; ++i) r.v[i] = 0.0f;
    }
}

template <typename TA>
__device__ __forceinline__ void store_a(uint16_t* lds, int tid, const ARegs<TA>& r) {
    uint32_t* dst = reinterpret_cast<uint32_t*>(lds + (tid >> 1) * kPitch + 32 * (tid & 1));
    uint32_t p[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) p[i] = pack_bf16(r.v[2 * i], r.v[2 * i + 1]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        reinterpret_cast<uint4*>(dst)[i] = make_uint4(p[4 * i], p[4 * i + 1], p[4 * i + 2], p[4 * i + 3]);
}

template <class P, typename TA, typename TC>
__global__ __launch_bounds__(kPThreads)
void gemm_prefill_kernel(const TA* __restrict__ A, const uint8_t* __restrict__ W, TC* __restrict__ C,
                         int M, int N, int K, int tiles_m, int tiles, int a_vec, int c_vec) {
    __shared__ __align__(16) uint16_t lds_a[2][kPM * kPitch];

    // XCD-aware tile order: blocks are dealt to the 8 XCDs round-robin, so consecutive tile
    // indices (which share a weight slice) are given to blocks on the same XCD.
    int b = blockIdx.x;
    if (tiles % 8 == 0) b = (b % 8) * (tiles / 8) + b / 8;
    const int tn = b / tiles_m, tm = b % tiles_m;
    const int m0 = tm * kPM, n0 = tn * kPN;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = tid >> 6;
    const int h = lane >> 5;
    const int l32 = lane & 31;
    const bool avec = a_vec != 0;

    // Weight rows of this lane: n0 + 64*wv + 32*r + l32 (clamped; rows past N are never stored).
    const size_t row_bytes = static_cast<size_t>(K / P::kQK) * P::kBytes;
    const uint8_t* wrow[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) wrow[r] = W + static_cast<size_t>(min(n0 + 64 * wv + 32 * r + l32, N - 1)) * row_bytes;

    const int nsteps = (K + kPK - 1) / kPK;

    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][r][v] = 0.0f;

    auto has2 = [&](int t) { return (t + 1) * kPK <= K; };

    u32x4p raw[2][P::kRaw];
    uint32_t wf[2][2][4][4];  // [buffer][row][mfma s][dword]
    ARegs<TA> areg;

    // prologue: step 0
    load_a<TA>(A, M, K, m0, 0, tid, avec, areg);
#pragma unroll
    for (int r = 0; r < 2; ++r) P::load(wrow[r], 0, h, has2(0), raw[r]);
    store_a<TA>(lds_a[0], tid, areg);
#pragma unroll
    for (int r = 0; r < 2; ++r) P::make(raw[r], 0, has2(0), wf[0][r], h);
    __syncthreads();

    auto step = [&](int t, const uint32_t (&wc)[2][4][4], uint32_t (&wn)[2][4][4]) {
        const bool more = t + 1 < nsteps;
        if (more) {
            load_a<TA>(A, M, K, m0, (t + 1) * kPK, tid, avec, areg);
#pragma unroll
            for (int r = 0; r < 2; ++r) P::load(wrow[r], t + 1, h, has2(t + 1), raw[r]);
        }
        const uint16_t* la = lds_a[t & 1];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            bf16x8 wfrag[2];
#pragma unroll
            for (int r = 0; r < 2; ++r) __builtin_memcpy(&wfrag[r], wc[r][s], 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint16_t* src = la + (32 * i + l32) * kPitch + kbase(s) + 16 * h;
                bf16x8 afrag;
                __builtin_memcpy(&afrag, src, 16);
#pragma unroll
                for (int r = 0; r < 2; ++r)
                    acc[i][r] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wfrag[r], afrag, acc[i][r], 0, 0, 0);
            }
        }
        if (more) {
            store_a<TA>(lds_a[(t + 1) & 1], tid, areg);
#pragma unroll
            for (int r = 0; r < 2; ++r) P::make(raw[r], t + 1, has2(t + 1), wn[r], h);
        }
        __syncthreads();
    };

    for (int t = 0; t < nsteps; t += 2) {
        step(t, wf[0], wf[1]);
        if (t + 1 < nsteps) step(t + 1, wf[1], wf[0]);
    }

    // D element v of tile (i, r): weight row n = n0 + 64wv + 32r + 8(v/4) + 4h + v%4,
    // activation row m = m0 + 32i + l32.
    const bool cv = c_vec != 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + 32 * i + l32;
        if (m >= M) continue;
        TC* crow = C + static_cast<size_t>(m) * N;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int n = n0 + 64 * wv + 32 * r + 8 * g + 4 * h;
                const float v0 = acc[i][r][4 * g], v1 = acc[i][r][4 * g + 1];
                const float v2 = acc[i][r][4 * g + 2], v3 = acc[i][r][4 * g + 3];
                if (cv && n + 3 < N) {
                    if constexpr (sizeof(TC) == 4) {
                        *reinterpret_cast<float4*>(crow + n) = make_float4(v0, v1, v2, v3);
                    } else {
                        const uint32_t lo = float_to_half_bits(v0) | (static_cast<uint32_t>(float_to_half_bits(v1)) << 16);
                        const uint32_t hi = float_to_half_bits(v2) | (static_cast<uint32_t>(float_to_half_bits(v3)) << 16);
                        *reinterpret_cast<uint2*>(crow + n) = make_uint2(lo, hi);
                    }
                } else {
                    const float vs[4] = {v0, v1, v2, v3};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (n + e < N) {
                            if constexpr (sizeof(TC) == 4) crow[n + e] = vs[e];
                            else reinterpret_cast<uint16_t*>(crow)[n + e] = float_to_half_bits(vs[e]);
                        }
                    }
                }
            }
        }
    }
}

template <class P, typename TA, typename TC>
hipError_t launch_p(const void* A, const void* W, void* C, int M, int N, int K, hipStream_t stream) {
    const int tiles_m = (M + kPM - 1) / kPM;
    const int tiles_n = (N + kPN - 1) / kPN;
    const int tiles = tiles_m * tiles_n;
    const bool a_vec = (reinterpret_cast<uintptr_t>(A) & 15u) == 0;
    const bool c_vec = (reinterpret_cast<uintptr_t>(C) & 15u) == 0 && N % 4 == 0;
    hipLaunchKernelGGL((gemm_prefill_kernel<P, TA, TC>), dim3(tiles), dim3(kPThreads), 0, stream,
                       static_cast<const TA*>(A), static_cast<const uint8_t*>(W), static_cast<TC*>(C), M, N, K,
                       tiles_m, tiles, a_vec ? 1 : 0, c_vec ? 1 : 0);
    return hipGetLastError();
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
    (void)ggml_type; (void)a_dtype; (void)c_dtype; (void)W;
    // Q4_K rows are read with 16-byte aligned loads: the packed matrix must start 16-byte aligned.
    if (ggml_type == QMM_TYPE_Q4_K && (reinterpret_cast<uintptr_t>(W) & 15u) != 0) return false;
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
