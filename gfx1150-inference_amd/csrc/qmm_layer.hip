// The transformer layer around the quantized projections, device-resident: RMSNorm (plain and
// fused with the residual add), RoPE with the KV-cache write, grouped-query attention over the
// cache, SwiGLU, the residual add, the KV-cache pool and the layer pipeline that chains them
// with the fused projection launches.
//
// Reference: src/kernels/rmsnorm.hip, rope.hip, attention.hip (gqa_online_softmax_kernel :35-123,
// DeviceKVCachePool :164-222, launch_forward_layer_cached_fp16 :603-695), mlp.hip.  Storage is
// fp16 and arithmetic fp32 with one rounding per stored value, as there.
//
// MI355X design:
//   * RMSNorm: one workgroup (4 waves) per row, 16-byte loads, wave64 DPP reductions.
//   * RoPE: one launch rotates q into its buffer, rotates k straight into the layer's K cache
//     at the token positions and copies v into the V cache (the reference copies K/V into the
//     pool separately); inverse frequencies come from the host in fp32, as in the reference.
//   * Attention: split over the KV length.  A wave owns (query row, query head, chunk of 64
//     keys): lanes hold head_dim / 64 consecutive query dimensions; keys are loaded 8 at a time
//     (8 rows in flight per wave), their dot products reduced across the wave together, and an
//     fp32 online softmax updates the running output.  Chunks are merged in a fixed order by a
//     second pass (deterministic), skipped for one chunk.  The query heads of one KV head sit
//     in one workgroup, so their K/V reads share the caches.
//   * SwiGLU and the residual add: 8 values per thread.
//   * Layer: q/k/v and gate/up each run as one fused projection launch (qmm_gemm_batch), all
//     kernels on the caller's stream with no host synchronisation; activations live in a
//     grow-only per-(device, stream) workspace.
#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "qmm_device.h"

namespace qmm {
namespace {

constexpr int kNormThreads = 256;
constexpr int kAttnChunk = 64;       // keys per attention chunk (one wave each)
constexpr int kMaxHeadDim = 256;
constexpr int kMaxRopePairs = kMaxHeadDim / 2;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// fp32 acc + the dot product of two f16 pairs (v_dot2_f32_f16)
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    h2v x, y;
    __builtin_memcpy(&x, &a, 4);
    __builtin_memcpy(&y, &b, 4);
    return __builtin_amdgcn_fdot2(x, y, acc, false);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float norm_weight(const void* w, int w_f32, int k) {
    // an F32 norm weight is rounded to f16 first, as the reference's host does
    if (w_f32) return static_cast<float>(static_cast<_Float16>(static_cast<const float*>(w)[k]));
    return static_cast<float>(static_cast<const _Float16*>(w)[k]);
}

// out[m] = half(v * rsqrt(mean(v^2) + eps) * w) with v = x[m] (res == nullptr) or
// v = half(x[m] + res[m]) (stored to h_out in the first pass and read back in the second, so
// h_out may alias x or res; out may alias x).  Each thread reads and writes only its own
// elements across the two passes.
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const _Float16* x, const _Float16* res,
                                                              const void* __restrict__ w, int w_f32, _Float16* h_out,
                                                              _Float16* out, int K, float eps) {
    const int m = blockIdx.x;
    const size_t base = static_cast<size_t>(m) * K;
    const int tid = threadIdx.x;
    const bool vec = (K % 8) == 0;
    auto value = [&](int k) -> float {
        if (res == nullptr) return static_cast<float>(x[base + k]);
        return static_cast<float>(static_cast<_Float16>(static_cast<float>(x[base + k]) + static_cast<float>(res[base + k])));
    };
    float ss = 0.0f;
    if (vec) {
        for (int c = tid; c < K / 8; c += kNormThreads) {
            const h8 a = *reinterpret_cast<const h8*>(x + base + 8 * c);
            h8 v = a;
            if (res != nullptr) {
                const h8 r = *reinterpret_cast<const h8*>(res + base + 8 * c);
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = static_cast<_Float16>(static_cast<float>(a[e]) + static_cast<float>(r[e]));
                *reinterpret_cast<h8*>(h_out + base + 8 * c) = v;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float f = static_cast<float>(v[e]);
                ss += f * f;
            }
        }
    } else {
        for (int k = tid; k < K; k += kNormThreads) {
            const float f = value(k);
            if (res != nullptr) h_out[base + k] = static_cast<_Float16>(f);
            ss += f * f;
        }
    }
    __shared__ float part[kNormThreads / 64];
    ss = wave_sum(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormThreads / 64; ++i) tot += part[i];
    const float scale = rsqrtf(tot / static_cast<float>(K) + eps);
    const _Float16* src = res == nullptr ? x : h_out;
    if (vec) {
        for (int c = tid; c < K / 8; c += kNormThreads) {
            const h8 v = *reinterpret_cast<const h8*>(src + base + 8 * c);
            h8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = static_cast<_Float16>(static_cast<float>(v[e]) * scale * norm_weight(w, w_f32, 8 * c + e));
            *reinterpret_cast<h8*>(out + base + 8 * c) = o;
        }
    } else {
        for (int k = tid; k < K; k += kNormThreads)
            out[base + k] = static_cast<_Float16>(static_cast<float>(src[base + k]) * scale * norm_weight(w, w_f32, k));
    }
}

// out = half(x + r), 8 values per thread (n % 8 == 0) or one.
__global__ __launch_bounds__(256) void residual_add_kernel(const _Float16* __restrict__ x, const _Float16* __restrict__ r,
                                                          _Float16* __restrict__ out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if ((n & 7) == 0) {
        if (8 * i >= n) return;
        const h8 a = *reinterpret_cast<const h8*>(x + 8 * i);
        const h8 b = *reinterpret_cast<const h8*>(r + 8 * i);
        h8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = static_cast<_Float16>(static_cast<float>(a[e]) + static_cast<float>(b[e]));
        *reinterpret_cast<h8*>(out + 8 * i) = o;
    } else if (i < n) {
        out[i] = static_cast<_Float16>(static_cast<float>(x[i]) + static_cast<float>(r[i]));
    }
}

// out = half(silu(g) * u), silu(g) = g / (1 + exp(-g)).
// y[r, i] = f16(f32(y[r, i]) + f32(b[i])) over `rows` rows of n values: a projection's bias added in
// fp32 to its fp16 output and rounded once (reference src/layer.py:274-282, 344-346).
__global__ __launch_bounds__(256) void bias_add_kernel(_Float16* __restrict__ y, const _Float16* __restrict__ b, int n,
                                                       int64_t total) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total; i += stride)
        y[i] = static_cast<_Float16>(static_cast<float>(y[i]) + static_cast<float>(b[i % n]));
}

__global__ __launch_bounds__(256) void swiglu_kernel(const _Float16* __restrict__ g, const _Float16* __restrict__ u,
                                                    _Float16* __restrict__ out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    auto f = [](float gv, float uv) { return static_cast<_Float16>(gv / (1.0f + expf(-gv)) * uv); };
    if ((n & 7) == 0) {
        if (8 * i >= n) return;
        const h8 a = *reinterpret_cast<const h8*>(g + 8 * i);
        const h8 b = *reinterpret_cast<const h8*>(u + 8 * i);
        h8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = f(static_cast<float>(a[e]), static_cast<float>(b[e]));
        *reinterpret_cast<h8*>(out + 8 * i) = o;
    } else if (i < n) {
        out[i] = f(static_cast<float>(g[i]), static_cast<float>(u[i]));
    }
}

struct RopeFreq {
    float inv[kMaxRopePairs];
};

// Rotates pairs of q (n_q heads) into q_out and of k (n_k heads) into k_out, and copies v
// (n_k heads) into v_out; rows are token positions pos_offset + s.  q_out / k_out / v_out row
// strides are given in elements (the KV cache rows hold n_k heads).  One thread per pair.
__global__ __launch_bounds__(256) void rope_kernel(const _Float16* __restrict__ q, _Float16* __restrict__ q_out, int n_q,
                                                  const _Float16* __restrict__ k, _Float16* __restrict__ k_out,
                                                  const _Float16* __restrict__ v, _Float16* __restrict__ v_out, int n_k,
                                                  int seq_len, int head_dim, int pos_offset, int neox, RopeFreq fr) {
    const int half_dim = head_dim / 2;
    const int heads = n_q + n_k;
    const int64_t total = static_cast<int64_t>(seq_len) * heads * half_dim;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) return;
    const int p = static_cast<int>(idx % half_dim);
    const int64_t t = idx / half_dim;
    const int hh = static_cast<int>(t % heads);
    const int s = static_cast<int>(t / heads);
    const float ang = static_cast<float>(pos_offset + s) * fr.inv[p];
    const float c = cosf(ang), sn = sinf(ang);
    const int i0 = neox ? p : 2 * p;
    const int i1 = neox ? p + half_dim : 2 * p + 1;
    const _Float16* src;
    _Float16* dst;
    if (hh < n_q) {
        src = q + (static_cast<size_t>(s) * n_q + hh) * head_dim;
        dst = q_out + (static_cast<size_t>(s) * n_q + hh) * head_dim;
    } else {
        const int kh = hh - n_q;
        src = k + (static_cast<size_t>(s) * n_k + kh) * head_dim;
        dst = k_out + (static_cast<size_t>(s) * n_k + kh) * head_dim;
        if (v != nullptr) {
            const _Float16* vs = v + (static_cast<size_t>(s) * n_k + kh) * head_dim;
            _Float16* vd = v_out + (static_cast<size_t>(s) * n_k + kh) * head_dim;
            vd[i0] = vs[i0];
            vd[i1] = vs[i1];
        }
    }
    const float a = static_cast<float>(src[i0]), b = static_cast<float>(src[i1]);
    dst[i0] = static_cast<_Float16>(a * c - b * sn);
    dst[i1] = static_cast<_Float16>(a * sn + b * c);
}

// Attention, one wave per (query row m, query head h, key chunk c).  Lane l holds the D
// consecutive dimensions D*l .. D*l + D - 1 of the head (head_dim <= 64 D), so a key row is one
// coalesced read across the wave.  Keys are taken 8 at a time: the 8 K and V rows are loaded
// together (8 reads in flight per wave instead of one), the 8 dot products are reduced across
// the wave together, then the fp32 online softmax takes them in key order.  Partial results
// (running max, sum and unnormalised output), or the fp16 output when there is one chunk.
template <int D>
__global__ __launch_bounds__(256) void attention_kernel(const _Float16* __restrict__ Q, const _Float16* __restrict__ Kc,
                                                       const _Float16* __restrict__ Vc, _Float16* __restrict__ out,
                                                       float* __restrict__ part, int q_len, int kv_len, int heads,
                                                       int kv_heads, int head_dim, int start_pos, float scale, int causal,
                                                       int chunks) {
    constexpr int G = 8;  // keys per batch
    const int lane = threadIdx.x & 63;
    // wave-uniform (scalar registers), so the head, chunk and row arithmetic below is scalar
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t total = static_cast<int64_t>(q_len) * heads * chunks;
    if (wave >= total) return;
    // waves of one workgroup: consecutive heads of the same (m, c), so the query heads that share
    // a KV head (consecutive h) read the same keys
    const int h = static_cast<int>(wave % heads);
    const int64_t t = wave / heads;
    const int c = static_cast<int>(t % chunks);
    const int m = static_cast<int>(t / chunks);
    const int group = heads / kv_heads;
    const int kvh = h / group;
    const int n_keys = causal ? min(kv_len, start_pos + m + 1) : kv_len;
    const int s0 = c * kAttnChunk;
    const int s1 = min(n_keys, s0 + kAttnChunk);
    const bool full = head_dim == 64 * D;  // every lane owns D valid dims: vector reads
    const int d0 = D * lane;

    auto load = [&](const _Float16* p, float (&o)[D]) {
        if (full) {
            _Float16 v[D];
            __builtin_memcpy(v, p + d0, sizeof(v));
#pragma unroll
            for (int i = 0; i < D; ++i) o[i] = static_cast<float>(v[i]);
        } else {
#pragma unroll
            for (int i = 0; i < D; ++i) o[i] = d0 + i < head_dim ? static_cast<float>(p[d0 + i]) : 0.0f;
        }
    };
    float qv[D], acc[D];
    load(Q + (static_cast<size_t>(m) * heads + h) * head_dim, qv);
#pragma unroll
    for (int i = 0; i < D; ++i) acc[i] = 0.0f;
    float mx = -INFINITY, sum = 0.0f;
    const size_t row = static_cast<size_t>(kv_heads) * head_dim;
    const _Float16* kbase = Kc + static_cast<size_t>(kvh) * head_dim;
    const _Float16* vbase = Vc + static_cast<size_t>(kvh) * head_dim;
    for (int s = s0; s < s1; s += G) {
        const int n = min(G, s1 - s);
        float kk[G][D], vv[G][D];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const size_t r = static_cast<size_t>(s + min(j, n - 1));  // rows past the end re-read the last
            load(kbase + r * row, kk[j]);
            load(vbase + r * row, vv[j]);
        }
        float dot[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
            dot[j] = 0.0f;
#pragma unroll
            for (int i = 0; i < D; ++i) dot[j] += qv[i] * kk[j][i];
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
#pragma unroll
            for (int j = 0; j < G; ++j) dot[j] += __shfl_xor(dot[j], o, 64);
#pragma unroll
        for (int j = 0; j < G; ++j) {
            if (j < n) {
                const float sc = dot[j] * scale;
                const float mn = fmaxf(mx, sc);
                const float a = expf(mx - mn);  // exp(-inf) = 0 for the first key
                const float e = expf(sc - mn);
                sum = sum * a + e;
#pragma unroll
                for (int i = 0; i < D; ++i) acc[i] = acc[i] * a + e * vv[j][i];
                mx = mn;
            }
        }
    }
    auto store = [&](auto* dst, auto cvt) {
        if (full) {
#pragma unroll
            for (int i = 0; i < D; ++i) dst[d0 + i] = cvt(acc[i]);
        } else {
#pragma unroll
            for (int i = 0; i < D; ++i)
                if (d0 + i < head_dim) dst[d0 + i] = cvt(acc[i]);
        }
    };
    if (chunks == 1) {
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        store(out + (static_cast<size_t>(m) * heads + h) * head_dim, [&](float v) { return static_cast<_Float16>(v * inv); });
        return;
    }
    float* pp = part + static_cast<size_t>(wave) * (head_dim + 2);
    if (lane == 0) {
        pp[0] = mx;
        pp[1] = sum;
    }
    store(pp + 2, [](float v) { return v; });
}

// Attention for head_dim a multiple of 8 up to 128, one wave per (query row m, query head h, chunk
// of 64 keys), with lanes over keys for the scores and over dimensions for the output:
//   * lane j reads the whole K row of key s0 + j (16-byte loads, all in flight at once) and
//     forms q . k with v_dot2 on f16 pairs (q is the same for every lane);
//   * one wave max and one wave sum give the chunk's softmax statistics;
//   * lane l then owns dims 2l, 2l + 1 of the output, reads the V rows of all the chunk's keys at
//     once and accumulates p_j v_j with p_j broadcast from lane j.
// Output: partial results (max, sum, unnormalised output) as attention_kernel, or fp16 output
// when there is one chunk.
// With kRope (one query row, the decode step): Q, k_new and v_new are the projections before
// RoPE; each wave rotates its query into LDS, the new key (position start_pos) is rotated into LDS
// and stands in for its cache row, and the first query head of each KV head's group writes the
// rotated key and the value into the cache row.  No wave of the launch uses that row's cache
// contents: the new key's lane takes the rotated key from LDS and its value from v_new (a load
// of the row issued for a masked or replaced lane is discarded).
struct DecodeRope {
    const _Float16* k_new;  // [kv_heads][head_dim]
    const _Float16* v_new;
    _Float16* kc;           // the layer's K / V cache (rows of kv_heads * head_dim)
    _Float16* vc;
    int neox;
    float cs[kMaxRopePairs / 2], sn[kMaxRopePairs / 2];  // cos / sin of pair p's angle at the new position
};

template <bool kRope>
__global__ __launch_bounds__(256) void attention_keys_kernel(const _Float16* __restrict__ Q, const _Float16* __restrict__ Kc,
                                                            const _Float16* __restrict__ Vc, _Float16* __restrict__ out,
                                                            float* __restrict__ part, int q_len, int kv_len, int heads,
                                                            int kv_heads, int head_dim, int start_pos, float scale,
                                                            int causal, int chunks, DecodeRope dr) {
    constexpr int kMaxPairs = 64;  // head_dim <= 128
    const int lane = threadIdx.x & 63;
    // wave-uniform (scalar registers), so the head, chunk and row arithmetic below is scalar
    const int wl = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + wl;
    const int64_t total = static_cast<int64_t>(q_len) * heads * chunks;
    if (wave >= total) return;
    const int h = static_cast<int>(wave % heads);
    const int64_t t = wave / heads;
    const int c = static_cast<int>(t % chunks);
    const int m = static_cast<int>(t / chunks);
    const int kvh = h / (heads / kv_heads);
    const int n_keys = causal ? min(kv_len, start_pos + m + 1) : kv_len;
    const int s0 = c * kAttnChunk;
    const int n = max(0, min(n_keys, s0 + kAttnChunk) - s0);  // keys of this chunk
    const int pairs = head_dim / 2;
    const size_t row = static_cast<size_t>(kv_heads) * head_dim;

    // scores: lane j <-> key s0 + j (lanes past the chunk re-read its first key and are masked)
    const uint32_t* qp = reinterpret_cast<const uint32_t*>(Q + (static_cast<size_t>(m) * heads + h) * head_dim);
    const int pos = start_pos + m;                       // the new key (kRope: m == 0)
    const int j_new = kRope && pos >= s0 && pos < s0 + kAttnChunk ? pos - s0 : -1;
    // The chunk's K and V rows are requested first: they do not depend on the rotation below, so
    // one memory round trip covers them, the query and the new key.
    // A dummy lane (and the new key's lane, which takes its key from LDS) reads a row below the
    // new key: s0 when the new key is not the chunk's first, else row 0 (pos > 0), else it is masked
    const int dummy = j_new == 0 ? 0 : s0;
    const int sj = lane < n && lane != j_new ? s0 + lane : (kRope ? min(dummy, max(pos - 1, 0)) : s0);
    const u32x4* kr = reinterpret_cast<const u32x4*>(Kc + static_cast<size_t>(sj) * row + static_cast<size_t>(kvh) * head_dim);
    u32x4 kv[kMaxPairs / 4];
#pragma unroll
    for (int i = 0; i < kMaxPairs / 4; ++i)
        if (4 * i < pairs) kv[i] = kr[i];
    // the chunk's V rows are requested together with the K rows (they do not depend on the scores):
    // lane l <-> dims 2l, 2l + 1 of every row; rows past the chunk re-read its last key
    const bool own = 2 * lane < head_dim;
    const int vl = own ? lane : 0;
    const uint32_t* vbase = reinterpret_cast<const uint32_t*>(Vc + static_cast<size_t>(kvh) * head_dim);  // uniform
    const size_t vrow = row / 2;  // in f16 pairs
    uint32_t vv[kAttnChunk];
    // in the kRope launch the new key's value comes from v_new and rows past the chunk's keys are
    // replaced by zeros below, so the loads stay below the new key's row where it is in this chunk
    const int vlast = j_new > 0 ? j_new - 1 : max(n - 1, 0);
#pragma unroll
    for (int j = 0; j < kAttnChunk; ++j) vv[j] = (vbase + static_cast<size_t>(s0 + min(j, vlast)) * vrow)[vl];
    __shared__ __align__(16) _Float16 rot[4][2][2 * kMaxPairs];  // [wave][q, k_new][dim]
    if constexpr (kRope) {
        // lane p rotates pair p (dims 2p, 2p + 1, or p, p + head_dim / 2) of the query and of the
        // new key, as rope_kernel does
        if (lane < pairs) {
            const float cs = dr.cs[lane], sn = dr.sn[lane];
            const int i0 = dr.neox ? lane : 2 * lane, i1 = dr.neox ? lane + pairs : 2 * lane + 1;
            const _Float16* qs = Q + (static_cast<size_t>(m) * heads + h) * head_dim;
            const _Float16* ks = dr.k_new + static_cast<size_t>(kvh) * head_dim;
            float a = static_cast<float>(qs[i0]), b = static_cast<float>(qs[i1]);
            rot[wl][0][i0] = static_cast<_Float16>(a * cs - b * sn);
            rot[wl][0][i1] = static_cast<_Float16>(a * sn + b * cs);
            a = static_cast<float>(ks[i0]);
            b = static_cast<float>(ks[i1]);
            const _Float16 k0 = static_cast<_Float16>(a * cs - b * sn), k1 = static_cast<_Float16>(a * sn + b * cs);
            rot[wl][1][i0] = k0;
            rot[wl][1][i1] = k1;
            if (j_new >= 0 && h % (heads / kv_heads) == 0) {  // one writer per KV head
                const size_t crow = static_cast<size_t>(pos) * row + static_cast<size_t>(kvh) * head_dim;
                dr.kc[crow + i0] = k0;
                dr.kc[crow + i1] = k1;
                const _Float16* vs = dr.v_new + static_cast<size_t>(kvh) * head_dim;
                dr.vc[crow + i0] = vs[i0];
                dr.vc[crow + i1] = vs[i1];
            }
        }
        // only this wave reads its LDS rows, and a wave's LDS operations complete in order
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        qp = reinterpret_cast<const uint32_t*>(rot[wl][0]);
    }
    if constexpr (kRope) {
        if (lane == j_new) {
            const u32x4* kn = reinterpret_cast<const u32x4*>(rot[wl][1]);
#pragma unroll
            for (int i = 0; i < kMaxPairs / 4; ++i)
                if (4 * i < pairs) kv[i] = kn[i];
        }
    }
    if constexpr (kRope) {
        const uint32_t vn = own ? reinterpret_cast<const uint32_t*>(dr.v_new + static_cast<size_t>(kvh) * head_dim)[lane] : 0u;
#pragma unroll
        for (int j = 0; j < kAttnChunk; ++j) vv[j] = j == j_new ? vn : (j < n ? vv[j] : 0u);
    }
    float dot = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxPairs / 4; ++i) {
        if (4 * i < pairs) {
            const uint32_t w[4] = {kv[i].x, kv[i].y, kv[i].z, kv[i].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) dot = dot2(qp[4 * i + e], w[e], dot);
        }
    }
    const float sc = lane < n ? dot * scale : -INFINITY;
    float mx = sc;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    const float e = n > 0 ? expf(sc - mx) : 0.0f;  // 0 on masked lanes
    const float sum = wave_sum(e);

    // output: lane l <-> dims 2l, 2l + 1
    float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
    for (int j = 0; j < kAttnChunk; ++j) {
        // lane j's weight, read into a scalar register (0 beyond the chunk's keys)
        const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j));
        h2v v;
        __builtin_memcpy(&v, &vv[j], 4);
        acc0 += pj * static_cast<float>(v[0]);
        acc1 += pj * static_cast<float>(v[1]);
    }
    if (chunks == 1) {
        if (own) {
            const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
            _Float16* op = out + (static_cast<size_t>(m) * heads + h) * head_dim + 2 * lane;
            op[0] = static_cast<_Float16>(acc0 * inv);
            op[1] = static_cast<_Float16>(acc1 * inv);
        }
        return;
    }
    float* pp = part + static_cast<size_t>(wave) * (head_dim + 2);
    if (lane == 0) {
        pp[0] = n > 0 ? mx : -INFINITY;
        pp[1] = sum;
    }
    if (own) {
        pp[2 + 2 * lane] = acc0;
        pp[3 + 2 * lane] = acc1;
    }
}

// Merges the chunks of each (m, h) in chunk order.  One thread per output element.
__global__ __launch_bounds__(256) void attention_combine_kernel(const float* __restrict__ part, _Float16* __restrict__ out,
                                                              int q_len, int heads, int head_dim, int chunks) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t total = static_cast<int64_t>(q_len) * heads * head_dim;
    if (idx >= total) return;
    const int d = static_cast<int>(idx % head_dim);
    const int64_t mh = idx / head_dim;
    const int h = static_cast<int>(mh % heads);
    const int m = static_cast<int>(mh / heads);
    const size_t stride = static_cast<size_t>(head_dim) + 2;
    auto at = [&](int c) { return part + ((static_cast<size_t>(m) * chunks + c) * heads + h) * stride; };
    // chunks are taken 8 at a time with all their loads issued first; the arithmetic runs in chunk
    // order
    constexpr int kG = 8;
    float mx = -INFINITY;
    for (int c0 = 0; c0 < chunks; c0 += kG) {
        float v[kG];
#pragma unroll
        for (int i = 0; i < kG; ++i) v[i] = c0 + i < chunks ? at(c0 + i)[0] : -INFINITY;
#pragma unroll
        for (int i = 0; i < kG; ++i) mx = fmaxf(mx, v[i]);
    }
    float sum = 0.0f, acc = 0.0f;
    for (int c0 = 0; c0 < chunks; c0 += kG) {
        float pm[kG], ps[kG], po[kG];
#pragma unroll
        for (int i = 0; i < kG; ++i) {
            const bool ok = c0 + i < chunks;
            const float* p = at(ok ? c0 + i : 0);
            pm[i] = p[0];
            ps[i] = ok ? p[1] : 0.0f;
            po[i] = p[2 + d];
        }
#pragma unroll
        for (int i = 0; i < kG; ++i) {
            if (ps[i] > 0.0f) {
                const float a = expf(pm[i] - mx);
                sum += ps[i] * a;
                acc += po[i] * a;
            }
        }
    }
    out[idx] = static_cast<_Float16>(sum > 0.0f ? acc / sum : 0.0f);
}

// ---- KV cache pool (one per device) ----------------------------------------------------------
struct KvPool {
    _Float16* k = nullptr;
    _Float16* v = nullptr;
    int layers = 0, max_seq = 0, kv_heads = 0, head_dim = 0;
    size_t cap = 0;
};
std::mutex g_kv_mutex;
std::unordered_map<int, KvPool> g_kv;

// ---- per-(device, stream) activation workspace of the layer pipeline --------------------------
struct LayerWs {
    void* buf = nullptr;
    size_t cap = 0;
};
std::mutex g_lws_mutex;
std::unordered_map<std::string, LayerWs> g_lws;

hipError_t layer_workspace(hipStream_t stream, size_t bytes, char** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const std::string key = std::to_string(dev) + ":" + std::to_string(reinterpret_cast<uintptr_t>(stream));
    std::lock_guard<std::mutex> lock(g_lws_mutex);
    LayerWs& ws = g_lws[key];
    if (ws.cap < bytes) {
        if (ws.buf) {
            if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
            if ((e = hipFree(ws.buf)) != hipSuccess) return e;
            ws.buf = nullptr;
            ws.cap = 0;
        }
        if ((e = hipMalloc(&ws.buf, bytes)) != hipSuccess) return e;
        ws.cap = bytes;
    }
    *out = static_cast<char*>(ws.buf);
    return hipSuccess;
}

// ---- prefill attention on the matrix cores --------------------------------------------------
// Flash-attention form for many query rows.  A workgroup of 4 waves owns 128 query rows: the
// 128 / G positions of a position tile times the G query heads of one KV head, which share every
// K and V row.  It walks the keys its rows can see in tiles of 64, staged through LDS
// (double-buffered, one barrier per tile):
//   * S = K Q^T on v_mfma_f32_32x32x16_f16.  A wave's 32 rows x 64 keys are two 32 x 32 tiles; K
//     fragments come from LDS, Q fragments stay in registers for the whole loop.  In an S tile a
//     lane holds one query row (lane mod 32) and 16 of the 32 keys, so the row's softmax
//     statistics need one exchange with the partner lane (lane ^ 32).
//   * fp32 online softmax in base 2 (scores multiplied by scale * log2 e).
//   * O^T += V^T P^T on the same instruction.  P goes from the S registers into the B fragment
//     without leaving the lane: the k order of each 16-key block is the order the lane holds its
//     keys in.  V is staged transposed ([dim][key]) so an A fragment is two 8-byte LDS reads.
// Rows are divided by their softmax sum and rounded to fp16 once.  Position tiles run longest
// first (causal rows near the end see the most keys); with 8 KV heads the workgroups of one KV
// head land on one XCD and share its L2.
constexpr int kFaRows = 128, kFaKeys = 64, kFaThreads = 256;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int D>
struct FaGeom {
    static constexpr int kRowK = D + 8;                      // f16 per staged K row (16-byte pad)
    static constexpr int kRowV = kFaKeys + 4;                // f16 per staged V^T row (8-byte pad)
    static constexpr int kK = kFaKeys * kRowK;               // f16 per K buffer
    static constexpr int kV = D * kRowV;                     // f16 per V^T buffer
    static constexpr int kBuf = kK + kV;
    static constexpr size_t kLdsBytes = 2 * static_cast<size_t>(kBuf) * sizeof(_Float16);
    static constexpr int kChunks = D / 8;                    // 16-byte chunks per row
    static constexpr int kKUnits = kFaKeys * kChunks / kFaThreads;        // K chunks per thread
    static constexpr int kVUnits = (kFaKeys / 2) * kChunks / kFaThreads;  // V (key pair, chunk) per thread
    static_assert(kKUnits >= 1 && kVUnits >= 1, "head_dim 64 or 128");
};

extern __shared__ __align__(16) _Float16 fa_lds[];

template <int D>
__global__ __launch_bounds__(kFaThreads, 2) void attention_mfma_kernel(
    const _Float16* __restrict__ Q, const _Float16* __restrict__ Kc, const _Float16* __restrict__ Vc,
    _Float16* __restrict__ out, int q_len, int kv_len, int heads, int kv_heads, int start_pos, float scale_log2,
    int causal, int ptiles) {
    using FG = FaGeom<D>;
    const int group = heads / kv_heads;
    const int ppw = kFaRows / group;  // positions per workgroup
    const int g = static_cast<int>(blockIdx.x % kv_heads);
    const int pt = ptiles - 1 - static_cast<int>(blockIdx.x / kv_heads);
    const int p0 = pt * ppw;
    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
    const int r = 32 * (tid >> 6) + l32;  // row of the workgroup
    const int pos = p0 + r / group;
    const int head = g * group + r % group;
    const int p_last = min(p0 + ppw, q_len) - 1;
    const int n_keys = causal ? min(kv_len, start_pos + p_last + 1) : kv_len;
    const int n_tiles = (n_keys + kFaKeys - 1) / kFaKeys;
    const int vis_all = causal ? min(kv_len, start_pos + p0 + 1) : kv_len;    // keys every row sees
    const int row_end = causal ? min(kv_len, start_pos + pos + 1) : kv_len;   // keys this row sees
    const size_t kv_row = static_cast<size_t>(kv_heads) * D;
    const _Float16* kbase = Kc + static_cast<size_t>(g) * D;
    const _Float16* vbase = Vc + static_cast<size_t>(g) * D;

    // Q fragments of row (pos, head): dims 16 db + 8 h .. + 7 (rows past q_len read the last row)
    f16x8 qf[D / 16];
    {
        const _Float16* qrow = Q + (static_cast<size_t>(min(pos, q_len - 1)) * heads + head) * D + 8 * h;
#pragma unroll
        for (int db = 0; db < D / 16; ++db) __builtin_memcpy(&qf[db], qrow + 16 * db, 16);
    }

    // Staging of key tile t: thread units of K (key, chunk) and of V (key pair, chunk); keys past
    // kv_len read the last key (finite values, masked out of the softmax).
    u32x4 kr[FG::kKUnits], vr[FG::kVUnits][2];
    auto load = [&](int t) {
        const int kb = t * kFaKeys;
#pragma unroll
        for (int i = 0; i < FG::kKUnits; ++i) {
            const int u = tid + kFaThreads * i, key = u / FG::kChunks, c = u % FG::kChunks;
            const int k = min(kb + key, kv_len - 1);
            kr[i] = *reinterpret_cast<const u32x4*>(kbase + static_cast<size_t>(k) * kv_row + 8 * c);
        }
#pragma unroll
        for (int i = 0; i < FG::kVUnits; ++i) {
            const int u = tid + kFaThreads * i, kp = u % (kFaKeys / 2), c = u / (kFaKeys / 2);
            const int k0 = min(kb + 2 * kp, kv_len - 1), k1 = min(kb + 2 * kp + 1, kv_len - 1);
            vr[i][0] = *reinterpret_cast<const u32x4*>(vbase + static_cast<size_t>(k0) * kv_row + 8 * c);
            vr[i][1] = *reinterpret_cast<const u32x4*>(vbase + static_cast<size_t>(k1) * kv_row + 8 * c);
        }
    };
    auto store = [&](int buf) {
        _Float16* sk = fa_lds + buf * FG::kBuf;
        _Float16* sv = sk + FG::kK;
#pragma unroll
        for (int i = 0; i < FG::kKUnits; ++i) {
            const int u = tid + kFaThreads * i, key = u / FG::kChunks, c = u % FG::kChunks;
            *reinterpret_cast<u32x4*>(sk + key * FG::kRowK + 8 * c) = kr[i];
        }
#pragma unroll
        for (int i = 0; i < FG::kVUnits; ++i) {
            const int u = tid + kFaThreads * i, kp = u % (kFaKeys / 2), c = u / (kFaKeys / 2);
            // V^T[8c + e][2kp, 2kp + 1] = (V[k0][8c + e], V[k1][8c + e]); dword m of a row chunk
            // holds dims 2m, 2m + 1
            uint32_t* col = reinterpret_cast<uint32_t*>(sv + 8 * c * FG::kRowV + 2 * kp);
            const u32x4 a = vr[i][0], b = vr[i][1];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                col[(2 * m) * (FG::kRowV / 2)] = __builtin_amdgcn_perm(b[m], a[m], 0x05040100u);
                col[(2 * m + 1) * (FG::kRowV / 2)] = __builtin_amdgcn_perm(b[m], a[m], 0x07060302u);
            }
        }
    };

    f32x16 o[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[dt][v] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    load(0);
    store(0);
    __syncthreads();
    for (int t = 0; t < n_tiles; ++t) {
        if (t + 1 < n_tiles) load(t + 1);
        const _Float16* sk = fa_lds + (t & 1) * FG::kBuf;
        const _Float16* sv = sk + FG::kK;
        // S^T tiles: register v of tile tt is key 32 tt + 8 (v / 4) + 4 h + v % 4 of the row l32
        f32x16 s[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
            for (int v = 0; v < 16; ++v) s[tt][v] = 0.0f;
#pragma unroll
            for (int db = 0; db < D / 16; ++db) {
                f16x8 kf;
                __builtin_memcpy(&kf, sk + (32 * tt + l32) * FG::kRowK + 16 * db + 8 * h, 16);
                s[tt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[db], s[tt], 0, 0, 0);
            }
        }
        const int kb = t * kFaKeys;
        const bool full = kb + kFaKeys <= vis_all;
        float mx = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                float x = s[tt][v] * scale_log2;
                if (!full && kb + 32 * tt + 8 * (v >> 2) + 4 * h + (v & 3) >= row_end) x = -INFINITY;
                s[tt][v] = x;
                mx = fmaxf(mx, x);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run, mx);  // finite: key 0 is visible to every row
        const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
        float sum = 0.0f;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float p = __builtin_amdgcn_exp2f(s[tt][v] - m_new);
                s[tt][v] = p;
                sum += p;
            }
        sum += __shfl_xor(sum, 32, 64);
        l_run = l_run * corr + sum;
        m_run = m_new;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[dt][v] *= corr;
        // 16-key block b: lane half h holds keys 16 b + 4 h + (0..3) and 16 b + 8 + 4 h + (0..3)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            f16x8 pf;
#pragma unroll
            for (int e = 0; e < 8; ++e) pf[e] = static_cast<_Float16>(s[b >> 1][8 * (b & 1) + e]);
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt) {
                const _Float16* vrow = sv + (32 * dt + l32) * FG::kRowV + 16 * b + 4 * h;
                f16x8 vf;
                __builtin_memcpy(&vf, vrow, 8);
                __builtin_memcpy(reinterpret_cast<char*>(&vf) + 8, vrow + 8, 8);
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf, o[dt], 0, 0, 0);
            }
        }
        if (t + 1 < n_tiles) store((t + 1) & 1);
        __syncthreads();
    }

    if (pos < q_len) {
        const float inv = 1.0f / l_run;
        _Float16* orow = out + (static_cast<size_t>(pos) * heads + head) * D;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                _Float16 v4[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) v4[i] = static_cast<_Float16>(o[dt][4 * q4 + i] * inv);
                __builtin_memcpy(orow + 32 * dt + 8 * q4 + 4 * h, v4, 8);
            }
    }
}

int attn_chunks(int kv_len) { return kv_len <= 0 ? 1 : (kv_len + kAttnChunk - 1) / kAttnChunk; }

size_t attn_part_bytes(int q_len, int heads, int head_dim, int kv_len) {
    const int ch = attn_chunks(kv_len);
    return ch > 1 ? static_cast<size_t>(q_len) * heads * ch * (head_dim + 2) * sizeof(float) : 0;
}

}  // namespace

// ---- launchers (validated arguments) --------------------------------------------------------
hipError_t launch_rmsnorm(const void* x, const void* res, const void* w, int w_f32, void* h_out, void* out, int M, int K,
                          float eps, hipStream_t stream) {
    if (M <= 0 || K <= 0) return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(M), dim3(kNormThreads), 0, stream, static_cast<const _Float16*>(x),
                       static_cast<const _Float16*>(res), w, w_f32, static_cast<_Float16*>(h_out),
                       static_cast<_Float16*>(out), K, eps);
    return hipGetLastError();
}

hipError_t launch_residual_add(const void* x, const void* r, void* out, int64_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int64_t items = (n & 7) == 0 ? n / 8 : n;
    hipLaunchKernelGGL(residual_add_kernel, dim3(static_cast<unsigned>((items + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const _Float16*>(x), static_cast<const _Float16*>(r), static_cast<_Float16*>(out), n);
    return hipGetLastError();
}

hipError_t launch_bias_add(void* y, const void* b, int rows, int n, hipStream_t stream) {
    const int64_t total = static_cast<int64_t>(rows) * n;
    const int blocks = static_cast<int>(std::min<int64_t>((total + 255) / 256, 4096));
    hipLaunchKernelGGL(bias_add_kernel, dim3(blocks), dim3(256), 0, stream, static_cast<_Float16*>(y),
                       static_cast<const _Float16*>(b), n, total);
    return hipGetLastError();
}

hipError_t launch_swiglu(const void* g, const void* u, void* out, int64_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int64_t items = (n & 7) == 0 ? n / 8 : n;
    hipLaunchKernelGGL(swiglu_kernel, dim3(static_cast<unsigned>((items + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const _Float16*>(g), static_cast<const _Float16*>(u), static_cast<_Float16*>(out), n);
    return hipGetLastError();
}

hipError_t launch_rope(const void* q, void* q_out, int n_q, const void* k, void* k_out, const void* v, void* v_out, int n_k,
                       int seq_len, int head_dim, int pos_offset, float freq_base, bool neox, hipStream_t stream) {
    if (seq_len <= 0 || n_q + n_k <= 0) return hipSuccess;
    RopeFreq fr;
    for (int i = 0; i < head_dim / 2; ++i)
        fr.inv[i] = 1.0f / std::pow(freq_base, static_cast<float>(2 * i) / static_cast<float>(head_dim));
    const int64_t total = static_cast<int64_t>(seq_len) * (n_q + n_k) * (head_dim / 2);
    hipLaunchKernelGGL(rope_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const _Float16*>(q), static_cast<_Float16*>(q_out), n_q, static_cast<const _Float16*>(k),
                       static_cast<_Float16*>(k_out), static_cast<const _Float16*>(v), static_cast<_Float16*>(v_out), n_k,
                       seq_len, head_dim, pos_offset, neox ? 1 : 0, fr);
    return hipGetLastError();
}

size_t attention_workspace_bytes(int q_len, int heads, int head_dim, int kv_len) {
    return attn_part_bytes(q_len, heads, head_dim, kv_len);
}

namespace {

// The matrix-core kernel serves head_dim 64 and 128, query groups dividing 128, at least
// kFaMinRows query positions (fewer rows leave the 32-row MFMA tiles mostly empty) and 16-byte
// aligned Q / K / V.
constexpr int kFaMinRows = 16;

template <int D>
hipError_t launch_attention_mfma(const void* Q, const void* K, const void* V, void* out, int q_len, int kv_len, int heads,
                                 int kv_heads, int start_pos, float scale, bool causal, hipStream_t stream) {
    using FG = FaGeom<D>;
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_mfma_kernel<D>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(FG::kLdsBytes));
    });
    if (attr != hipSuccess) return attr;
    const int ppw = kFaRows / (heads / kv_heads);
    const int ptiles = (q_len + ppw - 1) / ppw;
    const float scale_log2 = scale * 1.4426950408889634f;
    hipLaunchKernelGGL((attention_mfma_kernel<D>), dim3(static_cast<unsigned>(ptiles * kv_heads)), dim3(kFaThreads),
                       FG::kLdsBytes, stream, static_cast<const _Float16*>(Q), static_cast<const _Float16*>(K),
                       static_cast<const _Float16*>(V), static_cast<_Float16*>(out), q_len, kv_len, heads, kv_heads,
                       start_pos, scale_log2, causal ? 1 : 0, ptiles);
    return hipGetLastError();
}

bool attention_mfma_ok(const void* Q, const void* K, const void* V, int q_len, int kv_len, int heads, int kv_heads,
                       int head_dim) {
    const bool aligned = (reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(K) | reinterpret_cast<uintptr_t>(V)) % 16 == 0;
    const int group = heads / kv_heads;
    return (head_dim == 64 || head_dim == 128) && kFaRows % group == 0 && q_len >= kFaMinRows && kv_len > 0 && aligned;
}

}  // namespace

hipError_t launch_attention(const void* Q, const void* K, const void* V, void* out, void* part, int q_len, int kv_len,
                            int heads, int kv_heads, int head_dim, int start_pos, float scale, bool causal,
                            hipStream_t stream) {
    if (q_len <= 0 || heads <= 0) return hipSuccess;
    if (attention_mfma_ok(Q, K, V, q_len, kv_len, heads, kv_heads, head_dim)) {
        if (head_dim == 128)
            return launch_attention_mfma<128>(Q, K, V, out, q_len, kv_len, heads, kv_heads, start_pos, scale, causal, stream);
        return launch_attention_mfma<64>(Q, K, V, out, q_len, kv_len, heads, kv_heads, start_pos, scale, causal, stream);
    }
    const int chunks = attn_chunks(kv_len);
    const int64_t waves = static_cast<int64_t>(q_len) * heads * chunks;
    const dim3 grid(static_cast<unsigned>((waves + 3) / 4));
    auto go = [&](auto dc) {
        constexpr int D = decltype(dc)::value;
        hipLaunchKernelGGL((attention_kernel<D>), grid, dim3(256), 0, stream, static_cast<const _Float16*>(Q),
                           static_cast<const _Float16*>(K), static_cast<const _Float16*>(V), static_cast<_Float16*>(out),
                           static_cast<float*>(part), q_len, kv_len, heads, kv_heads, head_dim, start_pos, scale,
                           causal ? 1 : 0, chunks);
    };
    const bool aligned = (reinterpret_cast<uintptr_t>(Q) | reinterpret_cast<uintptr_t>(K) | reinterpret_cast<uintptr_t>(V)) % 16 == 0;
    if (head_dim % 8 == 0 && head_dim <= 128 && aligned)
        hipLaunchKernelGGL((attention_keys_kernel<false>), grid, dim3(256), 0, stream, static_cast<const _Float16*>(Q),
                           static_cast<const _Float16*>(K), static_cast<const _Float16*>(V), static_cast<_Float16*>(out),
                           static_cast<float*>(part), q_len, kv_len, heads, kv_heads, head_dim, start_pos, scale,
                           causal ? 1 : 0, chunks, DecodeRope{});
    else if (head_dim <= 64) go(std::integral_constant<int, 1>{});
    else if (head_dim <= 128) go(std::integral_constant<int, 2>{});
    else go(std::integral_constant<int, 4>{});
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || chunks == 1) return e;
    const int64_t n = static_cast<int64_t>(q_len) * heads * head_dim;
    hipLaunchKernelGGL(attention_combine_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const float*>(part), static_cast<_Float16*>(out), q_len, heads, head_dim, chunks);
    return hipGetLastError();
}

hipError_t launch_attention_decode_rope(const void* q, const void* k_new, const void* v_new, void* kc, void* vc, void* out,
                                        void* part, int kv_len, int heads, int kv_heads, int head_dim, float scale,
                                        float freq_base, bool neox, hipStream_t stream) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_new) |
                         reinterpret_cast<uintptr_t>(v_new) | reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc);
    if (kv_len <= 0 || heads <= 0 || head_dim % 8 != 0 || head_dim > 128 || (al & 15u) != 0) return hipErrorNotSupported;
    DecodeRope dr{};
    dr.k_new = static_cast<const _Float16*>(k_new);
    dr.v_new = static_cast<const _Float16*>(v_new);
    dr.kc = static_cast<_Float16*>(kc);
    dr.vc = static_cast<_Float16*>(vc);
    dr.neox = neox ? 1 : 0;
    // the angle as the RoPE kernel forms it (fp32 position x fp32 inverse frequency); its cosine
    // and sine evaluated here once for the step
    for (int i = 0; i < head_dim / 2; ++i) {
        const float inv = 1.0f / std::pow(freq_base, static_cast<float>(2 * i) / static_cast<float>(head_dim));
        const float ang = static_cast<float>(kv_len - 1) * inv;
        dr.cs[i] = static_cast<float>(std::cos(static_cast<double>(ang)));
        dr.sn[i] = static_cast<float>(std::sin(static_cast<double>(ang)));
    }
    const int chunks = attn_chunks(kv_len);
    const int64_t waves = static_cast<int64_t>(heads) * chunks;
    hipLaunchKernelGGL((attention_keys_kernel<true>), dim3(static_cast<unsigned>((waves + 3) / 4)), dim3(256), 0, stream,
                       static_cast<const _Float16*>(q), static_cast<const _Float16*>(kc), static_cast<const _Float16*>(vc),
                       static_cast<_Float16*>(out), static_cast<float*>(part), 1, kv_len, heads, kv_heads, head_dim,
                       kv_len - 1, scale, 1, chunks, dr);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || chunks == 1) return e;
    const int64_t n = static_cast<int64_t>(heads) * head_dim;
    hipLaunchKernelGGL(attention_combine_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const float*>(part), static_cast<_Float16*>(out), 1, heads, head_dim, chunks);
    return hipGetLastError();
}

// ---- KV cache pool ----------------------------------------------------------------------------
LayerStatus kv_cache_init(int layers, int max_seq, int kv_heads, int head_dim) {
    if (layers <= 0 || max_seq <= 0 || kv_heads <= 0 || head_dim <= 0)
        return {QMM_ERR_INVALID_ARGUMENT, "KV cache dimensions must all be positive."};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return {QMM_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(e)};
    std::lock_guard<std::mutex> lock(g_kv_mutex);
    KvPool& p = g_kv[dev];
    const size_t need = static_cast<size_t>(layers) * max_seq * kv_heads * head_dim * sizeof(_Float16);
    if (need > p.cap) {
        if (p.k) (void)hipFree(p.k);
        if (p.v) (void)hipFree(p.v);
        p = KvPool{};
        if ((e = hipMalloc(reinterpret_cast<void**>(&p.k), need)) != hipSuccess) {
            p.k = nullptr;
            return {QMM_ERR_HIP, std::string("hipMalloc (KV cache): ") + hipGetErrorString(e)};
        }
        if ((e = hipMalloc(reinterpret_cast<void**>(&p.v), need)) != hipSuccess) {
            (void)hipFree(p.k);
            p = KvPool{};
            return {QMM_ERR_HIP, std::string("hipMalloc (KV cache): ") + hipGetErrorString(e)};
        }
        p.cap = need;
    }
    p.layers = layers;
    p.max_seq = max_seq;
    p.kv_heads = kv_heads;
    p.head_dim = head_dim;
    return {QMM_OK, ""};
}

LayerStatus kv_cache_free() {
    std::lock_guard<std::mutex> lock(g_kv_mutex);
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return {QMM_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(e)};
    for (auto& kv : g_kv) {
        if (!kv.second.k) continue;
        if ((e = hipSetDevice(kv.first)) != hipSuccess) return {QMM_ERR_HIP, hipGetErrorString(e)};
        (void)hipDeviceSynchronize();  // queued kernels may still use the pool
        (void)hipFree(kv.second.k);
        (void)hipFree(kv.second.v);
    }
    g_kv.clear();
    (void)hipSetDevice(cur);
    return {QMM_OK, ""};
}

// Device K / V of layer `layer` for a call writing [start, start + q_len), checked against the
// pool's geometry (the reference's DeviceKVCachePool checks, attention.hip:316-331).
LayerStatus kv_cache_layer(int layer, int start, int q_len, int kv_heads, int head_dim, _Float16** k, _Float16** v,
                           int* max_seq) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return {QMM_ERR_HIP, std::string("hipGetDevice: ") + hipGetErrorString(e)};
    std::lock_guard<std::mutex> lock(g_kv_mutex);
    auto it = g_kv.find(dev);
    if (it == g_kv.end() || !it->second.k)
        return {QMM_ERR_UNSUPPORTED, "Device KV cache not initialized. Call kv_cache_init first."};
    const KvPool& p = it->second;
    if (layer < 0 || layer >= p.layers) return {QMM_ERR_OUT_OF_RANGE, "layer_idx out of range for DeviceKVCachePool."};
    if (start < 0 || static_cast<int64_t>(start) + q_len > p.max_seq)
        return {QMM_ERR_OUT_OF_RANGE, "start_pos + q_len exceeds max_seq_len in DeviceKVCachePool."};
    if (kv_heads != p.kv_heads || head_dim != p.head_dim)
        return {QMM_ERR_INVALID_ARGUMENT, "num_kv_heads or head_dim mismatch with DeviceKVCachePool."};
    const size_t layer_elems = static_cast<size_t>(p.max_seq) * p.kv_heads * p.head_dim;
    *k = p.k + static_cast<size_t>(layer) * layer_elems;
    *v = p.v + static_cast<size_t>(layer) * layer_elems;
    if (max_seq) *max_seq = p.max_seq;
    return {QMM_OK, ""};
}

// ---- the layer pipeline --------------------------------------------------------------------
LayerStatus forward_layer(const qmm_layer_config& cfg, const qmm_layer_weights& w, const void* x_in, void* x_out,
                          int layer_idx, int seq_len, int pos_offset, hipStream_t stream) {
    const int H = cfg.num_heads, KVH = cfg.num_kv_heads, D = cfg.head_dim;
    const int hid = cfg.hidden_size, inter = cfg.intermediate_size;
    if (seq_len <= 0 || hid <= 0 || inter <= 0 || H <= 0 || KVH <= 0 || D <= 0)
        return {QMM_ERR_INVALID_ARGUMENT, "seq_len and the layer dimensions must be positive."};
    if (H % KVH != 0) return {QMM_ERR_INVALID_ARGUMENT, "num_heads must be divisible by num_kv_heads."};
    if (D > kMaxHeadDim || D % 2 != 0) return {QMM_ERR_INVALID_ARGUMENT, "head_dim must be even and in (0, 256]."};
    if (x_in == nullptr || x_out == nullptr) return {QMM_ERR_INVALID_ARGUMENT, "x_in and x_out must be non-null."};
    const int qd = H * D, kvd = KVH * D;
    _Float16 *kc = nullptr, *vc = nullptr;
    LayerStatus st = kv_cache_layer(layer_idx, pos_offset, seq_len, KVH, D, &kc, &vc, nullptr);
    if (st.code != QMM_OK) return st;
    const int kv_len = pos_offset + seq_len;

    // activation workspace
    const size_t S = static_cast<size_t>(seq_len);
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off += (bytes + 255) & ~size_t{255};
        return at;
    };
    const size_t o_norm = take(S * hid * 2), o_q = take(S * qd * 2), o_k = take(S * kvd * 2), o_v = take(S * kvd * 2);
    const size_t o_qr = take(S * qd * 2), o_att = take(S * qd * 2), o_proj = take(S * hid * 2), o_h = take(S * hid * 2);
    const size_t o_g = take(S * inter * 2), o_u = take(S * inter * 2), o_act = take(S * inter * 2);
    const size_t o_down = take(S * hid * 2), o_part = take(attn_part_bytes(seq_len, H, D, kv_len));
    char* ws = nullptr;
    hipError_t e = layer_workspace(stream, off, &ws);
    if (e != hipSuccess) return {QMM_ERR_HIP, std::string("layer workspace: ") + hipGetErrorString(e)};
    auto fail = [](hipError_t err, const char* what) {
        return LayerStatus{QMM_ERR_HIP, std::string(what) + ": " + hipGetErrorString(err)};
    };
    auto gemms = [&](const qmm_gemm_desc* d, int n) -> LayerStatus {
        const int rc = qmm_gemm_batch(d, n, stream);
        if (rc != QMM_OK) return {rc, qmm_last_error()};
        return {QMM_OK, ""};
    };
    auto desc = [&](int t, const void* A, const void* W, void* C, int M, int N, int K) {
        qmm_gemm_desc d{};
        d.ggml_type = t;
        d.A = A;
        d.a_dtype = QMM_DTYPE_F16;
        d.W = W;
        d.C = C;
        d.c_dtype = QMM_DTYPE_F16;
        d.M = M;
        d.N = N;
        d.K = K;
        return d;
    };
    const int nw_f32 = w.attn_norm_dtype == QMM_DTYPE_F32 ? 1 : 0, fw_f32 = w.ffn_norm_dtype == QMM_DTYPE_F32 ? 1 : 0;
    // Decode (one row): the norms, SwiGLU and the last residual add are folded into the GEMV
    // launches (their activation staging and output epilogue); a step whose shapes the folded
    // kernels do not take runs the separate kernels instead.
    const bool fold = seq_len == 1;
    // Runs descriptors of `d` with fold `fz` on their common activations, consecutive descriptors
    // of one weight type as one launch, until one is not supported folded; `done` = how many ran.
    auto folded = [&](const qmm_gemm_desc* d, int n, const GemvFuse& fz, int& done) -> LayerStatus {
        done = 0;
        if (!fold) return {QMM_OK, ""};
        for (int i = 0; i < n;) {
            int j = i + 1;
            while (j < n && d[j].ggml_type == d[i].ggml_type) ++j;
            const void* W[3];
            void* C[3];
            int N[3];
            for (int t = i; t < j; ++t) {
                W[t - i] = d[t].W;
                C[t - i] = d[t].C;
                N[t - i] = d[t].N;
            }
            const hipError_t fe = launch_gemv_ex(d[i].ggml_type, d[i].A, QMM_DTYPE_F16, 1, d[i].K, W, C, N, j - i, fz, stream);
            if (fe == hipErrorNotSupported) return {QMM_OK, ""};  // the caller runs the rest unfolded
            if (fe != hipSuccess) return {QMM_ERR_HIP, std::string("folded GEMV: ") + hipGetErrorString(fe)};
            i = j;
            done = j;
        }
        return {QMM_OK, ""};
    };
    int done = 0;

    // 1.-2. pre-attention RMSNorm, q, k, v (one launch per weight type)
    const qmm_gemm_desc qkv[3] = {desc(w.wq_type, ws + o_norm, w.wq, ws + o_q, seq_len, qd, hid),
                                  desc(w.wk_type, ws + o_norm, w.wk, ws + o_k, seq_len, kvd, hid),
                                  desc(w.wv_type, ws + o_norm, w.wv, ws + o_v, seq_len, kvd, hid)};
    {
        GemvFuse fz;
        fz.kind = 1;
        fz.w = w.attn_norm;
        fz.w_f32 = nw_f32;
        fz.eps = cfg.rms_norm_eps;
        qmm_gemm_desc dq[3] = {qkv[0], qkv[1], qkv[2]};
        for (auto& d : dq) d.A = x_in;
        if ((st = folded(dq, 3, fz, done)).code != QMM_OK) return st;
    }
    if (done < 3) {
        if ((e = launch_rmsnorm(x_in, nullptr, w.attn_norm, nw_f32, nullptr, ws + o_norm, seq_len, hid, cfg.rms_norm_eps,
                                stream)) != hipSuccess)
            return fail(e, "rmsnorm");
        if ((st = gemms(qkv + done, 3 - done)).code != QMM_OK) return st;
    }
    // optional q / k / v biases, added to the projections before the rotation
    {
        const void* const bias[3] = {w.bq, w.bk, w.bv};
        const size_t at[3] = {o_q, o_k, o_v};
        const int bn[3] = {qd, kvd, kvd};
        for (int i = 0; i < 3; ++i)
            if (bias[i] != nullptr && (e = launch_bias_add(ws + at[i], bias[i], seq_len, bn[i], stream)) != hipSuccess)
                return fail(e, "q/k/v bias");
    }
    // 3.-4. RoPE on q and k (k and v land in the cache at their positions), attention over the
    // cache; in decode the rotation and the cache write run inside the attention kernel
    const float scale = cfg.scale != 0.0f ? cfg.scale : 1.0f / std::sqrt(static_cast<float>(D));
    e = fold ? launch_attention_decode_rope(ws + o_q, ws + o_k, ws + o_v, kc, vc, ws + o_att, ws + o_part, kv_len, H, KVH, D,
                                            scale, cfg.rope_freq_base, cfg.rope_neox != 0, stream)
             : hipErrorNotSupported;
    if (e == hipErrorNotSupported) {
        const size_t cache_off = static_cast<size_t>(pos_offset) * kvd;
        if ((e = launch_rope(ws + o_q, ws + o_qr, H, ws + o_k, kc + cache_off, ws + o_v, vc + cache_off, KVH, seq_len, D,
                             pos_offset, cfg.rope_freq_base, cfg.rope_neox != 0, stream)) != hipSuccess)
            return fail(e, "rope");
        e = launch_attention(ws + o_qr, kc, vc, ws + o_att, ws + o_part, seq_len, kv_len, H, KVH, D, pos_offset, scale, true,
                             stream);
    }
    if (e != hipSuccess) return fail(e, "attention");
    // 5. output projection
    const qmm_gemm_desc o = desc(w.wo_type, ws + o_att, w.wo, ws + o_proj, seq_len, hid, qd);
    if ((st = gemms(&o, 1)).code != QMM_OK) return st;
    if (w.bo != nullptr && (e = launch_bias_add(ws + o_proj, w.bo, seq_len, hid, stream)) != hipSuccess)
        return fail(e, "output bias");
    // 6.-7. residual + pre-FFN RMSNorm, gate, up (one launch per weight type)
    const qmm_gemm_desc gu[2] = {desc(w.wgate_type, ws + o_norm, w.wgate, ws + o_g, seq_len, inter, hid),
                                 desc(w.wup_type, ws + o_norm, w.wup, ws + o_u, seq_len, inter, hid)};
    bool h_ready = false;    // h = half(x_in + o) materialised at ws + o_h
    bool act_ready = false;  // SwiGLU's output already at ws + o_act
    {
        GemvFuse fz;
        fz.kind = 2;
        fz.R = ws + o_proj;
        fz.w = w.ffn_norm;
        fz.w_f32 = fw_f32;
        fz.eps = cfg.rms_norm_eps;
        qmm_gemm_desc dg[2] = {gu[0], gu[1]};
        for (auto& d : dg) d.A = x_in;
        if (w.wgate_type == w.wup_type) {
            // gate row n and up row n in one wave: the launch writes SwiGLU's output directly
            qmm_gemm_desc dp[2] = {dg[0], dg[1]};
            dp[0].C = ws + o_act;
            fz.pair = 1;
            if ((st = folded(dp, 2, fz, done)).code != QMM_OK) return st;
            act_ready = done == 2;
            fz.pair = 0;
        }
        if (!act_ready && (st = folded(dg, 2, fz, done)).code != QMM_OK) return st;
    }
    if (!act_ready && done < 2) {
        if ((e = launch_rmsnorm(x_in, ws + o_proj, w.ffn_norm, fw_f32, ws + o_h, ws + o_norm, seq_len, hid,
                                cfg.rms_norm_eps, stream)) != hipSuccess)
            return fail(e, "rmsnorm_residual");
        h_ready = true;
        if ((st = gemms(gu + done, 2 - done)).code != QMM_OK) return st;
    }
    // 8.-9. SwiGLU (unless the gate/up launch produced it), down and the second residual (folded
    // into down's output).  SwiGLU is not folded into down's staging: every down workgroup would
    // read both intermediate vectors and evaluate every exp (measured slower than a kernel).
    if (!act_ready &&
        (e = launch_swiglu(ws + o_g, ws + o_u, ws + o_act, static_cast<int64_t>(S) * inter, stream)) != hipSuccess)
        return fail(e, "swiglu");
    {
        GemvFuse fz;
        fz.ea = x_in;
        fz.eb = ws + o_proj;
        const qmm_gemm_desc dd = desc(w.wdown_type, ws + o_act, w.wdown, x_out, seq_len, hid, inter);
        if ((st = folded(&dd, 1, fz, done)).code != QMM_OK) return st;
    }
    if (done < 1) {
        const qmm_gemm_desc dn = desc(w.wdown_type, ws + o_act, w.wdown, ws + o_down, seq_len, hid, inter);
        if ((st = gemms(&dn, 1)).code != QMM_OK) return st;
        if (!h_ready &&
            (e = launch_residual_add(x_in, ws + o_proj, ws + o_h, static_cast<int64_t>(S) * hid, stream)) != hipSuccess)
            return fail(e, "residual_add");
        if ((e = launch_residual_add(ws + o_h, ws + o_down, x_out, static_cast<int64_t>(S) * hid, stream)) != hipSuccess)
            return fail(e, "residual_add");
    }
    return {QMM_OK, ""};
}

// A second per-(device, stream) buffer for the standalone attention entry points (their
// partial results), so they never resize the pipeline's activation workspace.
namespace {
std::unordered_map<std::string, LayerWs> g_scratch;
}

hipError_t layer_scratch(hipStream_t stream, size_t bytes, void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const std::string key = std::to_string(dev) + ":" + std::to_string(reinterpret_cast<uintptr_t>(stream));
    std::lock_guard<std::mutex> lock(g_lws_mutex);
    LayerWs& ws = g_scratch[key];
    if (ws.cap < bytes) {
        if (ws.buf) {
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

hipError_t release_layer_workspaces() {
    std::lock_guard<std::mutex> lock(g_lws_mutex);
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    // An entry is erased as soon as its buffer is freed, so an error part-way leaves no freed
    // pointer behind for the next layer_workspace() / layer_scratch() call to hand out.
    for (auto* m : {&g_lws, &g_scratch}) {
        for (auto it = m->begin(); it != m->end();) {
            if (it->second.buf) {
                const int dev = std::stoi(it->first.substr(0, it->first.find(':')));
                if ((e = hipSetDevice(dev)) != hipSuccess) return e;
                if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
                if ((e = hipFree(it->second.buf)) != hipSuccess) {
                    it = m->erase(it);  // the runtime owns the pointer now, whatever it reported
                    (void)hipSetDevice(cur);  // the free's error is the one reported
                    return e;
                }
            }
            it = m->erase(it);
        }
    }
    return hipSetDevice(cur);
}

}  // namespace qmm
