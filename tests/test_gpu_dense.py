"""GPU parity of the dense fp16 weight path (GGML F16, the reference's matmul_nt operand) and of
the drop-in ``matmul_module`` entry points for the dense matmuls and the layer operations.

Bars (written into each check):
* F16 GEMM through the C ABI: the operands are exact fp16 values, so against the fp64 product of
  the same values max_i|y - y64| / max_i|y64| <= 1e-5 with fp32 output (fp32 accumulation only);
* GEMV sizes give row results bit-identical for every M < qmm_gemv_max_m, fused launches bit-identical to
  single ones;
* matmul_module functions: the reference tests' own bars (tests/test_layer.py) against the CPU
  restatement in oracle/layer_oracle.py: 2e-3 absolute per kernel, 5e-3 for a whole layer;
  matmul / matmul_nt within 1e-3 relative of fp64 (fp16 output rounding).
"""

import math

import numpy as np
import pytest

import gguf_oracle as O
import layer_oracle as L

pytestmark = pytest.mark.gpu

F16 = 1
QUANT = {O.GGML_Q4_0: O.quantize_q4_0, O.GGML_Q8_0: O.quantize_q8_0, O.GGML_Q4_K: O.quantize_q4_k,
         O.GGML_Q6_K: O.quantize_q6_k}


@pytest.fixture(scope="module")
def dev(cuda):
    import qmm  # noqa: F401  (fails loudly if the library is not built)
    return cuda


def t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(np.max(np.abs(want)), 1e-30))


def maxerr(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float32) - np.asarray(b, np.float32))))


def dense_case(seed, M, N, K):
    r = np.random.default_rng(seed)
    A = r.standard_normal((M, K)).astype(np.float16)
    W = (r.standard_normal((N, K)) / math.sqrt(K)).astype(np.float16)
    return A, W


def gemm_f16(A, W, dev, out_dtype="f32"):
    import torch
    import qmm
    C = qmm.gemm(F16, t(A, dev), t(W, dev), W.shape[0], W.shape[1],
                 out_dtype=torch.float32 if out_dtype == "f32" else torch.float16)
    torch.cuda.synchronize()
    return C.float().cpu().numpy()


# GEMV fast path (K % 16 == 0), GEMV fallback (K % 16 != 0), prefill (M >= 17, K % 8 == 0; the
# 32-row tile up to M = 32),
# prefill-unsupported K (K % 8 != 0: the fallback GEMV serves every M).
@pytest.mark.parametrize("M,N,K", [(1, 300, 4096), (3, 129, 8192 + 64), (31, 64, 640), (1, 40, 200), (5, 17, 1001),
                                   (32, 300, 512), (100, 513, 1000), (64, 256, 4104), (40, 33, 99)])
def test_f16_gemm_vs_fp64(dev, M, N, K):
    A, W = dense_case(M * 7 + N + K, M, N, K)
    want = A.astype(np.float64) @ W.astype(np.float64).T
    assert rel(gemm_f16(A, W, dev), want) <= 1e-5


def test_f16_gemm_wide_tile(dev):
    """M = 256 and N = 32768 select the 256 x 256 tile; sampled columns against fp64."""
    M, N, K = 256, 32768, 512
    A, W = dense_case(11, M, N, K)
    got = gemm_f16(A, W, dev)
    cols = np.random.default_rng(3).choice(N, 256, replace=False)
    want = A.astype(np.float64) @ W[cols].astype(np.float64).T
    assert rel(got[:, cols], want) <= 1e-5


def test_f16_gemv_rows_bit_identical_across_m(dev):
    import qmm
    mmax = qmm.gemv_max_m() - 1
    A, W = dense_case(5, mmax, 777, 2048)
    full = gemm_f16(A, W, dev)
    for M in (1, 2, 4, 7, mmax):
        assert np.array_equal(gemm_f16(A[:M], W, dev), full[:M])


def test_f16_gemv_rows_bit_identical_across_m_long_k(dev):
    """K = 28672 fp16 weights: four staged activation rows (224 KiB) exceed the LDS, so M = 3, 4
    run two 2-row blocks, M = 2 one, M = 5, 8 the windowed kernel; fp32 and fp16 activations.
    Every row equals its M = 1 call bit for bit and an fp64 product within the GEMV bar."""
    N, K = 96, 28672
    A, W = dense_case(29, 8, N, K)
    import torch
    import qmm
    Wd = t(W, dev)
    for dt in (np.float32, np.float16):
        x = A.astype(dt)

        def run(a):
            C = qmm.gemm(F16, t(a, dev), Wd, N, K, out_dtype=torch.float32)
            torch.cuda.synchronize()
            return C.cpu().numpy()
        single = np.concatenate([run(x[m:m + 1]) for m in range(8)])
        assert rel(single, A.astype(np.float64) @ W.astype(np.float64).T) <= 1e-5
        for M in (2, 3, 4, 5, 8):
            np.testing.assert_array_equal(run(x[:M]), single[:M], err_msg=f"M={M} {dt.__name__}")


def test_f16_fused_batch_bit_identical(dev):
    import torch
    import qmm
    K = 1024
    r = np.random.default_rng(9)
    A = r.standard_normal((1, K)).astype(np.float16)
    Ws = [(r.standard_normal((n, K)) / 32).astype(np.float16) for n in (512, 128, 128)]
    Ad = t(A, dev)
    Wd = [t(w, dev) for w in Ws]
    single = [qmm.gemm(F16, Ad, w, w.shape[0], K) for w in Wd]
    outs = [torch.empty((1, w.shape[0]), dtype=torch.float32, device=dev) for w in Ws]
    descs = (qmm.GemmDesc * 3)()
    for d, w, o in zip(descs, Wd, outs):
        d.ggml_type, d.A, d.a_dtype, d.W, d.C, d.c_dtype = F16, Ad.data_ptr(), qmm.DTYPE_F16, w.data_ptr(), o.data_ptr(), \
            qmm.DTYPE_F32
        d.M, d.N, d.K = 1, w.shape[0], K
    qmm.gemm_batch(descs)
    torch.cuda.synchronize()
    for a, b in zip(single, outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("qt", [O.GGML_Q8_0, O.GGML_Q4_0])
def test_f16_prefill_bit_identical_to_q8_0_q4_0_prefill(dev, qt):
    """At prefill sizes a Q8_0 / Q4_0 weight enters the MFMA as exactly the reference's fp16
    dequantized value, so the F16 path on dequant(W) must reproduce the quantized path on W bit
    for bit (same tiles, same k order)."""
    import torch
    import qmm
    M, N, K = 64, 512, 1024
    r = np.random.default_rng(21 + qt)
    raw = QUANT[qt](r.standard_normal(N * K).astype(np.float32))
    w16 = O.dequantize_f16(qt, raw, N * K).reshape(N, K)
    A = t(r.standard_normal((M, K)).astype(np.float16), dev)
    q = qmm.gemm(qt, A, t(raw, dev), N, K)
    f = qmm.gemm(F16, A, t(w16, dev), N, K)
    torch.cuda.synchronize()
    assert torch.equal(q, f)


# ------------------------------------------------------------------ matmul_module (host arrays)

def test_module_matmul_and_matmul_nt(dev):
    import matmul_module as mm
    for M, N, K in ((1, 64, 256), (7, 100, 200), (70, 130, 96)):
        A, W = dense_case(M + N + K, M, N, K)
        want = A.astype(np.float64) @ W.astype(np.float64).T
        C = np.zeros((M, N), np.float16)
        mm.matmul_nt(A, W, C, M, N, K)
        assert rel(C, want) <= 1e-3
        C2 = np.zeros((M, N), np.float16)
        mm.matmul(A, np.ascontiguousarray(W.T), C2, M, N, K)
        assert np.array_equal(C2, C)  # the transposed operand is the same product


def test_module_layer_ops(dev):
    import matmul_module as mm
    r = np.random.default_rng(31)
    M, K = 5, 320
    x = r.standard_normal((M, K)).astype(np.float16)
    res = r.standard_normal((M, K)).astype(np.float16)
    w = (1 + 0.1 * r.standard_normal(K)).astype(np.float16)
    out = np.zeros_like(x)
    mm.rmsnorm(x, w, out, M, K)
    assert maxerr(out, L.rmsnorm(x, w, 1e-5)) < 2e-3
    h, n = np.zeros_like(x), np.zeros_like(x)
    mm.rmsnorm_residual(x, res, w, h, n, M, K, 1e-6)
    wh, wn = L.rmsnorm_residual(x, res, w, 1e-6)
    assert np.array_equal(h, wh) and maxerr(n, wn) < 2e-3
    o = np.zeros_like(x)
    mm.residual_add(x, res, o, M * K)
    assert np.array_equal(o, L.residual_add(x, res))
    g = (r.standard_normal(1000) * 3).astype(np.float16)
    u = r.standard_normal(1000).astype(np.float16)
    s = np.zeros_like(g)
    mm.swiglu(g, u, s, 1000)
    assert maxerr(s, L.swiglu(g, u)) < 2e-3
    for neox in (False, True):
        q = r.standard_normal((3, 4, 64)).astype(np.float16)
        qo = np.zeros_like(q)
        mm.rope(q, qo, 3, 4, 64, 17, 500000.0, neox)
        assert maxerr(qo, L.rope(q, 17, 500000.0, neox)) < 2e-3
    qo = np.zeros_like(q)
    mm.rope(q, qo, 3, 4, 64)  # defaults: position 0, base 10000, adjacent pairs
    assert maxerr(qo, L.rope(q, 0, 10000.0, False)) < 2e-3
    Q = r.standard_normal((4, 8, 64)).astype(np.float16)
    Kc = r.standard_normal((9, 2, 64)).astype(np.float16)
    V = r.standard_normal((9, 2, 64)).astype(np.float16)
    out = np.zeros_like(Q)
    mm.gqa_attention(Q, Kc, V, out, 4, 9, 8, 2, 64, 5)
    assert maxerr(out, L.gqa_attention(Q, Kc, V, 5)) < 2e-3
    out = np.zeros_like(Q)
    mm.gqa_attention(Q, Kc, V, out, 4, 9, 8, 2, 64, 0, 0.05, False)
    assert maxerr(out, L.gqa_attention(Q, Kc, V, 0, 0.05, False)) < 2e-3
    with pytest.raises(ValueError, match="num_heads must be divisible by num_kv_heads"):
        mm.gqa_attention(Q, Kc, V, out, 4, 4, 8, 3, 64)


def test_module_kv_cache_and_cached_attention(dev):
    import matmul_module as mm
    r = np.random.default_rng(41)
    H, KVH, D = 8, 2, 64
    Q = r.standard_normal((12, H, D)).astype(np.float16)
    K = r.standard_normal((12, KVH, D)).astype(np.float16)
    V = r.standard_normal((12, KVH, D)).astype(np.float16)
    mm.kv_cache_free()
    with pytest.raises(RuntimeError, match="not initialized"):
        mm.gqa_attention_cached(Q[:1], K[:1], V[:1], np.zeros((1, H, D), np.float16), 0, 1, 0, H, KVH, D)
    mm.kv_cache_init(2, 16, KVH, D)
    try:
        out = np.zeros((10, H, D), np.float16)
        mm.gqa_attention_cached(Q[:10], K[:10], V[:10], out, 1, 10, 0, H, KVH, D)
        assert maxerr(out, L.gqa_attention(Q[:10], K[:10], V[:10], 0)) < 2e-3
        out1 = np.zeros((1, H, D), np.float16)
        mm.gqa_attention_cached(Q[10:11], K[10:11], V[10:11], out1, 1, 1, 10, H, KVH, D)
        assert maxerr(out1, L.gqa_attention(Q[10:11], K[:11], V[:11], 10)) < 2e-3
        with pytest.raises(IndexError, match="layer_idx out of range"):
            mm.gqa_attention_cached(Q[:1], K[:1], V[:1], out1, 2, 1, 0, H, KVH, D)
        with pytest.raises(IndexError, match="exceeds max_seq_len"):
            mm.gqa_attention_cached(Q[:2], K[:2], V[:2], np.zeros((2, H, D), np.float16), 0, 2, 15, H, KVH, D)
        with pytest.raises(ValueError, match="mismatch"):
            mm.gqa_attention_cached(Q[:1], Q[:1, :4], Q[:1, :4], out1, 0, 1, 0, H, 4, D)
    finally:
        mm.kv_cache_free()


def layer_weights(r, hidden, inter, heads, kvh, d, types):
    shapes = {"q": (heads * d, hidden), "k": (kvh * d, hidden), "v": (kvh * d, hidden), "o": (hidden, heads * d),
              "gate": (inter, hidden), "up": (inter, hidden), "down": (hidden, inter)}
    packed, deq = {}, {}
    for name, (n, k) in shapes.items():
        w = (r.standard_normal((n, k)) / math.sqrt(k)).astype(np.float32)
        if types[name] == F16:
            deq[name] = w.astype(np.float16)
            packed[name] = deq[name]
        else:
            packed[name] = QUANT[types[name]](w.reshape(-1))
            deq[name] = O.dequantize_f16(types[name], packed[name], n * k).reshape(n, k)
    deq["attn_norm"] = (1 + 0.05 * r.standard_normal(hidden)).astype(np.float16)
    deq["ffn_norm"] = (1 + 0.05 * r.standard_normal(hidden)).astype(np.float16)
    return packed, deq


@pytest.mark.parametrize("prefill", [3, 33])
def test_module_forward_layer_cached(dev, prefill):
    """The reference's forward_layer_cached from host arrays, F16 and quantized weights mixed."""
    import matmul_module as mm
    r = np.random.default_rng(60 + prefill)
    hidden, inter, heads, kvh, d = 256, 512, 8, 2, 32
    types = {"q": F16, "k": F16, "v": F16, "o": O.GGML_Q8_0, "gate": F16, "up": F16, "down": O.GGML_Q4_K}
    packed, deq = layer_weights(r, hidden, inter, heads, kvh, d, types)
    cfg = {"num_heads": heads, "num_kv_heads": kvh, "head_dim": d, "rms_norm_eps": 1e-5, "rope_freq_base": 10000.0,
           "rope_neox": False}
    x = (r.standard_normal((prefill + 1, hidden)) * 0.5).astype(np.float16)
    kc, vc = np.zeros((64, kvh, d), np.float16), np.zeros((64, kvh, d), np.float16)
    want_pre = L.layer_forward(x[:prefill], deq, cfg, kc, vc, 0)
    want_dec = L.layer_forward(x[prefill:], deq, cfg, kc, vc, prefill)

    def run(xs, pos):
        out = np.zeros_like(xs)
        mm.forward_layer_cached(xs, out, deq["attn_norm"], packed["q"], types["q"], packed["k"], types["k"],
                                packed["v"], types["v"], packed["o"], types["o"], deq["ffn_norm"], packed["gate"],
                                types["gate"], packed["up"], types["up"], packed["down"], types["down"], 1, xs.shape[0],
                                pos, hidden, inter, heads, kvh, d, 1e-5, 10000.0, False, 0.0)
        return out

    mm.kv_cache_init(2, 64, kvh, d)
    try:
        assert maxerr(run(np.ascontiguousarray(x[:prefill]), 0), want_pre) < 5e-3
        assert maxerr(run(np.ascontiguousarray(x[prefill:]), prefill), want_dec) < 5e-3
    finally:
        mm.kv_cache_free()


def test_forward_layer_device_f16_weights(dev):
    """qmm_forward_layer on device tensors with every projection F16."""
    import torch
    import qmm
    r = np.random.default_rng(77)
    hidden, inter, heads, kvh, d = 128, 256, 4, 1, 32
    types = {n: F16 for n in ("q", "k", "v", "o", "gate", "up", "down")}
    packed, deq = layer_weights(r, hidden, inter, heads, kvh, d, types)
    dw = {n: t(a, dev) for n, a in packed.items()}
    norms = {n: t(deq[n], dev) for n in ("attn_norm", "ffn_norm")}
    w = qmm.LayerWeights()
    w.attn_norm, w.attn_norm_dtype = norms["attn_norm"].data_ptr(), qmm.DTYPE_F16
    w.ffn_norm, w.ffn_norm_dtype = norms["ffn_norm"].data_ptr(), qmm.DTYPE_F16
    for f, n in (("wq", "q"), ("wk", "k"), ("wv", "v"), ("wo", "o"), ("wgate", "gate"), ("wup", "up"), ("wdown", "down")):
        setattr(w, f, dw[n].data_ptr())
        setattr(w, f + "_type", F16)
    c = qmm.LayerConfig()
    c.hidden_size, c.intermediate_size, c.num_heads, c.num_kv_heads, c.head_dim = hidden, inter, heads, kvh, d
    c.rms_norm_eps, c.rope_freq_base, c.rope_neox, c.scale = 1e-5, 10000.0, 1, 0.0
    cfg = {"num_heads": heads, "num_kv_heads": kvh, "head_dim": d, "rms_norm_eps": 1e-5, "rope_freq_base": 10000.0,
           "rope_neox": True}
    x = (r.standard_normal((40, hidden)) * 0.5).astype(np.float16)
    kc, vc = np.zeros((64, kvh, d), np.float16), np.zeros((64, kvh, d), np.float16)
    want = L.layer_forward(x, deq, cfg, kc, vc, 0)
    lib = qmm.lib()
    qmm.check(lib.qmm_kv_cache_init(1, 64, kvh, d))
    try:
        X = t(x, dev)
        Y = torch.empty_like(X)
        qmm.check(lib.qmm_forward_layer(c, w, X.data_ptr(), Y.data_ptr(), 0, 40, 0,
                                        torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert maxerr(Y.cpu().numpy(), want) < 5e-3
    finally:
        qmm.check(lib.qmm_kv_cache_free())
