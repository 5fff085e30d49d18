"""Pins of oracle/layer_oracle.py (the CPU restatement of the reference's layer arithmetic)
by closed forms, invariants and float64 brute force, so that a dropped term, a wrong pairing or
index, or a transposed operand fails here before it can mask a kernel bug."""

import math

import numpy as np
import pytest

import layer_oracle as L


def rng(seed):
    return np.random.default_rng(seed)


def test_rmsnorm_closed_forms_and_brute_force():
    K = 256
    w = np.ones(K, np.float16)
    for c in (0.5, -3.0, 100.0):
        x = np.full((1, K), c, np.float16)
        y = L.rmsnorm(x, w, 1e-5).astype(np.float64)
        assert np.allclose(y, c / math.sqrt(c * c + 1e-5), rtol=1e-3)
    r = rng(1)
    x = r.standard_normal((5, 300)).astype(np.float16)
    w = (1 + 0.1 * r.standard_normal(300)).astype(np.float16)
    xd = x.astype(np.float64)
    want = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-5) * w.astype(np.float64)
    got = L.rmsnorm(x, w, 1e-5).astype(np.float64)
    assert np.max(np.abs(got - want) / (np.abs(want) + 1e-3)) < 1.5e-3  # one fp16 rounding
    # the weight multiplies the normalized row, column by column
    w2 = w.copy()
    w2[7] *= 2
    assert np.allclose(L.rmsnorm(x, w2)[:, 7].astype(np.float64), 2 * got[:, 7], rtol=1e-3)


def test_residual_forms():
    r = rng(2)
    x = r.standard_normal((3, 64)).astype(np.float16)
    res = r.standard_normal((3, 64)).astype(np.float16)
    h, nh = L.rmsnorm_residual(x, res, np.ones(64, np.float16))
    assert np.array_equal(h, (x.astype(np.float64) + res.astype(np.float64)).astype(np.float16))
    assert np.array_equal(nh, L.rmsnorm(h, np.ones(64, np.float16)))  # normalizes the rounded sum
    assert np.array_equal(L.residual_add(x, -x), np.zeros_like(x))


@pytest.mark.parametrize("neox", [False, True])
def test_rope_invariants(neox):
    r = rng(3)
    x = r.standard_normal((6, 4, 64)).astype(np.float16)
    assert np.array_equal(L.rope(x[:1], 0, 10000.0, neox), x[:1])  # position 0 is the identity
    y = L.rope(x, 5, 10000.0, neox).astype(np.float64)
    xd = x.astype(np.float64)
    if neox:
        pn_x = xd[..., :32] ** 2 + xd[..., 32:] ** 2
        pn_y = y[..., :32] ** 2 + y[..., 32:] ** 2
    else:
        pn_x = xd[..., 0::2] ** 2 + xd[..., 1::2] ** 2
        pn_y = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    assert np.allclose(pn_y, pn_x, rtol=4e-3, atol=1e-3)  # rotations keep each pair's norm
    # rotating by a then by b is rotating by a + b (up to the fp16 rounding in between)
    two = L.rope(L.rope(x, 3, 10000.0, neox), 5, 10000.0, neox).astype(np.float64)
    # rope(x, p) rotates row i by p + i, so composing shifts of 3 and 5 rotates row i by 8 + 2i
    want = np.stack([L.rope(x[i:i + 1], 8 + 2 * i, 10000.0, neox)[0] for i in range(6)]).astype(np.float64)
    assert np.max(np.abs(two - want)) < 1e-2  # two fp16 roundings of values up to ~4.5
    # brute force of one element in float64
    inv = 1.0 / 10000.0 ** (2.0 * 3 / 64)
    ang = (5 + 2) * inv
    a, b = (xd[2, 1, 3], xd[2, 1, 35]) if neox else (xd[2, 1, 6], xd[2, 1, 7])
    got = (y[2, 1, 3], y[2, 1, 35]) if neox else (y[2, 1, 6], y[2, 1, 7])
    assert abs(got[0] - (a * math.cos(ang) - b * math.sin(ang))) < 2e-3
    assert abs(got[1] - (a * math.sin(ang) + b * math.cos(ang))) < 2e-3


def test_rope_neox_is_the_adjacent_form_on_permuted_dims():
    r = rng(4)
    x = r.standard_normal((3, 2, 16)).astype(np.float16)
    perm = np.empty(16, int)
    perm[0::2], perm[1::2] = np.arange(8), np.arange(8, 16)   # adjacent slot -> neox dim
    adj = L.rope(x[..., perm], 9, 500000.0, False)
    neo = L.rope(x, 9, 500000.0, True)
    assert np.array_equal(adj, neo[..., perm])


def test_rope_inv_freq():
    f = L.rope_inv_freq(128, 500000.0).astype(np.float64)
    want = 1.0 / 500000.0 ** (np.arange(64) * 2.0 / 128)
    assert np.allclose(f, want, rtol=2e-6)


def test_attention_closed_forms():
    r = rng(5)
    H, G, d = 8, 2, 32
    v = r.standard_normal((7, G, d)).astype(np.float16)
    k = r.standard_normal((7, G, d)).astype(np.float16)
    q = r.standard_normal((1, H, d)).astype(np.float16)
    # one visible key: the output is that key's value
    out = L.gqa_attention(q, k[:1], v[:1], 0)
    assert np.array_equal(out[0, 0], v[0, 0]) and np.array_equal(out[0, H - 1], v[0, G - 1])
    # zero query: equal scores, the output is the mean of the visible values
    q0 = np.zeros((3, H, d), np.float16)
    out = L.gqa_attention(q0, k, v, start_pos=2)
    for m in range(3):
        want = v[:3 + m].astype(np.float64).mean(0)
        assert np.allclose(out[m, :H // G].astype(np.float64), want[0], atol=2e-3)
        assert np.allclose(out[m, H // G:].astype(np.float64), want[1], atol=2e-3)
    # causal rows see exactly their prefix
    qq = r.standard_normal((4, H, d)).astype(np.float16)
    full = L.gqa_attention(qq, k[:6], v[:6], start_pos=2)
    for m in range(4):
        assert np.array_equal(full[m], L.gqa_attention(qq[m:m + 1], k[:3 + m], v[:3 + m], start_pos=2 + m)[0])
    # heads of one group that carry the same query give the same output; other groups differ
    qs = np.repeat(qq[:, :1], H, axis=1)
    o = L.gqa_attention(qs, k[:6], v[:6], start_pos=2)
    assert np.array_equal(o[:, 0], o[:, H // G - 1]) and not np.array_equal(o[:, 0], o[:, H // G])
    # brute force float64
    sc = (k[:5, 1].astype(np.float64) @ qq[2, 5].astype(np.float64)) / math.sqrt(d)
    p = np.exp(sc - sc.max())
    p /= p.sum()
    assert np.allclose(full[2, 5].astype(np.float64), p @ v[:5, 1].astype(np.float64), atol=2e-3)


def test_swiglu_closed_forms():
    g = np.array([0.0, 12.0, -12.0, 1.0], np.float16)
    u = np.array([3.0, 2.0, 5.0, 1.0], np.float16)
    y = L.swiglu(g, u).astype(np.float64)
    assert y[0] == 0.0
    assert abs(y[1] - 24.0) < 0.02 and abs(y[2]) < 1e-3
    assert abs(y[3] - 1.0 / (1.0 + math.exp(-1.0))) < 1e-3


def _toy_layer(seed, hidden=64, inter=96, heads=4, kvh=2, d=16):
    r = rng(seed)
    cfg = {"num_heads": heads, "num_kv_heads": kvh, "head_dim": d, "rms_norm_eps": 1e-5,
           "rope_freq_base": 10000.0, "rope_neox": False}
    sh = {"q": (heads * d, hidden), "k": (kvh * d, hidden), "v": (kvh * d, hidden), "o": (hidden, heads * d),
          "gate": (inter, hidden), "up": (inter, hidden), "down": (hidden, inter)}
    w = {n: (r.standard_normal(s) / math.sqrt(s[1])).astype(np.float16) for n, s in sh.items()}
    w["attn_norm"] = (1 + 0.05 * r.standard_normal(hidden)).astype(np.float16)
    w["ffn_norm"] = (1 + 0.05 * r.standard_normal(hidden)).astype(np.float16)
    return cfg, w, r


def test_layer_with_zero_output_projections_is_identity():
    cfg, w, r = _toy_layer(6)
    w["o"] = np.zeros_like(w["o"])
    w["down"] = np.zeros_like(w["down"])
    x = r.standard_normal((3, 64)).astype(np.float16)
    kc = np.zeros((8, 2, 16), np.float16)
    vc = np.zeros_like(kc)
    assert np.array_equal(L.layer_forward(x, w, cfg, kc, vc, 0), x)
    assert np.any(kc[:3] != 0) and not np.any(kc[3:])  # the keys of this call land at 0..2


def test_layer_decode_after_prefill_matches_longer_prefill():
    cfg, w, r = _toy_layer(7)
    x = (r.standard_normal((5, 64)) * 0.5).astype(np.float16)
    kc, vc = np.zeros((8, 2, 16), np.float16), np.zeros((8, 2, 16), np.float16)
    full = L.layer_forward(x, w, cfg, kc, vc, 0)
    kc2, vc2 = np.zeros_like(kc), np.zeros_like(vc)
    first = L.layer_forward(x[:4], w, cfg, kc2, vc2, 0)
    last = L.layer_forward(x[4:], w, cfg, kc2, vc2, 4)
    assert np.max(np.abs(first.astype(np.float32) - full[:4].astype(np.float32))) < 2e-3
    assert np.max(np.abs(last.astype(np.float32) - full[4:].astype(np.float32))) < 2e-3


def test_add_bias_rounds_once_after_an_fp32_add():
    """add_bias (reference src/layer.py:274-282): fp32 sum of the fp16 output and the fp16 bias,
    rounded to fp16 once.  1 + 2^-11 and 3 + 2^-10 are ties (half an fp16 ulp): they round to
    even (1 and 3); -y cancels exactly; no bias leaves y unchanged; on random values the result is
    the exact sum rounded once (every fp32 sum of two fp16 values here is exact)."""
    y = np.array([[1.0, 3.0, -2.5, 65504.0]], np.float16)
    assert L.add_bias(y, None) is y
    b = np.array([2.0 ** -11, 2.0 ** -10, 2.5, -65504.0], np.float16)
    out = L.add_bias(y, b)
    assert out.dtype == np.float16
    assert out[0, 0] == np.float16(1.0)
    assert out[0, 1] == np.float16(3.0)
    assert out[0, 2] == 0.0 and out[0, 3] == 0.0
    r = rng(11)
    y = r.standard_normal((3, 40)).astype(np.float16)
    b = r.standard_normal(40).astype(np.float16)
    want = (y.astype(np.float64) + b.astype(np.float64)).astype(np.float16)  # exact sum, one rounding
    assert np.array_equal(L.add_bias(y, b), want)
