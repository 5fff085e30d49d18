"""Test infrastructure only: CPU restatement of the reference's transformer-layer arithmetic
around the quantized projections.  Product code never imports this module.

Each function follows the reference kernel it restates (fp16 storage, fp32 arithmetic, one
rounding to fp16 per stored result) and the NumPy reference of the reference's own tests:
* rmsnorm            src/kernels/rmsnorm.hip:24-76 (out = half(x * rsqrt(mean(x^2) + eps) * w));
                     tests/test_layer.py:37-41
* rmsnorm_residual   src/kernels/rmsnorm.hip:78-140 (h = half(x + r); norm of the rounded h)
* residual_add       src/kernels/rmsnorm.hip (out = half(x + r))
* rope               src/kernels/rope.hip:17-50 (inv_freq = 1 / base^(2i/d) in fp32; adjacent
                     pairs (2i, 2i+1), or (i, i + d/2) for NeoX); tests/test_layer.py:44-73
* gqa_attention      src/kernels/attention.hip:35-123 (query head h reads KV head h / group,
                     causal rows see keys < start_pos + m + 1; softmax in fp32); tests/test_layer.py:76-105
* swiglu             src/kernels/mlp.hip:16-29 (silu(g) * u); tests/test_layer.py:108-112
* layer_forward      src/kernels/attention.hip:603-695 (launch_forward_layer_cached_fp16) with the
                     projections as fp32 products of the fp16 dequantized weights rounded to fp16
                     (the reference's own layer reference, tests/test_layer.py:265-287)

Pinned in tests/test_layer_oracle.py by closed forms (constant rows, unit weights, identity
rotation at position 0, norm preservation, rotation composition, one-key and equal-score
attention, causal masking, silu(0) = 0) and by a float64 brute force of each formula.
"""

from __future__ import annotations

import math

import numpy as np


def _f16(a):
    return np.asarray(a, dtype=np.float32).astype(np.float16)


def rmsnorm(x, w, eps=1e-5):
    """Rows of x (fp16 [M, K]) scaled by rsqrt(mean(x^2) + eps) and by w (fp16 [K])."""
    xf = np.asarray(x, np.float16).astype(np.float32)
    ms = np.mean(xf * xf, axis=-1, keepdims=True, dtype=np.float32)
    scale = (np.float32(1.0) / np.sqrt(ms + np.float32(eps))).astype(np.float32)
    return _f16(xf * scale * np.asarray(w, np.float16).astype(np.float32))


def residual_add(x, r):
    return _f16(np.asarray(x, np.float16).astype(np.float32) + np.asarray(r, np.float16).astype(np.float32))


def rmsnorm_residual(x, r, w, eps=1e-5):
    """(h, norm(h)) with h = half(x + r)."""
    h = residual_add(x, r)
    return h, rmsnorm(h, w, eps)


def rope_inv_freq(head_dim, freq_base):
    i = np.arange(head_dim // 2, dtype=np.float32)
    return (np.float32(1.0) / np.power(np.float32(freq_base), (np.float32(2.0) * i) / np.float32(head_dim))).astype(np.float32)


def rope(x, pos_offset=0, freq_base=10000.0, neox=False):
    """x fp16 [seq, heads, head_dim] rotated by position pos_offset + row."""
    xf = np.asarray(x, np.float16).astype(np.float32)
    seq, _, d = xf.shape
    half = d // 2
    ang = (np.arange(pos_offset, pos_offset + seq, dtype=np.float32)[:, None] * rope_inv_freq(d, freq_base)[None, :])
    c = np.cos(ang.astype(np.float64)).astype(np.float32)[:, None, :]
    s = np.sin(ang.astype(np.float64)).astype(np.float32)[:, None, :]
    if neox:
        a, b = xf[..., :half], xf[..., half:]
        out = np.concatenate([a * c - b * s, a * s + b * c], axis=-1)
    else:
        a, b = xf[..., 0::2], xf[..., 1::2]
        out = np.empty_like(xf)
        out[..., 0::2] = a * c - b * s
        out[..., 1::2] = a * s + b * c
    return _f16(out)


def gqa_attention(q, k, v, start_pos=0, scale=0.0, causal=True):
    """q fp16 [q_len, heads, d], k / v fp16 [kv_len, kv_heads, d] -> fp16 [q_len, heads, d]."""
    qf = np.asarray(q, np.float16).astype(np.float32)
    kf = np.asarray(k, np.float16).astype(np.float32)
    vf = np.asarray(v, np.float16).astype(np.float32)
    q_len, heads, d = qf.shape
    kv_len, kv_heads, _ = kf.shape
    group = heads // kv_heads
    if scale == 0.0:
        scale = 1.0 / math.sqrt(d)
    out = np.zeros_like(qf)
    for m in range(q_len):
        n = min(kv_len, start_pos + m + 1) if causal else kv_len
        for h in range(heads):
            g = h // group
            sc = (kf[:n, g, :] @ qf[m, h, :]) * np.float32(scale)
            p = np.exp(sc - sc.max())
            out[m, h, :] = (p / p.sum()) @ vf[:n, g, :]
    return _f16(out)


def swiglu(gate, up):
    g = np.asarray(gate, np.float16).astype(np.float32)
    u = np.asarray(up, np.float16).astype(np.float32)
    return _f16(g / (np.float32(1.0) + np.exp(-g)) * u)


def project(x, w_deq_f16):
    """fp16 activations [M, K] @ fp16 dequantized weights [N, K]^T in fp32, rounded to fp16."""
    return _f16(np.asarray(x, np.float16).astype(np.float32) @ np.asarray(w_deq_f16, np.float16).astype(np.float32).T)


def add_bias(y, b):
    """fp16 projection output plus an optional fp16 bias, added in fp32 and rounded to fp16
    (reference src/layer.py:274-282, 344-346)."""
    if b is None:
        return y
    return _f16(np.asarray(y, np.float16).astype(np.float32) + np.asarray(b, np.float16).astype(np.float32))


def layer_forward(x, w, cfg, k_cache, v_cache, pos_offset):
    """One layer on fp16 activations x [seq, hidden]; w maps 'attn_norm', 'ffn_norm' (fp16 [hidden])
    and 'q', 'k', 'v', 'o', 'gate', 'up', 'down' (fp16 dequantized [N, K]), and optionally the fp16
    biases 'bq', 'bk', 'bv', 'bo' (reference src/layer.py:274-282, 344-346); k_cache / v_cache
    (fp16 [max_seq, kv_heads, d]) receive this call's rotated keys and values at pos_offset."""
    seq = x.shape[0]
    H, kvh, d = cfg["num_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    eps, base, neox = cfg["rms_norm_eps"], cfg["rope_freq_base"], cfg["rope_neox"]
    nx = rmsnorm(x, w["attn_norm"], eps)
    q = add_bias(project(nx, w["q"]), w.get("bq")).reshape(seq, H, d)
    k = add_bias(project(nx, w["k"]), w.get("bk")).reshape(seq, kvh, d)
    v = add_bias(project(nx, w["v"]), w.get("bv")).reshape(seq, kvh, d)
    q = rope(q, pos_offset, base, neox)
    k = rope(k, pos_offset, base, neox)
    k_cache[pos_offset:pos_offset + seq] = k
    v_cache[pos_offset:pos_offset + seq] = v
    att = gqa_attention(q, k_cache[:pos_offset + seq], v_cache[:pos_offset + seq], pos_offset,
                        cfg.get("scale", 0.0) or 1.0 / math.sqrt(d), True)
    proj = add_bias(project(att.reshape(seq, H * d), w["o"]), w.get("bo"))
    h, nh = rmsnorm_residual(x, proj, w["ffn_norm"], eps)
    act = swiglu(project(nh, w["gate"]), project(nh, w["up"]))
    return residual_add(h, project(act, w["down"]))
