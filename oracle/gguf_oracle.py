"""CPU oracle for the GGUF quantized-matmul path (TEST INFRASTRUCTURE ONLY).

This module checks results and is never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped path (``libqmm_gfx950.so`` and ``matmul_module``) never
calls into it and has no CPU fallback.

It restates, in NumPy, the reference repository's CPU path for fused
dequantize-and-multiply over GGUF ``Q4_0`` / ``Q8_0`` / ``Q4_K`` / ``Q6_K``
weight blocks:

* block layouts: ``src/kernels/dequantize.h:6-22`` and
  ``src/kernels/dequantize.hip:17-50`` (packed structs + ``static_assert`` sizes);
* ``get_scale_min_k4``: ``src/kernels/dequantize.hip:52-65``;
* CPU dequantizers (fp32 arithmetic, fp16 output):
  ``src/gguf_parser.py:374-384`` (Q4_0), ``:408-415`` (Q8_0),
  ``:471-502`` (Q4_K), ``:560-589`` (Q6_K);
* the reference matmul formula ``C = A.astype(f32) @ deq_f16(B).astype(f32).T``:
  ``tests/test_gguf_and_q4.py:126-128``, ``tests/test_phase5_scale.py:61-66, 92-99, 361-367``;
* the test-input quantizers ``quantize_*_cpu``: ``src/gguf_parser.py:344-371,
  387-405, 418-468, 505-557`` (used only to build inputs shaped like the
  reference's own tests).

Each function has two independent routes that tests compare bit-for-bit:
the vectorised restatement of the reference (``dequantize_*``), and a
"fields" decomposition ``w = a * code - b`` (``fields_*``) written from the
block-format description, which also yields the exact fp64 weights used as the
tolerance reference for GEMV/GEMM.  How each route is pinned (known-answer
blocks, closed forms, brute force) is recorded in ``tests/test_oracle.py``;
``tests/test_ref_vectors.py`` additionally pins the dequantizers and the
test-input quantizers byte-for-byte against outputs of the reference's own
``src/gguf_parser.py`` functions (``tests/golden/ref_vectors.npz``).  Every
function here has such a check; none is parity-unpinned.
"""

from __future__ import annotations

from typing import Callable, Dict, Tuple

import numpy as np

# GGMLType ids (src/gguf_parser.py:22-36) and (block_elems, block_bytes)
# (src/gguf_parser.py:40-55; src/kernels/dequantize.h:6-22).
GGML_F16 = 1
GGML_Q4_0 = 2
GGML_Q8_0 = 8
GGML_Q4_K = 12
GGML_Q6_K = 14

BLOCK_INFO: Dict[int, Tuple[int, int]] = {
    GGML_Q4_0: (32, 18),
    GGML_Q8_0: (32, 34),
    GGML_Q4_K: (256, 144),
    GGML_Q6_K: (256, 210),
}

TYPE_NAMES = {GGML_Q4_0: "q4_0", GGML_Q8_0: "q8_0", GGML_Q4_K: "q4_k", GGML_Q6_K: "q6_k"}
TYPE_BY_NAME = {v: k for k, v in TYPE_NAMES.items()}


def weight_bytes(ggml_type: int, n: int, k: int) -> int:
    """Packed byte size of an N x K weight (attention.hip:553-570 weight_bytes_for_type)."""
    qk, bb = BLOCK_INFO[ggml_type]
    if k % qk:
        raise ValueError(f"K={k} is not a multiple of {qk}")
    return n * (k // qk) * bb


def _blocks(raw: np.ndarray, ggml_type: int, num_elements: int) -> np.ndarray:
    qk, bb = BLOCK_INFO[ggml_type]
    nb = num_elements // qk
    return np.frombuffer(np.ascontiguousarray(raw).reshape(-1).view(np.uint8), dtype=np.uint8,
                         count=nb * bb).reshape(nb, bb)


def _f16_at(raw: np.ndarray, off: int) -> np.ndarray:
    """fp16 field at byte offset ``off`` of every block, as exact fp32 (nb, 1)."""
    return raw[:, off:off + 2].copy().view(np.float16).astype(np.float32)


# --------------------------------------------------------------------------------------
# Route 1: restatement of the reference's vectorised CPU dequantizers (fp16 output).
# --------------------------------------------------------------------------------------

def dequantize_q4_0_f32(raw: np.ndarray, num_elements: int) -> np.ndarray:
    """Q4_0 -> exact fp32 (src/gguf_parser.py:374-384 before its final fp16 cast)."""
    b = _blocks(raw, GGML_Q4_0, num_elements)
    d = _f16_at(b, 0)
    qs = b[:, 2:18]
    x0 = (qs & 0x0F).astype(np.int8) - 8
    x1 = (qs >> 4).astype(np.int8) - 8
    return (np.concatenate([x0, x1], axis=1).astype(np.float32) * d).reshape(-1)


def dequantize_q8_0_f32(raw: np.ndarray, num_elements: int) -> np.ndarray:
    """Q8_0 -> exact fp32 (src/gguf_parser.py:408-415)."""
    b = _blocks(raw, GGML_Q8_0, num_elements)
    d = _f16_at(b, 0)
    qs = b[:, 2:34].view(np.int8).astype(np.float32)
    return (qs * d).reshape(-1)


def dequantize_q4_k_f32(raw: np.ndarray, num_elements: int) -> np.ndarray:
    """Q4_K -> fp32 (src/gguf_parser.py:471-502): w = (d*sc)*q - dmin*m, one fp32 rounding."""
    b = _blocks(raw, GGML_Q4_K, num_elements)
    nsb = b.shape[0]
    d = _f16_at(b, 0)
    dmin = _f16_at(b, 2)
    scales = b[:, 4:16]
    qs = b[:, 16:144]
    sc_q = np.empty((nsb, 8), dtype=np.float32)
    m_q = np.empty((nsb, 8), dtype=np.float32)
    for j in range(4):
        sc_q[:, j] = (scales[:, j] & 63).astype(np.float32)
        m_q[:, j] = (scales[:, j + 4] & 63).astype(np.float32)
        sc_q[:, j + 4] = ((scales[:, j + 8] & 0x0F) | ((scales[:, j] >> 6) << 4)).astype(np.float32)
        m_q[:, j + 4] = ((scales[:, j + 8] >> 4) | ((scales[:, j + 4] >> 6) << 4)).astype(np.float32)
    out = np.empty((nsb, 256), dtype=np.float32)
    for chunk in range(4):
        q_chunk = qs[:, chunk * 32:(chunk + 1) * 32]
        q0 = (q_chunk & 0x0F).astype(np.float32)
        q1 = (q_chunk >> 4).astype(np.float32)
        d0 = (d[:, 0] * sc_q[:, 2 * chunk])[:, None]
        dm0 = (dmin[:, 0] * m_q[:, 2 * chunk])[:, None]
        d1 = (d[:, 0] * sc_q[:, 2 * chunk + 1])[:, None]
        dm1 = (dmin[:, 0] * m_q[:, 2 * chunk + 1])[:, None]
        out[:, chunk * 64:chunk * 64 + 32] = d0 * q0 - dm0
        out[:, chunk * 64 + 32:(chunk + 1) * 64] = d1 * q1 - dm1
    return out.reshape(-1)


def dequantize_q6_k_f32(raw: np.ndarray, num_elements: int) -> np.ndarray:
    """Q6_K -> exact fp32 (src/gguf_parser.py:560-589): w = d*sc*q, q in -32..31."""
    b = _blocks(raw, GGML_Q6_K, num_elements)
    nsb = b.shape[0]
    ql = b[:, 0:128]
    qh = b[:, 128:192]
    scales = b[:, 192:208].view(np.int8).astype(np.float32)
    d = _f16_at(b, 208)
    out = np.empty((nsb, 256), dtype=np.float32)
    for n in range(2):
        ql_n = ql[:, n * 64:(n + 1) * 64]
        qh_n = qh[:, n * 32:(n + 1) * 32]
        sc_n = scales[:, n * 8:(n + 1) * 8]
        q1 = (((ql_n[:, 0:32] & 0x0F) | (((qh_n >> 0) & 3) << 4)).astype(np.int8) - 32).astype(np.float32)
        q2 = (((ql_n[:, 32:64] & 0x0F) | (((qh_n >> 2) & 3) << 4)).astype(np.int8) - 32).astype(np.float32)
        q3 = (((ql_n[:, 0:32] >> 4) | (((qh_n >> 4) & 3) << 4)).astype(np.int8) - 32).astype(np.float32)
        q4 = (((ql_n[:, 32:64] >> 4) | (((qh_n >> 6) & 3) << 4)).astype(np.int8) - 32).astype(np.float32)
        for t, qt in enumerate((q1, q2, q3, q4)):
            base = n * 128 + 32 * t
            out[:, base:base + 16] = d * sc_n[:, 2 * t:2 * t + 1] * qt[:, 0:16]
            out[:, base + 16:base + 32] = d * sc_n[:, 2 * t + 1:2 * t + 2] * qt[:, 16:32]
    return out.reshape(-1)


DEQUANT_F32: Dict[int, Callable[[np.ndarray, int], np.ndarray]] = {
    GGML_Q4_0: dequantize_q4_0_f32,
    GGML_Q8_0: dequantize_q8_0_f32,
    GGML_Q4_K: dequantize_q4_k_f32,
    GGML_Q6_K: dequantize_q6_k_f32,
}


def dequantize_f16(ggml_type: int, raw: np.ndarray, num_elements: int) -> np.ndarray:
    """The reference CPU dequantizer output: fp32 result rounded to fp16 (RNE, subnormals kept)."""
    return DEQUANT_F32[ggml_type](raw, num_elements).astype(np.float16)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round fp32 to bf16 (round-to-nearest-even), returned as uint16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------------------------------
# Route 2: fields decomposition w = a * code - b, written from the block-format description
# (dequantize.hip:17-65). Exact in fp64; a*code is exact in fp32 for every format.
# --------------------------------------------------------------------------------------

def get_scale_min_k4(j: int, q: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """6-bit (scale, min) of Q4_K sub-block j from the 12 packed bytes (dequantize.hip:52-65)."""
    q = q.astype(np.int64)
    if j < 4:
        return q[..., j] & 63, q[..., j + 4] & 63
    sc = (q[..., j + 4] & 0x0F) | ((q[..., j - 4] >> 6) << 4)
    m = (q[..., j + 4] >> 4) | ((q[..., j] >> 6) << 4)
    return sc, m


def fields(ggml_type: int, raw: np.ndarray, num_elements: int):
    """Per-weight (a, code, b) with w = a*code - b; a, b fp64 exact, code int64."""
    qk, _ = BLOCK_INFO[ggml_type]
    blk = _blocks(raw, ggml_type, num_elements)
    nb = blk.shape[0]
    a = np.empty((nb, qk), dtype=np.float64)
    code = np.empty((nb, qk), dtype=np.int64)
    b = np.zeros((nb, qk), dtype=np.float64)
    if ggml_type == GGML_Q4_0:
        d = _f16_at(blk, 0).astype(np.float64)
        for j in range(16):
            byte = blk[:, 2 + j].astype(np.int64)
            code[:, j] = (byte & 15) - 8
            code[:, j + 16] = (byte >> 4) - 8
        a[:] = d
    elif ggml_type == GGML_Q8_0:
        d = _f16_at(blk, 0).astype(np.float64)
        code[:] = blk[:, 2:34].view(np.int8).astype(np.int64)
        a[:] = d
    elif ggml_type == GGML_Q4_K:
        d = _f16_at(blk, 0).astype(np.float64)[:, 0]
        dmin = _f16_at(blk, 2).astype(np.float64)[:, 0]
        sc_bytes = blk[:, 4:16]
        qs = blk[:, 16:144].astype(np.int64)
        for s in range(8):
            sc, m = get_scale_min_k4(s, sc_bytes)
            c, hi = divmod(s, 2)
            nib = (qs[:, 32 * c:32 * c + 32] >> (4 * hi)) & 15
            code[:, 32 * s:32 * s + 32] = nib
            a[:, 32 * s:32 * s + 32] = (d * sc)[:, None]
            b[:, 32 * s:32 * s + 32] = (dmin * m)[:, None]
    elif ggml_type == GGML_Q6_K:
        ql = blk[:, 0:128].astype(np.int64)
        qh = blk[:, 128:192].astype(np.int64)
        sc = blk[:, 192:208].view(np.int8).astype(np.float64)
        d = _f16_at(blk, 208).astype(np.float64)[:, 0]
        for i in range(256):
            n, r = divmod(i, 128)
            t, l = divmod(r, 32)
            lo = ql[:, 64 * n + l + 32 * (t & 1)]
            low4 = (lo >> (4 * (t >> 1))) & 15
            hi2 = (qh[:, 32 * n + l] >> (2 * t)) & 3
            code[:, i] = (low4 | (hi2 << 4)) - 32
            a[:, i] = d * sc[:, 8 * n + l // 16 + 2 * t]
    else:
        raise ValueError(f"unsupported ggml_type {ggml_type}")
    return a.reshape(-1), code.reshape(-1), b.reshape(-1)


def dequantize_f64(ggml_type: int, raw: np.ndarray, num_elements: int) -> np.ndarray:
    """Mathematically exact weights (no rounding at all), fp64."""
    a, code, b = fields(ggml_type, raw, num_elements)
    return a * code.astype(np.float64) - b


def dequantize_fields_f32(ggml_type: int, raw: np.ndarray, num_elements: int) -> np.ndarray:
    """fp32 weights via the fields route: a*code exact in fp32, one rounding at ``- b``."""
    a, code, b = fields(ggml_type, raw, num_elements)
    prod = (a.astype(np.float32) * code.astype(np.float32))
    return (prod - b.astype(np.float32)).astype(np.float32)


# --------------------------------------------------------------------------------------
# Matmul references.
# --------------------------------------------------------------------------------------

def matmul_reference(ggml_type: int, A: np.ndarray, raw: np.ndarray, N: int, K: int) -> np.ndarray:
    """The reference test formula: A.astype(f32) @ dequant_f16(B).astype(f32).T (fp32 result)."""
    W = dequantize_f16(ggml_type, raw, N * K).reshape(N, K).astype(np.float32)
    return np.asarray(A, dtype=np.float32).reshape(-1, K) @ W.T


def matmul_f64(ggml_type: int, A: np.ndarray, raw: np.ndarray, N: int, K: int) -> np.ndarray:
    """fp64 product of the activations (as given) with the exact weights."""
    W = dequantize_f64(ggml_type, raw, N * K).reshape(N, K)
    return np.asarray(A, dtype=np.float64).reshape(-1, K) @ W.T


def dequantize_f16_operands(ggml_type: int, raw: np.ndarray, num_elements: int) -> np.ndarray:
    """Weights as the f16 MFMA operands of the prefill GEMM, returned as exact fp32.

    With ``w = a*code - b`` (``fields``): the group scale ``a`` and offset ``-b`` are each rounded
    to f16 once (RNE), then ``w = f16(code*a16 + (-b)16)`` with a single rounding (a fused f16
    multiply-add; ``b = 0`` for Q4_0 / Q8_0 / Q6_K, where it is an f16 multiply).  ``a`` is exact
    in fp32 before its rounding (f16 ``d`` times a 6-bit or int8 sub-scale).  For Q4_0 / Q8_0 the
    scale is ``d`` itself, so the result equals the reference CPU dequantizer's fp16 output
    (src/gguf_parser.py:374-384, 408-415); for Q4_K / Q6_K rounding the scale first differs from
    the reference's fp32 route (src/gguf_parser.py:471-502, 560-589) by at most one f16 ulp of the
    weight.  ``code*a16 + b16`` is exact in fp64 for every representable field combination whose
    two terms lie within 2^36 of each other, so the fp64 -> f16 cast is the one rounding.
    """
    a, code, b = fields(ggml_type, raw, num_elements)
    a16 = a.astype(np.float16).astype(np.float64)
    nb16 = (-b).astype(np.float16).astype(np.float64)
    return (code.astype(np.float64) * a16 + nb16).astype(np.float16).astype(np.float32)


def matmul_f16_operands(ggml_type: int, A: np.ndarray, raw: np.ndarray, N: int, K: int) -> np.ndarray:
    """fp64 product of the prefill GEMM's f16 operands: f16(A) @ dequantize_f16_operands(W).T.

    This is the exact value an f16-MFMA GEMM with fp32 accumulation approximates (only its
    accumulation rounds), so it pins the prefill kernel's dequantization, scale rounding and k
    ordering far more tightly than the fp64 tolerance does.
    """
    W16 = dequantize_f16_operands(ggml_type, raw, N * K).reshape(N, K).astype(np.float64)
    A16 = np.asarray(A, dtype=np.float32).reshape(-1, K).astype(np.float16).astype(np.float64)
    return A16 @ W16.T


def max_rel_err(y: np.ndarray, y64: np.ndarray) -> float:
    """max_i |y_i - y64_i| / max_i |y64_i| (the tolerance metric for GEMV and GEMM)."""
    y = np.asarray(y, dtype=np.float64)
    denom = float(np.max(np.abs(y64)))
    return float(np.max(np.abs(y - y64))) / (denom if denom > 0 else 1.0)


# --------------------------------------------------------------------------------------
# Test-input quantizers, restated from src/gguf_parser.py (inputs only, not the hot path).
# --------------------------------------------------------------------------------------

def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """src/gguf_parser.py:344-371: d = fp16(max|x|/7), q = clip(round(x/d)+8, 0, 15)."""
    flat = np.asarray(w, dtype=np.float32).reshape(-1, 32)
    nb = flat.shape[0]
    d16 = (np.max(np.abs(flat), axis=1) / 7.0).astype(np.float16)
    d32 = d16.astype(np.float32)
    inv = np.where(d32 > 0.0, 1.0 / d32, 0.0)[:, None]
    q = np.clip(np.round(flat * inv) + 8.0, 0, 15).astype(np.uint8)
    out = np.empty((nb, 18), dtype=np.uint8)
    out[:, :2] = d16.view(np.uint8).reshape(nb, 2)
    out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    return out.reshape(-1)


def quantize_q8_0(w: np.ndarray) -> np.ndarray:
    """src/gguf_parser.py:387-405: d = fp16(max|x|/127), q = clip(round(x/d), -127, 127)."""
    flat = np.asarray(w, dtype=np.float32).reshape(-1, 32)
    nb = flat.shape[0]
    d16 = (np.max(np.abs(flat), axis=1) / 127.0).astype(np.float16)
    d32 = d16.astype(np.float32)
    inv = np.where(d32 > 0.0, 1.0 / d32, 0.0)[:, None]
    qs = np.clip(np.round(flat * inv), -127, 127).astype(np.int8)
    out = np.empty((nb, 34), dtype=np.uint8)
    out[:, :2] = d16.view(np.uint8).reshape(nb, 2)
    out[:, 2:] = qs.view(np.uint8)
    return out.reshape(-1)


def pack_q4_k(d16: np.ndarray, dmin16: np.ndarray, sc: np.ndarray, m: np.ndarray,
              q: np.ndarray) -> np.ndarray:
    """Pack Q4_K super-blocks from fields: d, dmin (fp16, [nsb]), 6-bit sc/m [nsb, 8], codes [nsb, 256].

    Byte layout follows get_scale_min_k4 (dequantize.hip:52-65) and the qs chunking of
    dequantize.hip:416-428 (low nibble = sub-block 2c, high nibble = 2c+1).
    """
    nsb = q.shape[0]
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    out = np.empty((nsb, 144), dtype=np.uint8)
    out[:, 0:2] = np.asarray(d16, dtype=np.float16).view(np.uint8).reshape(nsb, 2)
    out[:, 2:4] = np.asarray(dmin16, dtype=np.float16).view(np.uint8).reshape(nsb, 2)
    for j in range(4):
        out[:, 4 + j] = (sc[:, j] & 63) | ((sc[:, j + 4] >> 4) << 6)
        out[:, 8 + j] = (m[:, j] & 63) | ((m[:, j + 4] >> 4) << 6)
        out[:, 12 + j] = (sc[:, j + 4] & 0x0F) | ((m[:, j + 4] & 0x0F) << 4)
    qq = q.astype(np.uint8).reshape(nsb, 8, 32)
    for c in range(4):
        out[:, 16 + 32 * c:48 + 32 * c] = qq[:, 2 * c] | (qq[:, 2 * c + 1] << 4)
    return out.reshape(-1)


def quantize_q4_k(w: np.ndarray) -> np.ndarray:
    """src/gguf_parser.py:418-468 (mins-offset 4-bit codes, 6-bit sc/m, fp16 d/dmin)."""
    flat = np.asarray(w, dtype=np.float32).reshape(-1, 256)
    nsb = flat.shape[0]
    sub = flat.reshape(nsb, 8, 32)
    m_val = np.maximum(0.0, -np.min(sub, axis=2))
    shifted = sub + m_val[:, :, None]
    sc_val = np.max(shifted, axis=2) / 15.0
    d16 = (np.max(sc_val, axis=1) / 63.0).astype(np.float16)
    dmin16 = (np.max(m_val, axis=1) / 63.0).astype(np.float16)
    d32 = d16.astype(np.float32)[:, None]
    dmin32 = dmin16.astype(np.float32)[:, None]
    inv_d = np.where(d32 > 0.0, 1.0 / d32, 0.0)
    inv_dmin = np.where(dmin32 > 0.0, 1.0 / dmin32, 0.0)
    sc_q = np.clip(np.round(sc_val * inv_d), 0, 63).astype(np.uint8)
    m_q = np.clip(np.round(m_val * inv_dmin), 0, 63).astype(np.uint8)
    eff_d = (d32 * sc_q.astype(np.float32))[:, :, None]
    eff_m = (dmin32 * m_q.astype(np.float32))[:, :, None]
    inv_eff_d = np.where(eff_d > 0.0, 1.0 / eff_d, 0.0)
    q_sub = np.clip(np.round((sub + eff_m) * inv_eff_d), 0, 15).astype(np.uint8)
    return pack_q4_k(d16, dmin16, sc_q, m_q, q_sub.reshape(nsb, 256))


def pack_q6_k(d16: np.ndarray, sc: np.ndarray, u: np.ndarray) -> np.ndarray:
    """Pack Q6_K super-blocks from fields: d (fp16 [nsb]), int8 sc [nsb, 16], unsigned codes u [nsb, 256] (0..63).

    Layout: ql[128] @0, qh[64] @128, scales[16] @192, d @208 (dequantize.hip:39-44, 565-583).
    """
    nsb = u.shape[0]
    u = u.astype(np.uint8)
    ql = np.empty((nsb, 128), dtype=np.uint8)
    qh = np.empty((nsb, 64), dtype=np.uint8)
    for n in range(2):
        h = u[:, n * 128:(n + 1) * 128]
        q1, q2, q3, q4 = h[:, 0:32], h[:, 32:64], h[:, 64:96], h[:, 96:128]
        ql[:, n * 64:n * 64 + 32] = (q1 & 0x0F) | ((q3 & 0x0F) << 4)
        ql[:, n * 64 + 32:(n + 1) * 64] = (q2 & 0x0F) | ((q4 & 0x0F) << 4)
        qh[:, n * 32:(n + 1) * 32] = (((q1 >> 4) & 3) | (((q2 >> 4) & 3) << 2)
                                      | (((q3 >> 4) & 3) << 4) | (((q4 >> 4) & 3) << 6))
    out = np.empty((nsb, 210), dtype=np.uint8)
    out[:, 0:128] = ql
    out[:, 128:192] = qh
    out[:, 192:208] = np.asarray(sc, dtype=np.int8).view(np.uint8)
    out[:, 208:210] = np.asarray(d16, dtype=np.float16).view(np.uint8).reshape(nsb, 2)
    return out.reshape(-1)


def quantize_q6_k(w: np.ndarray) -> np.ndarray:
    """src/gguf_parser.py:505-557 (symmetric 6-bit codes, int8 sub-scales, fp16 d)."""
    flat = np.asarray(w, dtype=np.float32).reshape(-1, 256)
    nsb = flat.shape[0]
    sub = flat.reshape(nsb, 16, 16)
    sc_float = np.max(np.abs(sub), axis=2) / 31.0
    d16 = (np.max(sc_float, axis=1) / 127.0).astype(np.float16)
    d32 = d16.astype(np.float32)[:, None]
    inv_d = np.where(d32 > 0.0, 1.0 / d32, 0.0)
    sc_i8 = np.clip(np.round(sc_float * inv_d), -127, 127).astype(np.int8)
    eff = (d32 * sc_i8.astype(np.float32))[:, :, None]
    inv_eff = np.where(np.abs(eff) > 0.0, 1.0 / eff, 0.0)
    u = np.clip(np.round(sub * inv_eff) + 32.0, 0, 63).astype(np.uint8).reshape(nsb, 256)
    return pack_q6_k(d16, sc_i8, u)


QUANTIZE = {GGML_Q4_0: quantize_q4_0, GGML_Q8_0: quantize_q8_0,
            GGML_Q4_K: quantize_q4_k, GGML_Q6_K: quantize_q6_k}


# --------------------------------------------------------------------------------------
# Synthetic weights drawn directly in code space (the benchmark configurations).
# --------------------------------------------------------------------------------------

def _abs_normal_f16(rng: np.random.Generator, n: int, scale: float) -> np.ndarray:
    return (np.abs(rng.standard_normal(n)) * scale).astype(np.float16)


def synth_weights(ggml_type: int, N: int, K: int, rng: np.random.Generator) -> np.ndarray:
    """Random packed weights with the benchmark distributions.

    Q4_0: d = fp16(|N(0,1)|*0.02), 16 uniform random bytes per block.
    Q8_0: d = fp16(|N(0,1)|*0.01), codes uniform in -127..127.
    Q4_K: d, dmin = fp16(|N(0,1)|*0.01), 12 uniform scale bytes, 128 uniform qs bytes.
    Q6_K: d = fp16(|N(0,1)|*0.01), uniform ql/qh bytes, int8 scales uniform in -128..127.
    """
    qk, bb = BLOCK_INFO[ggml_type]
    nb = N * (K // qk)
    out = np.empty((nb, bb), dtype=np.uint8)
    if ggml_type == GGML_Q4_0:
        out[:, 0:2] = _abs_normal_f16(rng, nb, 0.02).view(np.uint8).reshape(nb, 2)
        out[:, 2:18] = rng.integers(0, 256, size=(nb, 16), dtype=np.uint8)
    elif ggml_type == GGML_Q8_0:
        out[:, 0:2] = _abs_normal_f16(rng, nb, 0.01).view(np.uint8).reshape(nb, 2)
        out[:, 2:34] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    elif ggml_type == GGML_Q4_K:
        out[:, 0:2] = _abs_normal_f16(rng, nb, 0.01).view(np.uint8).reshape(nb, 2)
        out[:, 2:4] = _abs_normal_f16(rng, nb, 0.01).view(np.uint8).reshape(nb, 2)
        out[:, 4:144] = rng.integers(0, 256, size=(nb, 140), dtype=np.uint8)
    elif ggml_type == GGML_Q6_K:
        out[:, 0:208] = rng.integers(0, 256, size=(nb, 208), dtype=np.uint8)
        out[:, 208:210] = _abs_normal_f16(rng, nb, 0.01).view(np.uint8).reshape(nb, 2)
    else:
        raise ValueError(f"unsupported ggml_type {ggml_type}")
    return out.reshape(-1)
