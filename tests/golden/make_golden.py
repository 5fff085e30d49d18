"""Generate the known-answer fixtures in ``tests/golden/kat_blocks.npz``.

The reference repository commits no golden vectors for this path
(``tests/fixtures/PROVENANCE.md:28-32``), so these are built from first principles:

* every block is packed byte by byte by the loops below, written directly from the GGML
  block layouts (``src/kernels/dequantize.h:6-22``, ``src/kernels/dequantize.hip:17-65``);
  the packing does not call the oracle;
* the chosen fields exercise every branch of the formats: Q4_0 low/high nibbles and a
  subnormal fp16 scale, the full int8 range of Q8_0, the ``j >= 4`` high-bit path of Q4_K's
  6-bit scales and mins, every 2-bit lane of Q6_K's ``qh`` and negative int8 scales;
* expected weights are ``a * code - b`` evaluated exactly in fp64, then rounded once to fp32
  and fp32 -> fp16 (the reference computes in fp32 and casts to fp16,
  ``src/gguf_parser.py:384, 415, 502, 589``);
* two tiny GEMV cases per format carry fp64 outputs ``y = x @ W^T``.

Run ``python tests/golden/make_golden.py`` to regenerate; the file is deterministic.
"""

from __future__ import annotations

import os
import struct

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kat_blocks.npz")


def f16_bytes(v: float) -> bytes:
    return struct.pack("<e", v)


def f16_value(v: float) -> float:
    return struct.unpack("<e", struct.pack("<e", v))[0]


def q4_0_block(d: float, codes):
    """codes: 32 ints in 0..15; w[j] = d * (codes[j] - 8)."""
    b = bytearray(f16_bytes(d))
    for j in range(16):
        b.append(codes[j] | (codes[j + 16] << 4))
    dd = f16_value(d)
    return bytes(b), [dd * (c - 8) for c in codes]


def q8_0_block(d: float, codes):
    """codes: 32 ints in -128..127; w[j] = d * codes[j]."""
    b = bytearray(f16_bytes(d))
    for c in codes:
        b += struct.pack("<b", c)
    dd = f16_value(d)
    return bytes(b), [dd * c for c in codes]


def q4_k_block(d: float, dmin: float, sc, mn, codes):
    """sc, mn: 8 six-bit ints; codes: 256 ints in 0..15; w = d*sc[s]*q - dmin*m[s], s = i // 32."""
    b = bytearray(f16_bytes(d) + f16_bytes(dmin))
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    b += bytes(s)
    for c in range(4):
        for l in range(32):
            b.append(codes[64 * c + l] | (codes[64 * c + 32 + l] << 4))
    dd, dm = f16_value(d), f16_value(dmin)
    w = [dd * sc[i // 32] * codes[i] - dm * mn[i // 32] for i in range(256)]
    return bytes(b), w


def q6_k_block(d: float, sc, ucodes):
    """sc: 16 int8; ucodes: 256 ints in 0..63; w[i] = d * sc[i // 16] * (ucodes[i] - 32)."""
    ql = [0] * 128
    qh = [0] * 64
    for i in range(256):
        n, r = divmod(i, 128)
        t, l = divmod(r, 32)
        u = ucodes[i]
        ql[64 * n + 32 * (t & 1) + l] |= (u & 15) << (4 * (t >> 1))
        qh[32 * n + l] |= ((u >> 4) & 3) << (2 * t)
    b = bytes(ql) + bytes(qh) + struct.pack("<16b", *sc) + f16_bytes(d)
    dd = f16_value(d)
    return b, [dd * sc[i // 16] * (ucodes[i] - 32) for i in range(256)]


def build():
    rng = np.random.default_rng(20261201)
    out = {}

    blocks = [
        q4_0_block(1.0, [j for j in range(16)] + [15 - j for j in range(16)]),
        q4_0_block(-0.5, [(5 * j) % 16 for j in range(32)]),
        q4_0_block(2.0 ** -20, [(11 * j + 3) % 16 for j in range(32)]),  # subnormal fp16 scale
        q4_0_block(1000.0, [15 if j % 2 else 0 for j in range(32)]),
    ]
    out["q4_0"] = blocks

    blocks = [
        q8_0_block(0.5, [8 * j - 128 for j in range(31)] + [127]),
        q8_0_block(2.0 ** -24, [int(v) for v in rng.integers(-128, 128, 32)]),  # min subnormal
        q8_0_block(-3.25, [int(v) for v in rng.integers(-128, 128, 32)]),
        q8_0_block(0.0999, [-128] * 16 + [127] * 16),
    ]
    out["q8_0"] = blocks

    blocks = [
        q4_k_block(1.0, 0.5, [1, 2, 3, 4, 40, 50, 60, 63], [5, 6, 7, 8, 33, 47, 18, 63],
                   [(7 * i + 3) % 16 for i in range(256)]),
        q4_k_block(0.01, 0.002, [int(v) for v in rng.integers(0, 64, 8)], [int(v) for v in rng.integers(0, 64, 8)],
                   [int(v) for v in rng.integers(0, 16, 256)]),
        q4_k_block(2.0 ** -18, 3.0, [63] * 8, [0, 63, 16, 48, 32, 15, 47, 31], [15] * 128 + [0] * 128),
    ]
    out["q4_k"] = blocks

    blocks = [
        q6_k_block(0.25, [-128, -1, 1, 127, 5, -7, 64, -64, 3, 2, -3, 100, -100, 17, -17, 0],
                   [(13 * i + 5) % 64 for i in range(256)]),
        q6_k_block(0.0123, [int(v) for v in rng.integers(-128, 128, 16)], [int(v) for v in rng.integers(0, 64, 256)]),
        q6_k_block(2.0 ** -22, [127] * 16, [63, 0] * 128),
    ]
    out["q6_k"] = blocks

    arrays = {}
    for name, blist in out.items():
        raw = b"".join(b for b, _ in blist)
        w64 = np.array([v for _, w in blist for v in w], dtype=np.float64)
        arrays[f"{name}_raw"] = np.frombuffer(raw, dtype=np.uint8).copy()
        arrays[f"{name}_w64"] = w64
        arrays[f"{name}_f32"] = w64.astype(np.float32)
        arrays[f"{name}_f16"] = w64.astype(np.float32).astype(np.float16)
        # Tiny GEMV: the blocks laid out as N rows of K weights; two activation rows.
        qk = 32 if name in ("q4_0", "q8_0") else 256
        n_rows = len(blist) if qk == 256 else 2
        k = w64.size // n_rows
        W = w64.reshape(n_rows, k)
        x = rng.standard_normal((2, k))
        arrays[f"{name}_gemv_n"] = np.array([n_rows, k], dtype=np.int64)
        arrays[f"{name}_gemv_x"] = x.astype(np.float32)
        arrays[f"{name}_gemv_y64"] = x.astype(np.float32).astype(np.float64) @ W.T
    return arrays


if __name__ == "__main__":
    arrays = build()
    np.savez(OUT, **arrays)
    print(OUT, sum(a.nbytes for a in arrays.values()), "bytes")
