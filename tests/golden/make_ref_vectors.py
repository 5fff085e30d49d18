"""Write ``tests/golden/ref_vectors.npz``: input/output vectors of the reference's own CPU
quantizers and dequantizers, produced by the reference code itself.

Run once, in a container that holds the reference checkout, as
``python tests/golden/make_ref_vectors.py [/path/to/reference]``.  The output is data only
(inputs and expected outputs); no reference source travels with it, and nothing at test time
reads the reference.

Why: the oracle's dequantizers are pinned by known-answer blocks and closed forms, but the
test-input quantizers it restates (``src/gguf_parser.py:344-371, 387-405, 418-468,
505-557``) are otherwise pinned only by round-trip error bounds.  Byte-exact outputs of the
reference functions on fixed seeded inputs pin the restatement (NumPy half-to-even rounding,
the fp16 cast of the scales, the ``max_abs / 7`` choice of Q4_0, the Q4_K scale/min search and
the Q6_K int8 sub-scales).  The dequantizer vectors add a second, independent pin of the
dequantize restatement against the reference code on random blocks.

Inputs (all seeded with ``numpy.random.default_rng``):
* quantizer inputs per format: N(0,1) * scale rows at several scales, plus special blocks
  (all zeros, a constant block, an all-negative block, a single spike, fp16-range extremes);
* dequantizer inputs per format: uniformly random bytes whose fp16 fields are replaced by
  finite values, plus the quantizer outputs above.
"""

from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "ref_vectors.npz")

FORMATS = {  # name: (block elems, block bytes, fp16 field offsets)
    "q4_0": (32, 18, (0,)),
    "q8_0": (32, 34, (0,)),
    "q4_k": (256, 144, (0, 2)),
    "q6_k": (256, 210, (208,)),
}


def load_reference_parser(ref_root: str):
    path = os.path.join(ref_root, "src", "gguf_parser.py")
    spec = importlib.util.spec_from_file_location("reference_gguf_parser", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod  # its dataclasses look themselves up in sys.modules
    spec.loader.exec_module(mod)
    return mod


def quantizer_inputs(qk: int, rng) -> np.ndarray:
    rows = []
    for scale in (0.02, 0.1, 0.4, 1.0, 7.5):
        rows.append(rng.standard_normal(4 * qk, dtype=np.float32) * np.float32(scale))
    special = np.zeros((6, qk), dtype=np.float32)
    special[1, :] = 0.3                                            # constant block
    special[2, :] = -np.abs(rng.standard_normal(qk, dtype=np.float32))  # all negative
    special[3, qk // 3] = 5.0                                      # single spike
    special[4, :] = rng.uniform(-60000.0, 60000.0, qk).astype(np.float32)  # near fp16 max
    special[5, :] = rng.standard_normal(qk).astype(np.float32) * np.float32(1e-5)  # subnormal d
    rows.append(special.reshape(-1))
    return np.concatenate(rows).astype(np.float32)


def dequant_inputs(name: str, rng) -> np.ndarray:
    qk, bb, f16_offsets = FORMATS[name]
    nb = 48
    raw = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    for off in f16_offsets:
        d = (np.abs(rng.standard_normal(nb)) * 0.01).astype(np.float16)
        d[:4] = np.array([0.0, 2.0 ** -20, 1.0, 65504.0], dtype=np.float16)  # zero, subnormal, one, max
        raw[:, off:off + 2] = d.view(np.uint8).reshape(nb, 2)
    return raw.reshape(-1)


def main(ref_root: str) -> None:
    ref = load_reference_parser(ref_root)
    quantize = {"q4_0": ref.quantize_q4_0_cpu, "q8_0": ref.quantize_q8_0_cpu,
                "q4_k": ref.quantize_q4_k_cpu, "q6_k": ref.quantize_q6_k_cpu}
    dequantize = {"q4_0": ref.dequantize_q4_0_cpu, "q8_0": ref.dequantize_q8_0_cpu,
                  "q4_k": ref.dequantize_q4_k_cpu, "q6_k": ref.dequantize_q6_k_cpu}
    out = {}
    with np.errstate(all="ignore"):
        for i, name in enumerate(FORMATS):
            qk = FORMATS[name][0]
            rng = np.random.default_rng(9000 + i)
            x = quantizer_inputs(qk, rng)
            q = np.asarray(quantize[name](x), dtype=np.uint8)
            out[f"{name}_quant_in"] = x
            out[f"{name}_quant_out"] = q
            out[f"{name}_quant_deq"] = np.asarray(dequantize[name](q, x.size), dtype=np.float16)
            raw = dequant_inputs(name, rng)
            n = raw.size // FORMATS[name][1] * qk
            out[f"{name}_deq_in"] = raw
            out[f"{name}_deq_out"] = np.asarray(dequantize[name](raw, n), dtype=np.float16)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {sum(v.nbytes for v in out.values())} bytes in {len(out)} arrays")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
