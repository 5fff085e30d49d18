"""Write ``tests/golden/ref_synthetic.gguf`` and ``tests/golden/ref_gguf.json``: a small GGUF
file written by the reference's own GGUF writer, what the reference's own parser reads from it,
and which malformed headers the reference parser rejects.

Run once, in a container that holds the reference checkout, as
``python tests/golden/make_ref_gguf.py [/path/to/reference]``.  The outputs are data only (a
GGUF file, the writer's inputs, the parser's outputs and the malformed inputs); no reference
source travels with them, and nothing at test time reads the reference.

Why: the GGUF module (``gguf.py``) restates ``write_synthetic_gguf`` and ``GGUFParser``
(reference ``src/gguf_parser.py:115-328, 590-648``).  The file pins the writer byte for byte,
the JSON pins the parser field by field (every metadata value type, arrays of arrays, a
non-default alignment, an interleaved foreign tensor for the layer spans), and the malformed
cases pin which inputs are rejected.
"""

from __future__ import annotations

import importlib.util
import io
import json
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT_GGUF = os.path.join(HERE, "ref_synthetic.gguf")
OUT_JSON = os.path.join(HERE, "ref_gguf.json")


def load_reference_parser(ref_root: str):
    path = os.path.join(ref_root, "src", "gguf_parser.py")
    spec = importlib.util.spec_from_file_location("reference_gguf_parser", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod  # its dataclasses look themselves up in sys.modules
    spec.loader.exec_module(mod)
    return mod


# Writer inputs: (key, value type id, value); arrays as [element type id, items].
METADATA = [
    ("general.architecture", 8, "llama"),
    ("general.alignment", 4, 64),
    ("llama.block_count", 4, 2),
    ("llama.embedding_length", 4, 256),
    ("test.u8", 0, 200), ("test.i8", 1, -100), ("test.u16", 2, 60000), ("test.i16", 3, -30000),
    ("test.i32", 5, -2000000000), ("test.f32", 6, 0.5), ("test.bool", 7, True), ("test.u64", 10, 2 ** 40 + 3),
    ("test.i64", 11, -(2 ** 40) - 5), ("test.f64", 12, 1.0e-5),
    ("test.str_array", 9, [8, ["alpha", "beta", "", "gamma"]]),
    ("test.u32_array", 9, [4, [1, 2, 3, 4, 5]]),
    ("test.nested", 9, [9, [[1, [-1, 2]], [1, []], [1, [7]]]]),
]
# (name, GGUF dims (ne[0] first), type id); payloads are seeded random bytes
TENSORS = [
    ("token_embd.weight", (64, 3), 8),
    ("blk.0.attn_q.weight", (256, 4), 12),
    ("blk.0.attn_norm.weight", (32,), 1),
    ("output_norm.weight", (16,), 0),  # a foreign tensor between layer-0 tensors
    ("blk.0.ffn_down.weight", (256, 2), 14),
    ("blk.1.attn_q.weight", (64, 2), 2),
    ("blk.1.ffn_up.weight", (256, 3), 12),
]
BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210)}


def payloads():
    rng = np.random.default_rng(2024)
    out = []
    for _, dims, t in TENSORS:
        qk, bb = BLOCK[t]
        n = int(np.prod(dims)) // qk * bb
        out.append(rng.integers(0, 256, n, dtype=np.uint8).tobytes())
    return out


def malformed(ref) -> list:
    """(label, bytes) of headers the parser must reject."""
    w = ref.write_synthetic_gguf
    T, V = ref.GGMLType, ref.GGUFValueType
    cases = []
    buf = io.BytesIO()
    w(buf, {"llama.block_count": (V.UINT32, 1)}, [("blk.0.attn_q.weight", (128,), T.F16, bytes(256))])
    cases.append(("truncated_data", buf.getvalue()[:-16]))
    cases.append(("bad_magic", b"GGUX" + buf.getvalue()[4:]))
    cases.append(("version_1", b"GGUF" + struct.pack("<IQQ", 1, 0, 0)))
    cases.append(("version_4", b"GGUF" + struct.pack("<IQQ", 4, 0, 0)))
    cases.append(("too_small", b"GG"))
    cases.append(("kv_count_huge", b"GGUF" + struct.pack("<IQQ", 3, 0, 10_000_000)))
    cases.append(("tensor_count_huge", b"GGUF" + struct.pack("<IQQ", 3, 10_000_000, 0)))
    for a in (0, 3, 30, 131072):
        b = io.BytesIO()
        w(b, {"general.alignment": (V.UINT32, a)}, [], alignment=32)
        cases.append((f"alignment_{a}", b.getvalue()))
    b = io.BytesIO()
    w(b, {"general.alignment": (V.STRING, "32")}, [], alignment=32)
    cases.append(("alignment_string", b.getvalue()))
    dims9 = bytearray(b"GGUF" + struct.pack("<IQQ", 3, 1, 0))
    dims9 += struct.pack("<Q", 3) + b"bad" + struct.pack("<I", 9) + struct.pack("<9Q", *([1] * 9))
    dims9 += struct.pack("<IQ", 1, 0)
    cases.append(("n_dims_9", bytes(dims9)))
    b = io.BytesIO()
    w(b, {}, [("dup", (32,), T.F16, bytes(64)), ("dup", (32,), T.F16, bytes(64))])
    cases.append(("duplicate_name", b.getvalue()))
    b = io.BytesIO()
    w(b, {}, [("zero", (0, 32), T.F16, b"")])
    cases.append(("zero_dim", b.getvalue()))
    unk = bytearray(b"GGUF" + struct.pack("<IQQ", 3, 1, 0))
    unk += struct.pack("<Q", 3) + b"unk" + struct.pack("<IQ", 1, 32) + struct.pack("<IQ", 999, 0)
    cases.append(("unknown_type", bytes(unk)))
    b = io.BytesIO()
    w(b, {}, [("odd", (33,), T.Q4_0, bytes(18))])
    cases.append(("not_block_multiple", b.getvalue()))
    return cases


def jsonable(v):
    if isinstance(v, list):
        return [jsonable(x) for x in v]
    return v


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    ref = load_reference_parser(ref_root)
    V, T = ref.GGUFValueType, ref.GGMLType

    def typed(vt, val):
        return [V(val[0]), [typed(val[0], x) for x in val[1]]] if vt == 9 else val

    meta = {k: (V(vt), (V(val[0]), [typed(val[0], x) for x in val[1]]) if vt == 9 else val) for k, vt, val in METADATA}
    tens = [(n, d, T(t), p) for (n, d, t), p in zip(TENSORS, payloads())]
    buf = io.BytesIO()
    ref.write_synthetic_gguf(buf, meta, tens, alignment=64)
    raw = buf.getvalue()
    p = ref.GGUFParser(raw)
    parsed = {
        "version": p.version, "tensor_count": p.tensor_count, "kv_count": p.kv_count, "alignment": p.alignment,
        "data_offset": p.data_offset,
        "metadata": {k: jsonable(v) for k, v in p.metadata.items()},
        "tensors": {n: {"dims": list(t.dims), "type": int(t.ggml_type), "rel_offset": t.rel_offset,
                        "abs_offset": t.abs_offset, "n_elements": t.n_elements, "n_bytes": t.n_bytes,
                        "shape_row_major": list(t.shape_row_major)} for n, t in p.tensors.items()},
        "layer_spans": {str(i): [list(s) for s in p.get_layer_byte_spans(i)] for i in (0, 1)},
        "layer_hull": {str(i): list(p.get_layer_byte_span(i)) for i in (0, 1)},
    }
    rejected = []
    for label, data in malformed(ref):
        try:
            ref.GGUFParser(data)
            outcome = "accepted"
        except ValueError as e:
            outcome = "ValueError: " + str(e)
        rejected.append({"label": label, "hex": data.hex(), "reference": outcome})
    with open(OUT_GGUF, "wb") as f:
        f.write(raw)
    doc = {"writer_inputs": {"metadata": METADATA, "tensors": [[n, list(d), t] for n, d, t in TENSORS],
                             "alignment": 64},
           "parsed": parsed, "malformed": rejected}
    with open(OUT_JSON, "w") as f:
        json.dump(doc, f, indent=1)
    print(f"wrote {OUT_GGUF} ({len(raw)} bytes) and {OUT_JSON} ({len(rejected)} malformed cases)")


if __name__ == "__main__":
    main()
