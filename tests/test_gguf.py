"""GGUF container parsing / writing and the library's parallel file reader (CPU only).

Pins:
* `tests/golden/ref_synthetic.gguf`, written by the reference's own `write_synthetic_gguf`
  (reference src/gguf_parser.py:590-648) from the inputs recorded in `ref_gguf.json`: gguf.py's
  writer reproduces it byte for byte, and gguf.py's parser reads every field the reference
  parser read (every metadata value type, nested arrays, alignment 64, tensor offsets, layer
  spans around an interleaved foreign tensor);
* the malformed headers the reference parser rejects raise ValueError here too, with the same
  leading text (reference src/gguf_parser.py:175-292; the reference tests
  tests/test_cpu_only.py:124-264);
* WeightStreamer's load-time type check (reference src/weight_loader.py:82-97) in ResidentWeights;
* qmm_read_file (host destinations): bytes equal the file's over many ranges, multi-piece
  ranges and empty ranges; out-of-file ranges raise ValueError, a missing file OSError.
"""

import io
import json
import os

import numpy as np
import pytest

import gguf
from gguf import GGMLType, GGUFParser, GGUFValueType, write_synthetic_gguf

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def ref():
    with open(os.path.join(GOLDEN, "ref_gguf.json")) as f:
        doc = json.load(f)
    with open(os.path.join(GOLDEN, "ref_synthetic.gguf"), "rb") as f:
        raw = f.read()
    return doc, raw


def _typed(vt, val):
    if vt == GGUFValueType.ARRAY:
        return (GGUFValueType(val[0]), [_typed(val[0], x) for x in val[1]])
    return val


def test_parser_reads_what_the_reference_parser_read(ref):
    doc, raw = ref
    want = doc["parsed"]
    p = GGUFParser(raw)
    assert (p.version, p.tensor_count, p.kv_count, p.alignment, p.data_offset) == (
        want["version"], want["tensor_count"], want["kv_count"], want["alignment"], want["data_offset"])
    assert json.loads(json.dumps(p.metadata)) == want["metadata"]
    assert list(p.tensors) == list(want["tensors"])
    for name, t in p.tensors.items():
        w = want["tensors"][name]
        assert (list(t.dims), int(t.ggml_type), t.rel_offset, t.abs_offset, t.n_elements, t.n_bytes,
                list(t.shape_row_major)) == (w["dims"], w["type"], w["rel_offset"], w["abs_offset"], w["n_elements"],
                                             w["n_bytes"], w["shape_row_major"]), name
        assert t.abs_offset % p.alignment == 0
    for i in (0, 1):
        assert [list(s) for s in p.get_layer_byte_spans(i)] == want["layer_spans"][str(i)]
        assert list(p.get_layer_byte_span(i)) == want["layer_hull"][str(i)]
    # the interleaved foreign tensor splits layer 0 into two spans that avoid it
    emb = p.tensors["output_norm.weight"]
    for a, n in p.get_layer_byte_spans(0):
        assert a + n <= emb.abs_offset or a >= emb.abs_offset + emb.n_bytes
    with pytest.raises(KeyError):
        p.get_layer_byte_spans(7)


def test_writer_reproduces_the_reference_writer_bytes(ref):
    doc, raw = ref
    inp = doc["writer_inputs"]
    meta = {k: (GGUFValueType(vt), _typed(vt, val)) for k, vt, val in inp["metadata"]}
    p = GGUFParser(raw)
    tens = []
    for name, dims, t in inp["tensors"]:
        info = p.tensors[name]
        tens.append((name, tuple(dims), GGMLType(t), raw[info.abs_offset:info.abs_offset + info.n_bytes]))
    buf = io.BytesIO()
    write_synthetic_gguf(buf, meta, tens, alignment=inp["alignment"])
    assert buf.getvalue() == raw


def test_malformed_headers_are_rejected_like_the_reference(ref):
    doc, _ = ref
    assert len(doc["malformed"]) >= 15
    for case in doc["malformed"]:
        assert case["reference"].startswith("ValueError: "), case["label"]
        with pytest.raises(ValueError) as e:
            GGUFParser(bytes.fromhex(case["hex"]))
        ref_lead = case["reference"][len("ValueError: "):].split(":")[0]
        assert str(e.value).split(":")[0] == ref_lead, (case["label"], str(e.value))


@pytest.mark.parametrize("alignment", [1, 32, 4096])
def test_round_trip_payloads_and_alignment(alignment):
    rng = np.random.default_rng(alignment)
    payloads = [rng.integers(0, 256, n, dtype=np.uint8).tobytes() for n in (18 * 4, 144 * 2, 2 * 7, 210)]
    tensors = [("blk.0.a", (128, 1), GGMLType.Q4_0, payloads[0]), ("blk.0.b", (512,), GGMLType.Q4_K, payloads[1]),
               ("c", (7,), GGMLType.F16, payloads[2]), ("blk.1.d", (256,), GGMLType.Q6_K, payloads[3])]
    meta = {"general.alignment": (GGUFValueType.UINT32, alignment), "k": (GGUFValueType.FLOAT64, -2.5)}
    buf = io.BytesIO()
    write_synthetic_gguf(buf, meta, tensors, alignment=alignment)
    raw = buf.getvalue()
    p = GGUFParser(memoryview(raw))
    assert p.alignment == alignment and p.metadata["k"] == -2.5
    for (name, dims, t, data) in tensors:
        info = p.tensors[name]
        assert info.dims == dims and info.ggml_type == t and info.abs_offset % alignment == 0
        assert raw[info.abs_offset:info.abs_offset + info.n_bytes] == data


def test_caller_buffer_stays_usable():
    buf = io.BytesIO()
    write_synthetic_gguf(buf, {}, [("blk.0.attn_norm.weight", (32,), GGMLType.F16, np.arange(32, dtype=np.float16).tobytes())])
    mv = memoryview(buf.getvalue())
    p = GGUFParser(mv)
    assert bytes(mv[:4]) == gguf.GGUF_MAGIC
    t = p.tensors["blk.0.attn_norm.weight"]
    assert np.array_equal(np.frombuffer(mv, np.float16, 32, t.abs_offset), np.arange(32, dtype=np.float16))
    mv.release()


def test_resident_weights_rejects_unsupported_types(tmp_path):
    import resident

    path = tmp_path / "q2k.gguf"
    with open(path, "wb") as f:
        write_synthetic_gguf(f, {}, [("blk.0.attn_q.weight", (256,), GGMLType.Q2_K, bytes(84))])
    with pytest.raises(ValueError) as e:
        resident.ResidentWeights(str(path))
    assert "Q2_K" in str(e.value) and "Supported types: F16, F32, Q4_0, Q4_K, Q6_K, Q8_0." in str(e.value)
    with pytest.raises(ValueError):  # truncated files fail at parse time
        with open(path, "rb") as f:
            data = f.read()
        with open(path, "wb") as f:
            f.write(data[:-8])
        resident.parse_file(str(path))


def test_read_file_ranges_matches_file_bytes(tmp_path):
    import resident

    rng = np.random.default_rng(7)
    data = rng.integers(0, 256, 11 << 20, dtype=np.uint8)  # 11 MiB: ranges span several 4 MiB pieces
    path = tmp_path / "blob.bin"
    data.tofile(path)
    specs = [(0, 100), (123, 9 << 20), (len(data) - 5, 5), (4 << 20, 0), (777, 1)] + \
            [(int(o), int(n)) for o, n in zip(rng.integers(0, len(data) - 70000, 40), rng.integers(1, 70000, 40))]
    bufs = [np.empty(n, np.uint8) for _, n in specs]
    resident.read_ranges_to_host(str(path), [(o, b) for (o, _), b in zip(specs, bufs)], threads=5)
    for (o, n), b in zip(specs, bufs):
        assert np.array_equal(b, data[o:o + n]), (o, n)


def test_read_file_errors(tmp_path):
    import resident

    path = tmp_path / "small.bin"
    np.arange(1000, dtype=np.uint8).tofile(path)
    with pytest.raises(ValueError):
        resident.read_ranges_to_host(str(path), [(990, np.empty(20, np.uint8))])
    with pytest.raises(ValueError):
        resident.read_ranges_to_host(str(path), [(-1, np.empty(2, np.uint8))])
    with pytest.raises(OSError):
        resident.read_ranges_to_host(str(tmp_path / "missing.bin"), [(0, np.empty(2, np.uint8))])
    b = np.empty(10, np.uint8)
    resident.read_ranges_to_host(str(path), [(990, b)])
    assert np.array_equal(b, np.arange(990, 1000) % 256)
