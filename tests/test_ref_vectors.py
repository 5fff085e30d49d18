"""The oracle against vectors produced by the reference's own CPU code (tests/golden/ref_vectors.npz,
written by tests/golden/make_ref_vectors.py from src/gguf_parser.py).

* quantize_*_cpu (src/gguf_parser.py:344-371, 387-405, 418-468, 505-557): the oracle's
  restatement must reproduce the reference's packed bytes exactly on N(0,1)-scaled rows and on
  special blocks (zeros, constant, all-negative, spike, near fp16 max, subnormal scale);
* dequantize_*_cpu (src/gguf_parser.py:374-384, 408-415, 471-502, 560-589): the oracle's fp16
  output must be bit-identical on random blocks (finite fp16 fields incl. 0, 2^-20, 1, 65504)
  and on the quantizer outputs above.
"""

import os

import numpy as np
import pytest

import gguf_oracle as O

REF = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_vectors.npz")
NAMES = ["q4_0", "q8_0", "q4_k", "q6_k"]


@pytest.fixture(scope="module")
def ref():
    return np.load(REF, allow_pickle=False)


@pytest.mark.parametrize("name", NAMES)
def test_quantizer_bytes_match_reference(ref, name):
    t = O.TYPE_BY_NAME[name]
    x = ref[f"{name}_quant_in"]
    with np.errstate(all="ignore"):
        got = O.QUANTIZE[t](x)
    np.testing.assert_array_equal(np.asarray(got, dtype=np.uint8), ref[f"{name}_quant_out"])


@pytest.mark.parametrize("name", NAMES)
@pytest.mark.parametrize("which", ["deq", "quant"])
def test_dequantizer_bits_match_reference(ref, name, which):
    t = O.TYPE_BY_NAME[name]
    if which == "deq":
        raw, want = ref[f"{name}_deq_in"], ref[f"{name}_deq_out"]
    else:
        raw, want = ref[f"{name}_quant_out"], ref[f"{name}_quant_deq"]
    with np.errstate(all="ignore"):
        got = O.dequantize_f16(t, raw, want.size)
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


def test_vectors_cover_special_fields(ref):
    # the random-block inputs carry zero, subnormal, one and fp16-max scales
    d = ref["q4_0_deq_in"].reshape(-1, 18)[:4, :2].copy().view(np.float16).ravel()
    np.testing.assert_array_equal(d, np.array([0.0, 2.0 ** -20, 1.0, 65504.0], dtype=np.float16))
