"""GPU parity of the token-embedding gather-dequant (qmm_embed / qmm.embed_tokens) against the
oracle's restatement of the reference's embed_tokens (src/tokenizer.py:336-389: gather rows of
token_embd.weight, dequantize with dequantize_*_cpu to fp16).

Bars: bit-exact fp16 output for every table type (quantized types through the oracle's
dequantize_f16, which tests/test_ref_vectors.py pins to the reference's own dequantizers; F32
tables rounded once RNE; F16 tables copied bit for bit); bit-exact fp32 / bf16 outputs against
the exact fp32 weights.
"""

import numpy as np
import pytest

import gguf_oracle as O

pytestmark = pytest.mark.gpu

QTYPES = [O.GGML_Q4_0, O.GGML_Q8_0, O.GGML_Q4_K, O.GGML_Q6_K]


@pytest.fixture(scope="module")
def dev(cuda):
    import qmm  # noqa: F401
    return cuda


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def gathered_raw(t, raw, hidden, ids):
    rb = O.weight_bytes(t, 1, hidden)
    rows = raw.reshape(-1, rb)
    return np.ascontiguousarray(rows[ids]).reshape(-1)


@pytest.mark.parametrize("t", QTYPES)
@pytest.mark.parametrize("hidden", [512, 4096])
def test_embed_quantized_fp16_bit_exact(dev, t, hidden):
    import torch
    import qmm
    rng = np.random.default_rng(7000 + t + hidden)
    n_rows = 300
    raw = O.synth_weights(t, n_rows, hidden, rng)
    ids = rng.integers(0, n_rows, size=37)
    ids[:3] = [0, n_rows - 1, 0]  # first, last, repeated
    out = qmm.embed_tokens(ids, t, to_dev(raw, dev), hidden)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16 and out.shape == (ids.size, hidden)
    ref = O.dequantize_f16(t, gathered_raw(t, raw, hidden, ids), ids.size * hidden).reshape(ids.size, hidden)
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("t", QTYPES)
def test_embed_quantized_fp32_and_bf16(dev, t):
    import torch
    import qmm
    rng = np.random.default_rng(7100 + t)
    n_rows, hidden = 64, 1024
    raw = O.synth_weights(t, n_rows, hidden, rng)
    ids = rng.integers(0, n_rows, size=20)
    f32 = O.DEQUANT_F32[t](gathered_raw(t, raw, hidden, ids), ids.size * hidden).reshape(ids.size, hidden)
    out32 = qmm.embed_tokens(ids, t, to_dev(raw, dev), hidden, out_dtype=torch.float32)
    outbf = qmm.embed_tokens(ids, t, to_dev(raw, dev), hidden, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out32.cpu().numpy().view(np.uint32), f32.view(np.uint32))
    np.testing.assert_array_equal(outbf.cpu().view(torch.int16).numpy().view(np.uint16), O.f32_to_bf16_bits(f32))


def test_embed_f32_table_rounds_once(dev):
    import torch
    import qmm
    rng = np.random.default_rng(7200)
    n_rows, hidden = 50, 256
    table = (rng.standard_normal((n_rows, hidden)) * 3).astype(np.float32)
    table[0, :4] = [65520.0, -1e-8, 1e-7, np.inf]  # overflow to inf, subnormal/zero results, inf
    ids = np.array([0, 5, 49, 5, 0])
    out = qmm.embed_tokens(ids, qmm.GGML_F32, to_dev(table, dev), hidden)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint16), table[ids].astype(np.float16).view(np.uint16))


def test_embed_f16_table_copies_bits(dev):
    import torch
    import qmm
    rng = np.random.default_rng(7300)
    n_rows, hidden = 40, 128
    bits = rng.integers(0, 1 << 16, size=(n_rows, hidden), dtype=np.uint16)  # includes NaN payloads
    table = to_dev(bits.view(np.float16), dev)
    ids = rng.integers(0, n_rows, size=9)
    out = qmm.embed_tokens(ids, qmm.GGML_F16, table, hidden)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint16), bits[ids])


def test_embed_device_ids_out_of_range_zero_fill_and_flag(dev):
    # Raw C ABI with device ids: ids outside [0, n_rows) read nothing out of bounds, their rows are
    # zero-filled and the flag is set; the valid rows are unaffected.
    import torch
    import qmm
    t = O.GGML_Q4_K
    rng = np.random.default_rng(7400)
    n_rows, hidden = 16, 512
    raw = O.synth_weights(t, n_rows, hidden, rng)
    ids = np.array([3, -1, 15, 16, 1 << 40, 0], dtype=np.int64)
    d_ids = to_dev(ids, dev)
    out = torch.full((ids.size, hidden), 7.0, device=dev, dtype=torch.float16)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    W = to_dev(raw, dev)
    qmm.check(qmm.lib().qmm_embed(t, W.data_ptr(), n_rows, hidden, d_ids.data_ptr(), ids.size, out.data_ptr(),
                                  qmm.DTYPE_F16, flag.data_ptr(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert int(flag.item()) == 1
    o = out.cpu().numpy()
    good = np.array([0, 2, 5])
    ref = O.dequantize_f16(t, gathered_raw(t, raw, hidden, ids[good]), good.size * hidden).reshape(good.size, hidden)
    np.testing.assert_array_equal(o[good].view(np.uint16), ref.view(np.uint16))
    assert np.all(o[[1, 3, 4]] == 0)
    # all ids valid: the flag stays clear
    flag.zero_()
    qmm.check(qmm.lib().qmm_embed(t, W.data_ptr(), n_rows, hidden, d_ids.data_ptr(), 1, out.data_ptr(),
                                  qmm.DTYPE_F16, flag.data_ptr(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert int(flag.item()) == 0


def test_embed_llama3_8b_vocab_slice(dev):
    # 8B hidden size on a 32000-row Q6_K table (the 128256-row table's layout, fewer rows).
    import torch
    import qmm
    t = O.GGML_Q6_K
    rng = np.random.default_rng(7500)
    n_rows, hidden = 32000, 4096
    raw = O.synth_weights(t, n_rows, hidden, rng)
    ids = rng.integers(0, n_rows, size=512)
    out = qmm.embed_tokens(ids, t, to_dev(raw, dev), hidden)
    torch.cuda.synchronize()
    sel = np.array([0, 1, 255, 511])
    ref = O.dequantize_f16(t, gathered_raw(t, raw, hidden, ids[sel]), sel.size * hidden).reshape(sel.size, hidden)
    np.testing.assert_array_equal(out.cpu().numpy()[sel].view(np.uint16), ref.view(np.uint16))
