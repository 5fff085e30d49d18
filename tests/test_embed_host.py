"""Host-side behaviour of qmm.embed_tokens (no GPU): the reference's validation
(src/tokenizer.py:327-389) happens before any device work."""

import numpy as np
import pytest
import torch

import qmm


def test_empty_ids_give_empty_fp16_result():
    table = torch.zeros(4 * 144, dtype=torch.uint8)  # 4 rows of one Q4_K super-block (hidden 256)
    out = qmm.embed_tokens([], qmm.GGML_Q4_K, table, 256)
    assert out.shape == (0, 256) and out.dtype == torch.float16


@pytest.mark.parametrize("bad", [-1, 4, 1000])
def test_out_of_range_id_raises_like_the_reference(bad):
    table = torch.zeros(4 * 144, dtype=torch.uint8)
    with pytest.raises(ValueError, match=f"Token ID {bad} is out of range for embedding table with 4 rows"):
        qmm.embed_tokens([0, 1, bad, 2], qmm.GGML_Q4_K, table, 256)


def test_first_bad_id_is_reported():
    table = torch.zeros(3 * 128, dtype=torch.float16)  # F16 table: 3 rows of hidden 128
    with pytest.raises(ValueError, match="Token ID 7 is out of range"):
        qmm.embed_tokens(np.array([0, 7, -3]), qmm.GGML_F16, table, 128)


def test_unsupported_type_raises():
    with pytest.raises(ValueError, match="Unsupported token_embd.weight type: 3"):
        qmm.embed_tokens([0], 3, torch.zeros(64, dtype=torch.uint8), 32)
