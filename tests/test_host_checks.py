"""Host-side argument checks of the Python device API (CPU; nothing here launches a kernel).

Every device entry point must reject, before its C call, a tensor that is not on the GPU, on
another device, or smaller than the bytes the kernels will touch: a host pointer or an
undersized buffer handed to a kernel is an out-of-bounds device access, not an error.  The
layer checks follow the reference's forward_layer_cached, which rejects undersized buffers
(src/python_bindings/bindings.cpp:562-627).
"""

import numpy as np
import pytest
import torch

import qmm
import layer
from gguf import GGMLType, GGUFTensorInfo


def test_gemm_rejects_host_tensors():
    A = torch.zeros((1, 256))
    W = torch.zeros(qmm.weight_bytes(qmm.GGML_Q4_K, 4, 256), dtype=torch.uint8)
    with pytest.raises(ValueError, match="device tensor"):
        qmm.gemm(qmm.GGML_Q4_K, A, W, 4, 256)


def test_dequantize_rejects_host_and_undersized():
    W = torch.zeros(144, dtype=torch.uint8)
    with pytest.raises(ValueError, match="device tensor"):
        qmm.dequantize(qmm.GGML_Q4_K, W, 256)


CFG = layer.LlamaLayerConfig(hidden_size=256, intermediate_size=512, num_heads=8, num_kv_heads=2, head_dim=32)


def _block(cfg=CFG, override=None):
    """{name: (info, view)} of one block on the host; `override` maps a tensor name to
    (dims, n_bytes) to plant a mismatch."""
    dims = layer.projection_dims(cfg)
    out = {}
    for name in ("attn_norm", "ffn_norm"):
        n = cfg.hidden_size if not override or name not in override else override[name]
        info = GGUFTensorInfo(f"blk.0.{name}.weight", (n,), GGMLType.F32, 0, 0, n, 4 * n)
        out[info.name] = (info, torch.ones(n))
    for name, (N, K) in dims.items():
        t = GGMLType.Q6_K if name == "ffn_down" else GGMLType.Q4_K
        d, nb = (K, N), qmm.weight_bytes(int(t), N, K)
        if override and name in override:
            d, nb = override[name]
        info = GGUFTensorInfo(f"blk.0.{name}.weight", d, t, 0, 0, d[0] * d[1], nb)
        out[info.name] = (info, torch.zeros(nb, dtype=torch.uint8))
    return out


def test_layer_struct_accepts_matching_block():
    w = layer.layer_weights_struct(_block(), "blk.0.", CFG, torch.device("cpu"))
    assert w.wq_type == int(GGMLType.Q4_K) and w.wdown_type == int(GGMLType.Q6_K)


@pytest.mark.parametrize("name,override,match", [
    ("attn_k", ((256, 128), qmm.weight_bytes(12, 128, 256)), "GGUF dims"),          # 2 KV heads x 32 = 64 rows
    ("ffn_down", ((512, 256), qmm.weight_bytes(14, 256, 512) - 1), "need"),         # one byte short
    ("attn_q", ((256, 256), 100), "need"),
    ("ffn_norm", 255, "hidden_size"),
])
def test_layer_struct_rejects_mismatch(name, override, match):
    with pytest.raises(ValueError, match=match):
        layer.layer_weights_struct(_block(override={name: override}), "blk.0.", CFG, torch.device("cpu"))


def test_layer_struct_rejects_other_device_and_strided_views():
    with pytest.raises(ValueError, match="on cpu"):
        layer.layer_weights_struct(_block(), "blk.0.", CFG, torch.device("cuda:0"))
    blk = _block()
    info, view = blk["blk.0.attn_v.weight"]
    blk["blk.0.attn_v.weight"] = (info, torch.zeros(2 * view.numel(), dtype=torch.uint8)[::2])
    with pytest.raises(ValueError, match="contiguous"):
        layer.layer_weights_struct(blk, "blk.0.", CFG, torch.device("cpu"))


class _FakeCache:
    pass


def test_forward_rejects_host_hidden_states():
    tl = layer.TransformerLayer(CFG)
    x = torch.zeros((2, 256), dtype=torch.float16)
    with pytest.raises(ValueError, match="hidden_states"):
        tl.forward_with_weights(x, _block(), 0, 0, _FakeCache())
