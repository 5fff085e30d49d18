"""CPU tests of the drop-in pybind11 ``matmul_module``: names, argument names and the
argument guards of the reference binding (src/python_bindings/bindings.cpp:20-51, 100-322,
653-728; guard cases from tests/test_phase5_scale.py:382-418).  Every case raises before the
library touches a GPU."""

import numpy as np
import pytest

import matmul_module

REF_ARGS = {
    "dequantize_q4_0": ["q4_buf", "out_fp16", "num_elements"],
    "dequantize_q8_0": ["q8_buf", "out_fp16", "num_elements"],
    "dequantize_q4_k": ["q4k_buf", "out_fp16", "num_elements"],
    "dequantize_q6_k": ["q6k_buf", "out_fp16", "num_elements"],
    "matmul_q4_0": ["A", "B_q4", "C", "M", "N", "K"],
    "matmul_q8_0": ["A", "B_q8", "C", "M", "N", "K"],
    "matmul_q4_k": ["A", "B_q4k", "C", "M", "N", "K"],
    "matmul_q6_k": ["A", "B_q6k", "C", "M", "N", "K"],
    "matmul": ["A", "B", "C", "M", "N", "K"],
    "matmul_nt": ["A", "B_nt", "C", "M", "N", "K"],
    "rmsnorm": ["x", "weight", "out", "M", "K", "eps"],
    "rmsnorm_residual": ["x", "residual", "weight", "h_out", "norm_out", "M", "K", "eps"],
    "residual_add": ["x", "residual", "out", "num_elements"],
    "rope": ["x_in", "x_out", "seq_len", "num_heads", "head_dim", "pos_offset", "freq_base", "neox_style"],
    "gqa_attention": ["Q", "K", "V", "Out", "q_len", "kv_len", "num_heads", "num_kv_heads", "head_dim", "start_pos",
                      "scale", "causal"],
    "swiglu": ["gate", "up", "out", "num_elements"],
    "kv_cache_init": ["num_layers", "max_seq_len", "num_kv_heads", "head_dim"],
    "gqa_attention_cached": ["Q", "K_new", "V_new", "Out", "layer_idx", "q_len", "start_pos", "num_heads",
                             "num_kv_heads", "head_dim", "scale", "causal"],
    "forward_layer_cached": ["x_in", "x_out", "attn_norm_w", "wq", "wq_type", "wk", "wk_type", "wv", "wv_type", "wo",
                             "wo_type", "ffn_norm_w", "wgate", "wgate_type", "wup", "wup_type", "wdown", "wdown_type",
                             "layer_idx", "seq_len", "pos_offset", "hidden_size", "intermediate_size", "num_heads",
                             "num_kv_heads", "head_dim", "rms_norm_eps", "rope_freq_base", "rope_neox", "scale"],
}

# Defaults of the reference's m.def (bindings.cpp:738-831).
REF_DEFAULTS = {
    "rmsnorm": [("eps", "9.999999747378752e-06")],
    "rope": [("pos_offset", "0"), ("freq_base", "10000.0"), ("neox_style", "False")],
    "gqa_attention": [("start_pos", "0"), ("scale", "0.0"), ("causal", "True")],
    "gqa_attention_cached": [("scale", "0.0"), ("causal", "True")],
}


@pytest.mark.parametrize("name,args", sorted(REF_ARGS.items()))
def test_entry_points_and_arg_names(name, args):
    fn = getattr(matmul_module, name)
    sig = fn.__doc__.splitlines()[0]
    for a in args:
        assert f"{a}:" in sig, (name, a, sig)


@pytest.mark.parametrize("name,defaults", sorted(REF_DEFAULTS.items()))
def test_defaults(name, defaults):
    import re

    sig = getattr(matmul_module, name).__doc__.splitlines()[0]
    for arg, value in defaults:
        assert re.search(rf"\b{arg}: [^,=]* = {re.escape(value)}[,)]", sig), (name, arg, sig)


def test_kv_cache_free_exists():
    assert callable(matmul_module.kv_cache_free)


def test_module_loaded_from_tree():
    import os

    assert os.path.dirname(matmul_module.__file__).endswith("gfx1150-inference_amd")


a_ok = np.zeros((2, 32), dtype=np.float16)
c_ok = np.zeros((2, 4), dtype=np.float16)


def test_int16_activation_rejected():
    with pytest.raises(ValueError, match="FP16"):
        matmul_module.matmul_q4_0(np.zeros((2, 32), dtype=np.int16), np.zeros(4 * 18, np.uint8), c_ok, 2, 4, 32)


def test_float32_activation_rejected():
    with pytest.raises(ValueError):
        matmul_module.matmul_q8_0(np.zeros((2, 32), dtype=np.float32), np.zeros(4 * 34, np.uint8), c_ok, 2, 4, 32)


def test_read_only_output_rejected():
    c_ro = np.zeros((2, 4), dtype=np.float16)
    c_ro.setflags(write=False)
    with pytest.raises(ValueError, match="writeable"):
        matmul_module.matmul_q4_0(a_ok, np.zeros(4 * 18, np.uint8), c_ro, 2, 4, 32)


def test_strided_quant_buffer_rejected():
    q4_strided = np.zeros((4, 36), dtype=np.uint8)[:, ::2]
    with pytest.raises(ValueError, match="C-contiguous"):
        matmul_module.matmul_q4_0(a_ok, q4_strided, c_ok, 2, 4, 32)


def test_non_contiguous_activation_rejected():
    a = np.zeros((2, 64), dtype=np.float16)[:, ::2]
    with pytest.raises(ValueError, match="C-contiguous"):
        matmul_module.matmul_q4_0(a, np.zeros(4 * 18, np.uint8), c_ok, 2, 4, 32)


def test_short_buffers_rejected():
    with pytest.raises(ValueError, match="smaller than required"):
        matmul_module.matmul_q4_k(np.zeros((1, 256), np.float16), np.zeros(143, np.uint8), np.zeros((1, 1), np.float16),
                                  1, 1, 256)
    with pytest.raises(ValueError, match="smaller than expected"):
        matmul_module.matmul_q6_k(np.zeros((1, 255), np.float16), np.zeros(210, np.uint8), np.zeros((1, 1), np.float16),
                                  1, 1, 256)
    with pytest.raises(ValueError, match="smaller than required"):
        matmul_module.dequantize_q8_0(np.zeros(33, np.uint8), np.zeros(32, np.float16), 32)


@pytest.mark.parametrize("fn,K", [(matmul_module.matmul_q4_0, 48), (matmul_module.matmul_q8_0, 0),
                                  (matmul_module.matmul_q4_k, 128), (matmul_module.matmul_q6_k, 300)])
def test_bad_k_rejected(fn, K):
    with pytest.raises(ValueError, match="K must be a positive multiple"):
        fn(np.zeros((1, 512), np.float16), np.zeros(4096, np.uint8), np.zeros((1, 8), np.float16), 1, 8, K)


@pytest.mark.parametrize("fn,n", [(matmul_module.dequantize_q4_0, 31), (matmul_module.dequantize_q4_k, 0),
                                  (matmul_module.dequantize_q6_k, 255), (matmul_module.dequantize_q8_0, -32)])
def test_bad_num_elements_rejected(fn, n):
    with pytest.raises(ValueError, match="num_elements must be a positive multiple"):
        fn(np.zeros(4096, np.uint8), np.zeros(512, np.float16), n)


def test_memoryview_and_mmap_style_buffers_accepted_by_guards():
    # A read-only uint8 memoryview (the reference's mmap views) passes the buffer guard; the
    # call then fails only on the undersized output check, before any device work.
    buf = memoryview(bytes(18 * 4))
    with pytest.raises(ValueError, match="out_fp16"):
        matmul_module.dequantize_q4_0(buf, np.zeros(64, np.float16), 128)


# ---- guards of the dense and layer entry points (bindings.cpp:53-98, 324-627): all raise before
# any device work

def test_matmul_nt_shape_guard():
    with pytest.raises(ValueError, match="B_nt must be a 2D array with shape"):
        matmul_module.matmul_nt(np.zeros((2, 8), np.float16), np.zeros(32, np.float16), np.zeros((2, 4), np.float16),
                                2, 4, 8)
    with pytest.raises(ValueError, match="B_nt must be a 2D array with shape"):
        matmul_module.matmul_nt(np.zeros((2, 8), np.float16), np.zeros((8, 4), np.float16),
                                np.zeros((2, 4), np.float16), 2, 4, 8)


def test_matmul_guards():
    with pytest.raises(ValueError, match="B buffer is smaller"):
        matmul_module.matmul(np.zeros((2, 8), np.float16), np.zeros((8, 3), np.float16), np.zeros((2, 4), np.float16),
                             2, 4, 8)
    with pytest.raises(ValueError, match="FP16"):
        matmul_module.matmul(np.zeros((2, 8), np.float32), np.zeros((8, 4), np.float16), np.zeros((2, 4), np.float16),
                             2, 4, 8)


def test_layer_op_guards():
    x = np.zeros((2, 8), np.float16)
    with pytest.raises(ValueError, match="weight buffer is smaller"):
        matmul_module.rmsnorm(x, np.zeros(7, np.float16), np.zeros_like(x), 2, 8)
    ro = np.zeros_like(x)
    ro.setflags(write=False)
    with pytest.raises(ValueError, match="h_out must be a writeable"):
        matmul_module.rmsnorm_residual(x, x, np.zeros(8, np.float16), ro, np.zeros_like(x), 2, 8)
    with pytest.raises(ValueError, match="residual must be a 2-byte FP16"):
        matmul_module.residual_add(x, np.zeros((2, 8), np.float32), np.zeros_like(x), 16)
    with pytest.raises(ValueError, match="x_in buffer is smaller"):
        matmul_module.rope(x, np.zeros_like(x), 2, 2, 8)
    with pytest.raises(ValueError, match="up must be a C-contiguous"):
        matmul_module.swiglu(x, np.zeros((8, 4), np.float16).T, np.zeros_like(x), 16)
    with pytest.raises(ValueError, match="K buffer is smaller"):
        matmul_module.gqa_attention(x, np.zeros(3, np.float16), x, np.zeros_like(x), 1, 1, 2, 1, 8)


def test_kv_cache_init_rejects_bad_dimensions():
    with pytest.raises(ValueError, match="KV cache dimensions must all be positive"):
        matmul_module.kv_cache_init(0, 16, 2, 64)


def test_forward_layer_cached_weight_guards():
    hid, inter, H, KVH, D = 256, 512, 4, 2, 64
    x = np.zeros((1, hid), np.float16)
    norm = np.ones(hid, np.float16)
    q4k = lambda n, k: np.zeros(n * (k // 256) * 144, np.uint8)  # noqa: E731
    args = dict(x_in=x, x_out=np.zeros_like(x), attn_norm_w=norm, wq=q4k(H * D, hid), wq_type=12,
                wk=q4k(KVH * D, hid), wk_type=12, wv=q4k(KVH * D, hid), wv_type=12, wo=q4k(hid, H * D), wo_type=12,
                ffn_norm_w=norm, wgate=q4k(inter, hid), wgate_type=12, wup=q4k(inter, hid), wup_type=12,
                wdown=q4k(hid, inter), wdown_type=12, layer_idx=0, seq_len=1, pos_offset=0, hidden_size=hid,
                intermediate_size=inter, num_heads=H, num_kv_heads=KVH, head_dim=D, rms_norm_eps=1e-5,
                rope_freq_base=10000.0, rope_neox=False, scale=0.0)
    with pytest.raises(ValueError, match="wo weight buffer is smaller than required"):
        matmul_module.forward_layer_cached(**{**args, "wo": q4k(hid, H * D)[:-1]})
    with pytest.raises(ValueError, match="wgate has unsupported ggml_type"):
        matmul_module.forward_layer_cached(**{**args, "wgate_type": 3})
    with pytest.raises(ValueError, match="wdown K must be divisible by 256 for Q4_K"):
        matmul_module.forward_layer_cached(**{**args, "intermediate_size": 300, "wgate": q4k(300, hid),
                                              "wup": q4k(300, hid)})
    with pytest.raises(ValueError, match="ffn_norm_w buffer is smaller"):
        matmul_module.forward_layer_cached(**{**args, "ffn_norm_w": norm[:-1]})
