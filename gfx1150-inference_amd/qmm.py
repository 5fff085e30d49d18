"""Host-side Python interface to ``libqmm_gfx950.so`` for device-resident buffers.

This is the device-pointer counterpart of the drop-in ``matmul_module`` (which keeps the
reference's host-array API).  Every call goes through the C ABI declared in
``include/qmm.h``; PyTorch is used only to own device memory and to supply the current
HIP stream.  There is no CPU fallback: if the library is missing, importing this module
raises ``ImportError``.

Weight type ids are the GGMLType integers of the reference (``src/gguf_parser.py:22-36``);
device launchers mirror ``launch_matmul_q*_device`` (``src/kernels/dequantize.h:98-132``)
and raise ``ValueError`` / ``RuntimeError`` where the reference throws
``std::invalid_argument`` / ``std::runtime_error``.
"""

from __future__ import annotations

import ctypes
import os
import re
from typing import Optional

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
_REPO_DIR = os.path.dirname(_PKG_DIR)
LIB_PATH = os.path.join(_PKG_DIR, "libqmm_gfx950.so")
HEADER_PATH = os.path.join(_REPO_DIR, "include", "qmm.h")

GGML_F32 = 0   # token-embedding tables only
GGML_F16 = 1   # dense fp16 rows: GEMM weights (matmul_nt) and token-embedding tables
GGML_Q4_0 = 2
GGML_Q8_0 = 8
GGML_Q4_K = 12
GGML_Q6_K = 14

# (block_elems, block_bytes) of every supported type (src/kernels/dequantize.h:6-22).
BLOCK_INFO = {GGML_Q4_0: (32, 18), GGML_Q8_0: (32, 34), GGML_Q4_K: (256, 144), GGML_Q6_K: (256, 210)}

QMM_OK = 0
QMM_ERR_INVALID_ARGUMENT = 1
QMM_ERR_UNSUPPORTED = 2
QMM_ERR_HIP = 3
QMM_ERR_IO = 4
QMM_ERR_OUT_OF_RANGE = 5

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is not built; run `python gfx1150-inference_amd/build_ext.py` "
        "(or __graft_entry__.build()) first. There is no CPU fallback.")

# In a process that also uses PyTorch, torch must load its HIP runtime first: the library's
# libamdhip64.so.7 dependency then binds to that already-loaded runtime instead of bringing a
# second HIP/HSA runtime into the process.
try:
    import torch  # noqa: F401
except ImportError:
    pass

_lib = ctypes.CDLL(LIB_PATH)

_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64


class FileRange(ctypes.Structure):
    """Mirror of qmm_file_range (include/qmm.h)."""

    _fields_ = [("offset", _i64), ("bytes", _i64), ("dst", _vp)]


class LayerConfig(ctypes.Structure):
    """Mirror of qmm_layer_config (include/qmm.h)."""

    _fields_ = [("hidden_size", _i), ("intermediate_size", _i), ("num_heads", _i), ("num_kv_heads", _i),
                ("head_dim", _i), ("rms_norm_eps", ctypes.c_float), ("rope_freq_base", ctypes.c_float),
                ("rope_neox", _i), ("scale", ctypes.c_float)]


class LayerWeights(ctypes.Structure):
    """Mirror of qmm_layer_weights (include/qmm.h)."""

    _fields_ = [("attn_norm", _vp), ("attn_norm_dtype", _i), ("wq", _vp), ("wq_type", _i), ("wk", _vp), ("wk_type", _i),
                ("wv", _vp), ("wv_type", _i), ("wo", _vp), ("wo_type", _i), ("ffn_norm", _vp), ("ffn_norm_dtype", _i),
                ("wgate", _vp), ("wgate_type", _i), ("wup", _vp), ("wup_type", _i), ("wdown", _vp), ("wdown_type", _i),
                ("bq", _vp), ("bk", _vp), ("bv", _vp), ("bo", _vp)]


class GemmDesc(ctypes.Structure):
    """Mirror of qmm_gemm_desc (include/qmm.h)."""

    _fields_ = [("ggml_type", _i), ("A", _vp), ("a_dtype", _i), ("W", _vp), ("C", _vp), ("c_dtype", _i),
                ("M", _i), ("N", _i), ("K", _i), ("ev_before", _vp), ("ev_after", _vp)]

_SIGNATURES = {
    "qmm_last_error": (ctypes.c_char_p, []),
    "qmm_version": (_i, []),
    "qmm_gemv_max_m": (_i, []),
    "qmm_set_gemv_max_m": (_i, [_i]),
    "qmm_set_thread_gemv_max_m": (_i, [_i]),
    "qmm_set_row_identity": (_i, [_i]),
    "qmm_row_identity": (_i, []),
    "qmm_weight_bytes": (ctypes.c_size_t, [_i, _i64, _i64]),
    "qmm_gemm": (_i, [_i, _vp, _i, _vp, _vp, _i, _i, _i, _i, _vp]),
    "qmm_gemm_noalloc": (_i, [_i, _vp, _i, _vp, _vp, _i, _i, _i, _i, _vp]),
    "qmm_noalloc_scratch_bytes": (ctypes.c_size_t, []),
    "qmm_dequantize": (_i, [_i, _vp, _vp, _i, _i64, _vp]),
    "qmm_embed": (_i, [_i, _vp, _i64, _i, _vp, _i64, _vp, _i, _vp, _vp]),
    "qmm_gemm_batch": (_i, [ctypes.POINTER(GemmDesc), _i, _vp]),
    "qmm_release_workspace": (_i, []),
    "qmm_upload_file": (_i, [ctypes.c_char_p, ctypes.POINTER(FileRange), _i, _i64, _i, _i, _vp]),
    "qmm_read_file": (_i, [ctypes.c_char_p, ctypes.POINTER(FileRange), _i, _i]),
    "qmm_rmsnorm": (_i, [_vp, _vp, _i, _vp, _i, _i, ctypes.c_float, _vp]),
    "qmm_rmsnorm_residual": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _i, _i, ctypes.c_float, _vp]),
    "qmm_residual_add": (_i, [_vp, _vp, _vp, _i64, _vp]),
    "qmm_swiglu": (_i, [_vp, _vp, _vp, _i64, _vp]),
    "qmm_rope": (_i, [_vp, _vp, _i, _i, _i, _i, ctypes.c_float, _i, _vp]),
    "qmm_gqa_attention": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, ctypes.c_float, _i, _vp]),
    "qmm_kv_cache_init": (_i, [_i, _i, _i, _i]),
    "qmm_kv_cache_free": (_i, []),
    "qmm_gqa_attention_cached": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, ctypes.c_float, _i, _vp]),
    "qmm_forward_layer": (_i, [ctypes.POINTER(LayerConfig), ctypes.POINTER(LayerWeights), _vp, _vp, _i, _i, _i, _vp]),
    "qmm_matmul_fp16_nt_device": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "qmm_matmul_fp16_nt_host": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "qmm_matmul_fp16_host": (_i, [_vp, _vp, _vp, _i, _i, _i]),
    "qmm_rmsnorm_host": (_i, [_vp, _vp, _vp, _i, _i, ctypes.c_float]),
    "qmm_rmsnorm_residual_host": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, ctypes.c_float]),
    "qmm_residual_add_host": (_i, [_vp, _vp, _vp, _i64]),
    "qmm_swiglu_host": (_i, [_vp, _vp, _vp, _i64]),
    "qmm_rope_host": (_i, [_vp, _vp, _i, _i, _i, _i, ctypes.c_float, _i]),
    "qmm_gqa_attention_host": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, ctypes.c_float, _i]),
    "qmm_gqa_attention_cached_host": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, ctypes.c_float, _i]),
    "qmm_forward_layer_host": (_i, [ctypes.POINTER(LayerConfig), ctypes.POINTER(LayerWeights), _vp, _vp, _i, _i, _i]),
}
for _t in ("q4_0", "q8_0", "q4_k", "q6_k"):
    _SIGNATURES[f"qmm_matmul_{_t}_device"] = (_i, [_vp, _vp, _vp, _i, _i, _i, _vp])
    _SIGNATURES[f"qmm_matmul_{_t}_host"] = (_i, [_vp, _vp, _vp, _i, _i, _i])
    _SIGNATURES[f"qmm_dequantize_{_t}_host"] = (_i, [_vp, _vp, _i])

for _name, (_res, _args) in _SIGNATURES.items():
    _fn = getattr(_lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


def lib() -> ctypes.CDLL:
    return _lib


def header_symbols() -> list:
    """Function names declared in include/qmm.h (used to check the exported ABI)."""
    text = open(HEADER_PATH).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+char\s*\*|int|size_t)\s+(qmm_\w+)\s*\(", text, re.M)))


def last_error() -> str:
    return _lib.qmm_last_error().decode()


def check(rc: int) -> None:
    if rc == QMM_OK:
        return
    msg = last_error()
    if rc == QMM_ERR_INVALID_ARGUMENT:
        raise ValueError(msg)
    if rc == QMM_ERR_IO:
        raise OSError(msg)
    if rc == QMM_ERR_OUT_OF_RANGE:
        raise IndexError(msg)
    raise RuntimeError(msg)


def weight_bytes(ggml_type: int, n: int, k: int) -> int:
    return int(_lib.qmm_weight_bytes(ggml_type, n, k))


def gemv_max_m() -> int:
    return int(_lib.qmm_gemv_max_m())


def set_gemv_max_m(m: int) -> None:
    """Moves the GEMV / prefill threshold for the process: M < m runs the GEMV kernels; the
    default is 17."""
    check(_lib.qmm_set_gemv_max_m(int(m)))


def set_thread_gemv_max_m(m: int) -> None:
    """The calling thread's GEMV / prefill threshold (0: the process value again)."""
    check(_lib.qmm_set_thread_gemv_max_m(int(m)))


def row_identity() -> bool:
    return bool(_lib.qmm_row_identity())


def set_row_identity(on: bool) -> None:
    """Calling thread's row-identity mode: when on, every GEMV-size M of a format runs one kernel
    family (Q4_K the matrix-core GEMV, the other formats v_dot2), so that row m of any
    M < gemv_max_m() is bit-identical to the M = 1 call (the reference's invariant); when off (the
    default), each M takes the faster family (Q4_K matrix-core from M = 2, Q6_K from M = 3)."""
    check(_lib.qmm_set_row_identity(1 if on else 0))


class row_identity_mode:
    """Context manager: row-identity mode on (or off) for the calling thread, restored on exit."""

    def __init__(self, on: bool = True):
        self._on = bool(on)
        self._prev = False

    def __enter__(self):
        self._prev = row_identity()
        set_row_identity(self._on)
        return self

    def __exit__(self, *exc):
        set_row_identity(self._prev)
        return False


def _torch():
    import torch
    return torch


def _stream_handle(stream=None) -> Optional[int]:
    torch = _torch()
    s = torch.cuda.current_stream() if stream is None else stream
    return s.cuda_stream


def _dtype_code(t) -> int:
    torch = _torch()
    if t == torch.float32:
        return DTYPE_F32
    if t == torch.float16:
        return DTYPE_F16
    if t == torch.bfloat16:
        return DTYPE_BF16
    raise ValueError(f"unsupported dtype {t}")


def gemm(ggml_type: int, A, W, N: int, K: int, out=None, out_dtype=None, stream=None):
    """C[M, N] = A[M, K] @ dequant(W)[N, K]^T on the GPU (device tensors, asynchronous).
    W holds packed GGUF blocks (uint8), or fp16 values [N, K] for GGML_F16 (the matmul_nt
    operand)."""
    torch = _torch()
    if not A.is_cuda or A.dim() != 2 or A.shape[1] != K or not A.is_contiguous():
        raise ValueError("A must be a contiguous [M, K] device tensor")
    if not W.is_cuda or W.device != A.device:
        raise ValueError("W must be a device tensor on A's device")
    dense = ggml_type == GGML_F16
    if not W.is_contiguous() or W.dtype not in ((torch.uint8, torch.float16) if dense else (torch.uint8,)):
        raise ValueError("W must be a contiguous uint8 device tensor (or float16 for GGML_F16)")
    if W.numel() * W.element_size() < weight_bytes(ggml_type, N, K):
        raise ValueError("W is smaller than N * (K / block) * block_bytes")
    M = A.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype or torch.float32, device=A.device)
    elif out.shape != (M, N) or not out.is_contiguous() or out.device != A.device:
        raise ValueError("out must be a contiguous [M, N] device tensor on A's device")
    check(_lib.qmm_gemm(ggml_type, A.data_ptr(), _dtype_code(A.dtype), W.data_ptr(), out.data_ptr(),
                        _dtype_code(out.dtype), M, N, K, _stream_handle(stream)))
    return out


def gemm_batch(descs, stream=None) -> None:
    """Launch a ctypes array of GemmDesc back to back on `stream` (one C call)."""
    check(_lib.qmm_gemm_batch(descs, len(descs), _stream_handle(stream)))


def dequantize(ggml_type: int, W, num_elements: int, out=None, out_dtype=None, stream=None):
    """dequant(W) -> [num_elements] device tensor (fp16 / bf16 / fp32), bit-exact."""
    torch = _torch()
    if not W.is_cuda or not W.is_contiguous():
        raise ValueError("W must be a contiguous device tensor")
    if num_elements < 0:
        raise ValueError("num_elements must be non-negative")
    qk = BLOCK_INFO[ggml_type][0] if ggml_type in BLOCK_INFO else 1
    if num_elements % qk == 0 and W.numel() * W.element_size() < weight_bytes(ggml_type, 1, num_elements):
        raise ValueError("W is smaller than (num_elements / block) * block_bytes")
    if out is None:
        out = torch.empty((num_elements,), dtype=out_dtype or torch.float16, device=W.device)
    elif not out.is_cuda or out.device != W.device or not out.is_contiguous() or out.numel() < num_elements:
        raise ValueError("out must be a contiguous device tensor on W's device with at least num_elements values")
    check(_lib.qmm_dequantize(ggml_type, W.data_ptr(), out.data_ptr(), _dtype_code(out.dtype),
                              num_elements, _stream_handle(stream)))
    return out


def _row_bytes(ggml_type: int, hidden: int) -> int:
    if ggml_type == GGML_F32:
        return 4 * hidden
    if ggml_type == GGML_F16:
        return 2 * hidden
    qk, bb = BLOCK_INFO[ggml_type]
    return (hidden // qk) * bb


def embed_tokens(token_ids, ggml_type: int, table, hidden_size: int, out_dtype=None, stream=None):
    """Token embeddings ``(len(token_ids), hidden_size)`` (fp16 by default) from the token table,
    gathered and dequantized on the GPU.

    Mirrors the reference's ``embed_tokens(token_ids, embd_info, embd_view, hidden_size)``
    (src/tokenizer.py:336-389): the same result dtype and values (bit-exact with its CPU
    dequantizers), an empty ``(0, hidden_size)`` result for no ids, and the same ``ValueError``
    for an unsupported table type or an id outside the table (checked on the host before any GPU
    work, like the reference).  ``table`` is the packed ``token_embd.weight`` as a device tensor:
    uint8 bytes for Q4_0 / Q8_0 / Q4_K / Q6_K, or float16 / float32 values for F16 / F32.
    """
    import numpy as np
    torch = _torch()
    ids = np.asarray(token_ids, dtype=np.int64).reshape(-1)
    dt = out_dtype or torch.float16
    if ids.size == 0:
        return torch.empty((0, hidden_size), dtype=dt, device=table.device)
    if ggml_type not in (GGML_F32, GGML_F16) and ggml_type not in BLOCK_INFO:
        raise ValueError(f"Unsupported token_embd.weight type: {ggml_type}")
    row_bytes = _row_bytes(ggml_type, hidden_size)
    n_rows = (table.numel() * table.element_size()) // row_bytes
    bad = (ids < 0) | (ids >= n_rows)
    if bad.any():
        raise ValueError(f"Token ID {int(ids[bad][0])} is out of range for embedding table with {n_rows} rows")
    dev_ids = torch.from_numpy(ids).to(table.device)  # copied on the current stream
    out = torch.empty((ids.size, hidden_size), dtype=dt, device=table.device)
    if stream is not None:
        # the kernel on `stream` must see the copied ids, and the ids must outlive it there
        stream.wait_stream(torch.cuda.current_stream(table.device))
        dev_ids.record_stream(stream)
        out.record_stream(stream)
    check(_lib.qmm_embed(ggml_type, table.data_ptr(), n_rows, hidden_size, dev_ids.data_ptr(), ids.size,
                         out.data_ptr(), _dtype_code(dt), None, _stream_handle(stream)))
    return out


def _device_launcher(name):
    fn = getattr(_lib, name)

    def launch(d_A_fp16, d_B, d_C_fp16, M: int, N: int, K: int, stream=None) -> None:
        check(fn(d_A_fp16.data_ptr(), d_B.data_ptr(), d_C_fp16.data_ptr(), M, N, K, _stream_handle(stream)))

    launch.__name__ = name
    launch.__doc__ = (f"{name}: fp16 A [M,K], packed B [N,K], fp16 C [M,N] device tensors "
                      "(launch_matmul_*_device of src/kernels/dequantize.h:98-132).")
    return launch


matmul_q4_0_device = _device_launcher("qmm_matmul_q4_0_device")
matmul_q8_0_device = _device_launcher("qmm_matmul_q8_0_device")
matmul_q4_k_device = _device_launcher("qmm_matmul_q4_k_device")
matmul_q6_k_device = _device_launcher("qmm_matmul_q6_k_device")
