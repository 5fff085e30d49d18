"""One Llama transformer layer on device-resident weights.

Host-side mirror of the reference's `src/layer.py` (LlamaLayerConfig :58-110, TransformerLayer
:174-392) and of the GPU-resident branch of its KV cache manager (`src/kv_cache.py`,
KVCacheManager with mode "gpu"): the same configuration keys and defaults, the same layer
arithmetic, the same KV pool geometry.  The reference copies the hidden state and every weight
from the host for each layer call (forward_layer_cached -> launch_forward_layer_cached_fp16,
src/kernels/attention.hip:603-695); here weights are device tensors from
`resident.ResidentWeights`, activations are device fp16 tensors, and one `qmm_forward_layer`
call runs the whole layer on the stream with no host round trip.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import qmm
from gguf import GGMLType

_NEOX_ROPE_ARCHS = frozenset({"qwen2", "stablelm", "falcon", "gptneox", "phi2", "phi3", "starcoder2"})
_QUANTIZED = (GGMLType.Q4_0, GGMLType.Q8_0, GGMLType.Q4_K, GGMLType.Q6_K)


def _arch_meta(metadata: Dict[str, object], arch: str, suffix: str, default: object = None) -> object:
    """`{arch}.{suffix}`, else `llama.{suffix}`, else `default` (KeyError when none)."""
    for key in (f"{arch}.{suffix}", f"llama.{suffix}"):
        if key in metadata:
            return metadata[key]
    if default is not None:
        return default
    raise KeyError(f"Missing required GGUF metadata key '{arch}.{suffix}' (or 'llama.{suffix}')")


@dataclass(frozen=True)
class LlamaLayerConfig:
    hidden_size: int
    intermediate_size: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    rms_norm_eps: float = 1e-5
    rope_freq_base: float = 10000.0
    rope_neox: bool = False

    @classmethod
    def from_gguf_metadata(cls, metadata: Dict[str, object], rope_neox: Optional[bool] = None) -> "LlamaLayerConfig":
        arch = str(metadata.get("general.architecture", "llama")).lower()
        hidden = int(_arch_meta(metadata, arch, "embedding_length"))
        heads = int(_arch_meta(metadata, arch, "attention.head_count"))
        if rope_neox is None:
            if f"{arch}.rope.neox" in metadata:
                rope_neox = bool(metadata[f"{arch}.rope.neox"])
            elif "llama.rope.neox" in metadata:
                rope_neox = bool(metadata["llama.rope.neox"])
            else:
                rope_neox = arch in _NEOX_ROPE_ARCHS
        return cls(hidden_size=hidden,
                   intermediate_size=int(_arch_meta(metadata, arch, "feed_forward_length")),
                   num_heads=heads,
                   num_kv_heads=int(_arch_meta(metadata, arch, "attention.head_count_kv", heads)),
                   head_dim=int(_arch_meta(metadata, arch, "rope.dimension_count", hidden // heads)),
                   rms_norm_eps=float(_arch_meta(metadata, arch, "attention.layer_norm_rms_epsilon", 1e-5)),
                   rope_freq_base=float(_arch_meta(metadata, arch, "rope.freq_base", 10000.0)),
                   rope_neox=bool(rope_neox))


class DeviceKVCache:
    """The device KV pool: [num_layers][max_seq_len][num_kv_heads][head_dim] fp16 for K and V
    (qmm_kv_cache_init; one pool per device, as the reference's DeviceKVCachePool)."""

    def __init__(self, num_layers: int, max_seq_len: int, num_kv_heads: int, head_dim: int):
        qmm.check(qmm.lib().qmm_kv_cache_init(num_layers, max_seq_len, num_kv_heads, head_dim))
        self.num_layers, self.max_seq_len = num_layers, max_seq_len
        self.num_kv_heads, self.head_dim = num_kv_heads, head_dim
        self.mode = "gpu"
        self._open = True

    @property
    def nbytes(self) -> int:
        return 2 * self.num_layers * self.max_seq_len * self.num_kv_heads * self.head_dim * 2

    def close(self) -> None:
        if self._open:
            qmm.check(qmm.lib().qmm_kv_cache_free())
            self._open = False

    def __enter__(self) -> "DeviceKVCache":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


def _norm_arg(view) -> Tuple[int, int]:
    import torch

    if view.dtype == torch.float32:
        return view.data_ptr(), qmm.DTYPE_F32
    if view.dtype == torch.float16:
        return view.data_ptr(), qmm.DTYPE_F16
    raise ValueError(f"Unsupported norm weight dtype: {view.dtype}")


_PROJECTIONS = (("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"), ("wo", "attn_output"),
                ("wgate", "ffn_gate"), ("wup", "ffn_up"), ("wdown", "ffn_down"))


def projection_dims(config: LlamaLayerConfig) -> Dict[str, Tuple[int, int]]:
    """(N, K) of each projection: N output rows of K weights (GGUF dims are (K, N))."""
    h, f = config.hidden_size, config.intermediate_size
    q, kv = config.num_heads * config.head_dim, config.num_kv_heads * config.head_dim
    return {"attn_q": (q, h), "attn_k": (kv, h), "attn_v": (kv, h), "attn_output": (h, q),
            "ffn_gate": (f, h), "ffn_up": (f, h), "ffn_down": (h, f)}


def _nbytes(view) -> int:
    return view.numel() * view.element_size()


def layer_weights_struct(layer_weights: Dict[str, Tuple[object, object]], prefix: str,
                         config: Optional[LlamaLayerConfig] = None, device=None) -> "qmm.LayerWeights":
    """qmm_layer_weights from {name: (GGUFTensorInfo, device view)} of one block.

    With `config`, every tensor is checked against the layer's dimensions before its pointer is
    taken (the kernels read exactly N * (K / block) * block_bytes bytes of each projection and
    hidden_size values of each norm): GGUF dims (K, N), a contiguous view of at least that many
    bytes, and, with `device`, residence on that device.  A mismatch raises ValueError, as the
    reference's forward_layer_cached rejects undersized buffers (src/python_bindings/bindings.cpp
    :562-627)."""

    def on_device(name, view):
        if not view.is_contiguous():
            raise ValueError(f"{name}: weight view must be contiguous")
        if device is not None and view.device != device:
            raise ValueError(f"{name}: weight view is on {view.device}, the activations on {device}")

    w = qmm.LayerWeights()
    for field, name in (("attn_norm", "attn_norm"), ("ffn_norm", "ffn_norm")):
        view = layer_weights[f"{prefix}{name}.weight"][1]
        if config is not None:
            on_device(name, view)
            if view.numel() != config.hidden_size:
                raise ValueError(f"{name}.weight has {view.numel()} values, hidden_size is {config.hidden_size}")
        ptr, dt = _norm_arg(view)
        setattr(w, field, ptr)
        setattr(w, field + "_dtype", dt)
    dims = projection_dims(config) if config is not None else {}
    for field, name in _PROJECTIONS:
        info, view = layer_weights[f"{prefix}{name}.weight"]
        if info.ggml_type not in _QUANTIZED:
            raise ValueError(f"Unsupported weight quantization type: {info.ggml_type}")
        if config is not None:
            N, K = dims[name]
            on_device(name, view)
            if tuple(info.dims) != (K, N):
                raise ValueError(f"{name}.weight has GGUF dims {tuple(info.dims)}, the layer needs ({K}, {N})")
            need = qmm.weight_bytes(int(info.ggml_type), N, K)
            if _nbytes(view) < need:
                raise ValueError(f"{name}.weight view holds {_nbytes(view)} bytes, N={N} K={K} need {need}")
        setattr(w, field, view.data_ptr())
        setattr(w, field + "_type", int(info.ggml_type))
    # Optional projection biases (reference src/layer.py:274-282, 344-346), passed as fp16 vectors: an
    # F32 bias is rounded to fp16 first, as the reference's norm_weight_fp16 does (layer.py:161-167).
    # The converted copies are kept on the struct for the duration of the call.
    import torch

    keep = []
    for field, name, n in (("bq", "attn_q", None if config is None else config.num_heads * config.head_dim),
                           ("bk", "attn_k", None if config is None else config.num_kv_heads * config.head_dim),
                           ("bv", "attn_v", None if config is None else config.num_kv_heads * config.head_dim),
                           ("bo", "attn_output", None if config is None else config.hidden_size)):
        entry = layer_weights.get(f"{prefix}{name}.bias")
        if entry is None:
            continue
        view = entry[1]
        if view.dtype == torch.float32:
            view = view.to(torch.float16)
        elif view.dtype != torch.float16:
            raise ValueError(f"Unsupported bias dtype for {name}.bias: {view.dtype}")
        if config is not None:
            on_device(name + ".bias", view)
            if view.numel() != n:
                raise ValueError(f"{name}.bias has {view.numel()} values, the projection has {n} outputs")
        keep.append(view)
        setattr(w, field, view.data_ptr())
    w._keep = keep
    return w


class TransformerLayer:
    """One Llama block; `forward_with_weights` runs it on device tensors."""

    def __init__(self, config: LlamaLayerConfig):
        self.cfg = config
        self.scale = 1.0 / math.sqrt(config.head_dim)
        c = qmm.LayerConfig()
        c.hidden_size, c.intermediate_size = config.hidden_size, config.intermediate_size
        c.num_heads, c.num_kv_heads, c.head_dim = config.num_heads, config.num_kv_heads, config.head_dim
        c.rms_norm_eps, c.rope_freq_base, c.rope_neox, c.scale = (config.rms_norm_eps, config.rope_freq_base,
                                                                   int(config.rope_neox), self.scale)
        self._c = c

    def forward_with_weights(self, hidden_states, layer_weights: Dict[str, Tuple[object, object]], layer_idx: int,
                             pos_offset: int = 0, kv_cache: Optional[DeviceKVCache] = None, out=None, stream=None):
        """hidden_states: device fp16 [seq_len, hidden]; layer_weights: {name: (info, device view)}
        as yielded by ResidentWeights.layer_context; kv_cache: the device pool (its layer
        `layer_idx` receives this call's K/V at pos_offset).  Returns (out, None)."""
        import torch

        if kv_cache is None:
            raise ValueError("the device layer needs a DeviceKVCache")
        x = hidden_states
        if (not x.is_cuda or x.dtype != torch.float16 or not x.is_contiguous() or x.dim() != 2
                or x.shape[1] != self.cfg.hidden_size):
            raise ValueError("hidden_states must be a contiguous fp16 device tensor [seq_len, hidden_size]")
        if out is not None and (out.device != x.device or out.dtype != torch.float16 or not out.is_contiguous()
                                or tuple(out.shape) != tuple(x.shape)):
            raise ValueError("out must be a contiguous fp16 tensor of hidden_states' shape on its device")
        y = torch.empty_like(x) if out is None else out
        s = torch.cuda.current_stream(x.device) if stream is None else stream
        with torch.cuda.stream(s):  # bias conversions are ordered before the layer's kernels
            w = layer_weights_struct(layer_weights, f"blk.{layer_idx}.", self.cfg, x.device)
        qmm.check(qmm.lib().qmm_forward_layer(self._c, w, x.data_ptr(), y.data_ptr(), layer_idx, x.shape[0], pos_offset,
                                              s.cuda_stream))
        return y, None

    def forward_resident(self, hidden_states, weights, layer_idx: int, pos_offset: int = 0,
                         kv_cache: Optional[DeviceKVCache] = None, out=None, stream=None):
        """forward_with_weights with the block's tensors taken from a ResidentWeights store."""
        with weights.layer_context(layer_idx) as lw:
            return self.forward_with_weights(hidden_states, lw, layer_idx, pos_offset, kv_cache, out, stream)
