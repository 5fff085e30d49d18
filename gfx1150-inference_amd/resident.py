"""A GGUF model's tensors loaded once into HBM.

Replaces, for MI355X, the reference's weight path: WeightStreamer (src/weight_loader.py:45-203)
maps the file, advises the page cache per layer and hands out host views, and every projection
then copies its packed bytes to the GPU before its kernel (project_on_device,
src/kernels/attention.hip:572-599; the host wrappers, src/kernels/dequantize.hip:729-762).  A
whole quantized model fits in the 288 GB of HBM, so ResidentWeights reads every tensor's bytes
from the file once, through the library's parallel loader (qmm_upload_file: pread into pinned
staging buffers overlapped with host -> device copies), into one device arena, and hands out
device tensors that stay valid until close().

The surface follows WeightStreamer: `gguf`, `num_layers`, `validate_supported_tensors()`,
`get_tensor_view(name)`, `layer_context(idx)` (yielding {name: (info, view)}), the
prefetch / release calls (no-ops: everything is resident) and close / context manager.  Views
are device tensors instead of NumPy arrays: uint8 packed bytes for quantized tensors, float16 /
float32 of `shape_row_major` for F16 / F32 ones.
"""

from __future__ import annotations

import contextlib
import mmap
import os
import time
from typing import Dict, FrozenSet, Iterable, Iterator, Optional, Tuple

import gguf
import qmm
from gguf import GGMLType, GGUFParser, GGUFTensorInfo

SUPPORTED_COMPUTE_GGML_TYPES: FrozenSet[GGMLType] = frozenset(
    {GGMLType.F32, GGMLType.F16, GGMLType.Q4_0, GGMLType.Q8_0, GGMLType.Q4_K, GGMLType.Q6_K})

ARENA_ALIGN = 256  # every tensor starts on a 256-byte boundary of the arena


def parse_file(model_path: str) -> GGUFParser:
    """GGUF header and tables of a file (read through a private read-only map)."""
    with open(model_path, "rb") as f:
        with mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
            return GGUFParser(mm)


def unsupported_tensors(parser: GGUFParser) -> list:
    return [f"{t.name} ({t.ggml_type.name})" for t in parser.tensors.values()
            if t.ggml_type not in SUPPORTED_COMPUTE_GGML_TYPES]


class ResidentWeights:
    """All (or the named) tensors of a GGUF file, resident in device memory."""

    def __init__(self, model_path: str, validate_types: bool = True, device=None,
                 names: Optional[Iterable[str]] = None, chunk_bytes: int = 16 << 20, depth: int = 2,
                 threads: int = 8, stream=None):
        import torch

        self.model_path = model_path
        self.gguf = parse_file(model_path)
        arch = str(self.gguf.metadata.get("general.architecture", "llama"))
        self.num_layers = int(self.gguf.metadata.get(f"{arch}.block_count",
                                                     self.gguf.metadata.get("llama.block_count", 0)))
        if validate_types:
            self.validate_supported_tensors()
        wanted = None if names is None else set(names)
        if wanted is not None:
            missing = sorted(wanted - set(self.gguf.tensors))
            if missing:
                raise KeyError(f"Tensors not in {model_path}: {', '.join(missing[:8])}")
        infos = sorted((t for n, t in self.gguf.tensors.items() if wanted is None or n in wanted),
                       key=lambda t: t.abs_offset)
        self._place: Dict[str, int] = {}
        size = 0
        for t in infos:
            self._place[t.name] = size
            size = gguf.align_offset(size + t.n_bytes, ARENA_ALIGN)
        self.device = torch.device("cuda") if device is None else torch.device(device)
        self.arena = torch.empty(max(size, ARENA_ALIGN), dtype=torch.uint8, device=self.device)
        ranges = (qmm.FileRange * max(len(infos), 1))()
        base = self.arena.data_ptr()
        for r, t in zip(ranges, infos):
            r.offset, r.bytes, r.dst = t.abs_offset, t.n_bytes, base + self._place[t.name]
        s = torch.cuda.current_stream(self.device) if stream is None else stream
        t0 = time.perf_counter()
        qmm.check(qmm.lib().qmm_upload_file(os.fsencode(model_path), ranges, len(infos), int(chunk_bytes), int(depth),
                                            int(threads), s.cuda_stream))
        self.upload_seconds = time.perf_counter() - t0
        self.nbytes = sum(t.n_bytes for t in infos)

    # ---- WeightStreamer surface
    def validate_supported_tensors(self) -> None:
        """ValueError naming the tensors whose type the kernels do not compute (reference
        src/weight_loader.py:82-97)."""
        bad = unsupported_tensors(self.gguf)
        if bad:
            supported = ", ".join(sorted(t.name for t in SUPPORTED_COMPUTE_GGML_TYPES))
            raise ValueError(f"Model contains tensors with unsupported quantization types: {', '.join(bad[:8])}. "
                             f"Supported types: {supported}.")

    def info(self, name: str) -> GGUFTensorInfo:
        return self.gguf.tensors[name]

    def device_ptr(self, name: str) -> int:
        """Device address of the tensor's packed bytes (for qmm_gemm / qmm_gemm_batch)."""
        return self.arena.data_ptr() + self._place[name]

    def get_tensor_view(self, name: str):
        """Device view of a resident tensor: uint8 packed bytes, or float16 / float32 of
        `shape_row_major` for F16 / F32 tensors."""
        import torch

        t = self.gguf.tensors[name]
        if name not in self._place:
            raise KeyError(f"Tensor {name!r} was not loaded")
        p = self._place[name]
        raw = self.arena[p:p + t.n_bytes]
        if t.ggml_type == GGMLType.F16:
            return raw.view(torch.float16).reshape(t.shape_row_major)
        if t.ggml_type == GGMLType.F32:
            return raw.view(torch.float32).reshape(t.shape_row_major)
        return raw

    @contextlib.contextmanager
    def layer_context(self, layer_idx: int, prefetch_next: bool = True
                      ) -> Iterator[Dict[str, Tuple[GGUFTensorInfo, object]]]:
        """{name: (info, device view)} of block `layer_idx`'s resident tensors."""
        views = {n: (t, self.get_tensor_view(n)) for n, t in self.gguf.get_layer_tensors(layer_idx).items()
                 if n in self._place}
        try:
            yield views
        finally:
            views.clear()

    def prefetch_layer(self, layer_idx: int) -> None:
        """Resident: nothing to prefetch."""

    def release_layer(self, layer_idx: int) -> None:
        """Resident: nothing to release."""

    def prefetch_tensor(self, name: str) -> None:
        """Resident: nothing to prefetch."""

    def release_tensor(self, name: str) -> None:
        """Resident: nothing to release."""

    def close(self) -> None:
        """Drops the arena (freed once no view of it is alive)."""
        self.arena = None
        self._place = {}

    def __enter__(self) -> "ResidentWeights":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


def read_ranges_to_host(model_path: str, ranges: Iterable[Tuple[int, object]], threads: int = 8) -> None:
    """Fills writable host buffers from file offsets with the library's parallel reader:
    `ranges` holds (file offset, buffer) pairs; each buffer receives len(buffer) bytes."""
    import numpy as np

    items = list(ranges)
    arr = (qmm.FileRange * max(len(items), 1))()
    keep = []
    for r, (off, buf) in zip(arr, items):
        a = np.asarray(buf)
        if not a.flags.c_contiguous or not a.flags.writeable:
            raise ValueError("buffers must be C-contiguous and writeable")
        keep.append(a)
        r.offset, r.bytes, r.dst = int(off), a.nbytes, a.ctypes.data
    qmm.check(qmm.lib().qmm_read_file(os.fsencode(model_path), arr, len(items), int(threads)))
