"""GPU tests of the resident weight store (qmm_upload_file through resident.ResidentWeights).

Bars:
* every tensor's device bytes equal the file's, bit for bit, for chunk sizes that split tensors
  across staging buffers and for ones that pack several tensors into one chunk;
* F16 / F32 views have the tensor's row-major shape and values; layer_context yields the
  layer's tensors;
* a GEMV / prefill GEMM on a resident weight is within the kernel bars of the oracle (1e-3 and
  1e-2 of fp64), i.e. the resident bytes are usable in place.
"""

import numpy as np
import pytest

import gguf_oracle as O
from gguf import GGMLType, GGUFValueType, write_synthetic_gguf

pytestmark = pytest.mark.gpu

MiB = 1 << 20


@pytest.fixture(scope="module")
def dev(cuda):
    import qmm  # noqa: F401  (fails loudly if the library is not built)
    return cuda


def make_model(path, rng):
    """Two layers of mixed formats; sizes chosen so 4 MiB chunks split several tensors."""
    H, F = 1024, 2816
    specs = [
        ("token_embd.weight", GGMLType.Q6_K, 512, H),
        ("blk.0.attn_norm.weight", GGMLType.F32, 1, H),
        ("blk.0.attn_q.weight", GGMLType.Q4_K, H, H),
        ("blk.0.ffn_gate.weight", GGMLType.Q4_K, F, H),
        ("blk.0.ffn_down.weight", GGMLType.Q6_K, H, F),
        ("output_norm.weight", GGMLType.F16, 1, H),
        ("blk.1.attn_q.weight", GGMLType.Q8_0, H, H),
        ("blk.1.ffn_up.weight", GGMLType.Q4_0, F, H),
        ("blk.1.attn_norm.weight", GGMLType.F16, 1, H),
    ]
    tensors, raws = [], {}
    for name, t, n, k in specs:
        if t == GGMLType.F32:
            raw = rng.standard_normal(n * k).astype(np.float32).view(np.uint8)
        elif t == GGMLType.F16:
            raw = rng.standard_normal(n * k).astype(np.float16).view(np.uint8)
        else:
            raw = O.synth_weights(int(t), n, k, rng)
        dims = (k,) if n == 1 else (k, n)
        tensors.append((name, dims, t, raw.tobytes()))
        raws[name] = raw
    meta = {"general.architecture": (GGUFValueType.STRING, "llama"), "llama.block_count": (GGUFValueType.UINT32, 2)}
    with open(path, "wb") as f:
        write_synthetic_gguf(f, meta, tensors)
    return raws


@pytest.mark.parametrize("chunk_mb,depth,threads", [(4, 2, 3), (64, 3, 16)])
def test_resident_bytes_equal_file(dev, tmp_path, chunk_mb, depth, threads):
    import torch
    import resident

    rng = np.random.default_rng(31 + chunk_mb)
    path = tmp_path / "model.gguf"
    raws = make_model(path, rng)
    with resident.ResidentWeights(str(path), chunk_bytes=chunk_mb * MiB, depth=depth, threads=threads) as rw:
        assert rw.num_layers == 2
        assert rw.nbytes == sum(r.nbytes for r in raws.values())
        for name, raw in raws.items():
            v = rw.get_tensor_view(name)
            got = v.contiguous().view(torch.uint8).reshape(-1).cpu().numpy()
            assert np.array_equal(got, raw.reshape(-1)), name
            assert rw.device_ptr(name) % resident.ARENA_ALIGN == 0
        norm = rw.get_tensor_view("blk.1.attn_norm.weight")
        assert norm.dtype == torch.float16 and tuple(norm.shape) == (1024,)
        with rw.layer_context(0) as layer:
            assert sorted(layer) == ["blk.0.attn_norm.weight", "blk.0.attn_q.weight", "blk.0.ffn_down.weight",
                                     "blk.0.ffn_gate.weight"]
            info, view = layer["blk.0.attn_norm.weight"]
            assert info.ggml_type == GGMLType.F32 and view.dtype == torch.float32


def test_resident_weights_feed_the_kernels(dev, tmp_path):
    import torch
    import qmm
    import resident

    rng = np.random.default_rng(77)
    path = tmp_path / "model.gguf"
    raws = make_model(path, rng)
    names = ["blk.0.ffn_gate.weight", "blk.0.ffn_down.weight"]
    rw = resident.ResidentWeights(str(path), names=names, chunk_bytes=4 * MiB)
    assert rw.nbytes == sum(raws[n].nbytes for n in names)
    for name, t, n, k in (("blk.0.ffn_gate.weight", O.GGML_Q4_K, 2816, 1024),
                          ("blk.0.ffn_down.weight", O.GGML_Q6_K, 1024, 2816)):
        w = rw.get_tensor_view(name)
        for M, tol in ((1, 1e-3), (64, 1e-2)):
            x = rng.standard_normal((M, k)).astype(np.float32)
            y = qmm.gemm(t, torch.from_numpy(x).to(dev), w, n, k)
            torch.cuda.synchronize()
            assert O.max_rel_err(y.cpu().numpy().astype(np.float64), O.matmul_f64(t, x, raws[name], n, k)) <= tol
    with pytest.raises(KeyError):
        rw.get_tensor_view("blk.1.ffn_up.weight")  # not loaded
    rw.close()


def test_upload_rejects_bad_ranges_before_copying(dev, tmp_path):
    import torch
    import qmm

    path = tmp_path / "blob.bin"
    np.arange(4096, dtype=np.uint8).tofile(path)
    dst = torch.zeros(8192, dtype=torch.uint8, device=dev)
    rr = (qmm.FileRange * 1)()
    rr[0].offset, rr[0].bytes, rr[0].dst = 4000, 200, dst.data_ptr()
    with pytest.raises(ValueError):
        qmm.check(qmm.lib().qmm_upload_file(str(path).encode(), rr, 1, 4 * MiB, 2, 4, None))
    rr[0].offset, rr[0].bytes = 96, 4000
    with pytest.raises(ValueError):  # depth outside [2, 8]
        qmm.check(qmm.lib().qmm_upload_file(str(path).encode(), rr, 1, 4 * MiB, 1, 4, None))
    qmm.check(qmm.lib().qmm_upload_file(str(path).encode(), rr, 1, 4 * MiB, 2, 4, None))
    assert np.array_equal(dst[:4000].cpu().numpy(), (np.arange(96, 4096) % 256).astype(np.uint8))
    assert int(dst[4000:].sum()) == 0
