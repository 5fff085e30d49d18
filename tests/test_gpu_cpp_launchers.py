"""A C++ caller of include/qmm_launchers.hpp, linked to libqmm_gfx950.so and run on the GPU.

tests/cpp/launchers_caller.cpp is written against the reference's launcher signatures
(src/kernels/dequantize.h:25-132): it calls launch_matmul_<t> on host buffers, launch_matmul_<t>_device
on device buffers (null stream) and launch_dequantize_<t>, and checks that a K the block format
cannot represent throws std::invalid_argument as the reference does.  Bars: host and device
results bit-identical to each other and to qmm_gemm in row-identity mode (the mode the reference
launchers run in), within max_i|y_i - y64_i| / max_i|y64_i| <= 1e-3 of the fp64 product (fp16
outputs included), and the dequantization bit-exact against the oracle.  The program is built by
build() (tests/cpp/Makefile).
"""

import os
import subprocess

import numpy as np
import pytest

import gguf_oracle as O

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CALLER = os.path.join(REPO, "tests", "cpp", "_build", "launchers_caller")


@pytest.mark.parametrize("t", [O.GGML_Q4_0, O.GGML_Q8_0, O.GGML_Q4_K, O.GGML_Q6_K])
@pytest.mark.parametrize("M", [1, 5])
def test_cpp_caller_of_reference_launchers(cuda, tmp_path, t, M):
    import torch
    import qmm
    if not os.path.exists(CALLER):
        pytest.fail(f"{CALLER} is not built: run __graft_entry__.build() (make -C tests/cpp)")
    N, K = 96, 4096
    rng = np.random.default_rng(1500 + 10 * t + M)
    raw = O.synth_weights(t, N, K, rng)
    x = rng.standard_normal((M, K)).astype(np.float16)
    inp, out = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(inp, "wb") as f:
        f.write(np.array([t, M, N, K], np.int32).tobytes())
        f.write(x.tobytes())
        f.write(raw.tobytes())
    print(f"cpp caller type={O.TYPE_NAMES[t]} M={M} N={N} K={K}", flush=True)
    r = subprocess.run([CALLER, str(inp), str(out)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    buf = np.fromfile(out, np.uint8)
    mn, nk = M * N * 2, N * K * 2
    assert buf.size == 2 * mn + nk + 4
    c_host = buf[:mn].view(np.float16).reshape(M, N)
    c_dev = buf[mn:2 * mn].view(np.float16).reshape(M, N)
    deq = buf[2 * mn:2 * mn + nk].view(np.float16)
    threw = int(buf[2 * mn + nk:].view(np.int32)[0])
    assert threw == 1
    np.testing.assert_array_equal(c_host.view(np.uint16), c_dev.view(np.uint16))
    np.testing.assert_array_equal(deq.view(np.uint16), O.dequantize_f16(t, raw, N * K).view(np.uint16))
    assert O.max_rel_err(c_host.astype(np.float64), O.matmul_f64(t, x.astype(np.float32), raw, N, K)) <= 1e-3
    with qmm.row_identity_mode():
        y = qmm.gemm(t, torch.from_numpy(x).to(cuda), torch.from_numpy(raw).to(cuda), N, K, out_dtype=torch.float16)
        torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy().view(np.uint16), c_host.view(np.uint16))
