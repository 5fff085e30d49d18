"""CPU tests of the C ABI boundary (no compute call needs a GPU here).

* libqmm_gfx950.so loads and exports every function include/qmm.h declares;
* argument validation happens before any HIP call and maps to the reference's error
  classes (src/kernels/dequantize.hip:734-736, 771-773: std::invalid_argument);
* the C++ shim header compiles against the reference's launcher signatures.
"""

import ctypes
import os
import subprocess

import pytest

import qmm

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_declared_symbol():
    declared = qmm.header_symbols()
    assert len(declared) >= 19
    nm = subprocess.run(["nm", "-D", "--defined-only", qmm.LIB_PATH], capture_output=True, text=True, check=True)
    exported = {line.split()[-1] for line in nm.stdout.splitlines() if " T " in line}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    for s in declared:
        getattr(qmm.lib(), s)


def test_version_and_limits():
    assert qmm.lib().qmm_version() == 1000
    assert qmm.gemv_max_m() >= 16  # the reference's M in {4, 7, 16} bit-identity cases stay in GEMV


def test_gemv_threshold_setting():
    """qmm_set_gemv_max_m moves the GEMV / prefill threshold within [1, 65536]; out-of-range
    values are rejected and leave it unchanged (host logic only, no kernel runs)."""
    before = qmm.gemv_max_m()
    assert before == 17
    try:
        qmm.set_gemv_max_m(1024)
        assert qmm.gemv_max_m() == 1024
        for bad in (0, -3, 65537):
            with pytest.raises(ValueError, match="qmm_set_gemv_max_m"):
                qmm.set_gemv_max_m(bad)
            assert qmm.gemv_max_m() == 1024
        qmm.set_gemv_max_m(65536)
        assert qmm.gemv_max_m() == 65536
    finally:
        qmm.set_gemv_max_m(before)
    assert qmm.gemv_max_m() == before


def test_thread_threshold_and_row_identity_settings():
    """qmm_set_thread_gemv_max_m overrides the threshold for the calling thread (0 restores the
    process value); qmm_set_row_identity takes 0 or 1; both reject other values unchanged and
    leave other threads alone (host logic only, no kernel runs)."""
    import threading
    base = qmm.gemv_max_m()
    assert not qmm.row_identity()
    try:
        qmm.set_thread_gemv_max_m(300)
        qmm.set_row_identity(True)
        for bad in (-1, 65537):
            with pytest.raises(ValueError, match="qmm_set_thread_gemv_max_m"):
                qmm.set_thread_gemv_max_m(bad)
        with pytest.raises(ValueError, match="qmm_set_row_identity"):
            qmm.check(qmm.lib().qmm_set_row_identity(2))
        assert qmm.gemv_max_m() == 300 and qmm.row_identity()
        seen = []
        th = threading.Thread(target=lambda: seen.append((qmm.gemv_max_m(), qmm.row_identity())))
        th.start()
        th.join()
        assert seen == [(base, False)]
        qmm.set_gemv_max_m(40)  # the process value moves; this thread keeps its own
        assert qmm.gemv_max_m() == 300
        qmm.set_thread_gemv_max_m(0)
        assert qmm.gemv_max_m() == 40
    finally:
        qmm.set_thread_gemv_max_m(0)
        qmm.set_row_identity(False)
        qmm.set_gemv_max_m(base)
    assert qmm.gemv_max_m() == base and not qmm.row_identity()
    with qmm.row_identity_mode():
        assert qmm.row_identity()
    assert not qmm.row_identity()


@pytest.mark.parametrize("t,n,k,expected", [
    (qmm.GGML_Q4_0, 4096, 4096, 9_437_184),
    (qmm.GGML_Q8_0, 4096, 4096, 17_825_792),
    (qmm.GGML_Q4_K, 28672, 8192, 132_120_576),
    (qmm.GGML_Q6_K, 8192, 28672, 192_675_840),
    (qmm.GGML_Q6_K, 128256, 4096, 430_940_160),
    (qmm.GGML_Q4_K, 10, 100, 0),   # K not a multiple of 256
    (99, 10, 256, 0),              # unknown type
])
def test_weight_bytes(t, n, k, expected):
    assert qmm.weight_bytes(t, n, k) == expected


def _gemm(t, M, N, K, a=1, w=1, c=1, a_dtype=qmm.DTYPE_F32, c_dtype=qmm.DTYPE_F32):
    return qmm.lib().qmm_gemm(t, a, a_dtype, w, c, c_dtype, M, N, K, None)


@pytest.mark.parametrize("t,K,msg", [
    (qmm.GGML_Q4_0, 48, "multiple of 32 for Q4_0"),
    (qmm.GGML_Q8_0, 0, "multiple of 32 for Q8_0"),
    (qmm.GGML_Q4_K, 512 + 32, "multiple of 256 for Q4_K"),
    (qmm.GGML_Q6_K, -256, "multiple of 256 for Q6_K"),
])
def test_gemm_rejects_bad_k(t, K, msg):
    assert _gemm(t, 1, 8, K) == qmm.QMM_ERR_INVALID_ARGUMENT
    assert msg in qmm.last_error()


def test_gemm_rejects_bad_arguments():
    assert _gemm(5, 1, 8, 256) == qmm.QMM_ERR_INVALID_ARGUMENT
    assert "Unsupported ggml_type" in qmm.last_error()
    assert _gemm(qmm.GGML_Q4_K, 1, 8, 256, a_dtype=qmm.DTYPE_BF16) == qmm.QMM_ERR_INVALID_ARGUMENT
    assert _gemm(qmm.GGML_Q4_K, 1, 8, 256, c_dtype=7) == qmm.QMM_ERR_INVALID_ARGUMENT
    assert _gemm(qmm.GGML_Q4_K, -1, 8, 256) == qmm.QMM_ERR_INVALID_ARGUMENT
    assert _gemm(qmm.GGML_Q4_K, 1, -8, 256) == qmm.QMM_ERR_INVALID_ARGUMENT
    assert _gemm(qmm.GGML_Q4_K, 1, 8, 256, w=0) == qmm.QMM_ERR_INVALID_ARGUMENT
    assert "non-null" in qmm.last_error()
    with pytest.raises(ValueError):
        qmm.check(_gemm(qmm.GGML_Q4_K, 1, 8, 100))


def test_empty_shapes_are_no_ops():
    # M == 0 or N == 0 returns before touching the device.
    assert _gemm(qmm.GGML_Q4_K, 0, 8, 256, a=0, w=0, c=0) == qmm.QMM_OK
    assert _gemm(qmm.GGML_Q6_K, 3, 0, 2048, a=0, w=0, c=0) == qmm.QMM_OK
    assert qmm.lib().qmm_dequantize(qmm.GGML_Q4_K, None, None, qmm.DTYPE_F16, 0, None) == qmm.QMM_OK
    assert qmm.lib().qmm_matmul_q4_0_host(None, None, None, 0, 4, 32) == qmm.QMM_OK


def test_dequantize_rejects_bad_arguments():
    L = qmm.lib()
    assert L.qmm_dequantize(qmm.GGML_Q4_K, 1, 16, qmm.DTYPE_F16, 300, None) == qmm.QMM_ERR_INVALID_ARGUMENT
    assert "multiple of 256 for Q4_K dequantization" in qmm.last_error()
    assert L.qmm_dequantize(qmm.GGML_Q4_0, 1, 16, 9, 32, None) == qmm.QMM_ERR_INVALID_ARGUMENT
    assert L.qmm_dequantize(qmm.GGML_Q4_0, 1, 18, qmm.DTYPE_F16, 32, None) == qmm.QMM_ERR_INVALID_ARGUMENT
    assert "16-byte aligned" in qmm.last_error()
    assert L.qmm_dequantize_q8_0_host(1, 1, 33) == qmm.QMM_ERR_INVALID_ARGUMENT
    assert L.qmm_matmul_q6_k_host(1, 1, 1, 1, 1, 255) == qmm.QMM_ERR_INVALID_ARGUMENT


def test_last_error_is_thread_local():
    import threading

    _gemm(qmm.GGML_Q4_K, 1, 8, 100)
    main_msg = qmm.last_error()
    seen = {}

    def worker():
        seen["before"] = qmm.last_error()
        _gemm(qmm.GGML_Q4_0, 1, 8, 48)
        seen["after"] = qmm.last_error()

    th = threading.Thread(target=worker)
    th.start()
    th.join()
    assert seen["before"] == ""
    assert "Q4_0" in seen["after"]
    assert qmm.last_error() == main_msg


def test_cpp_shim_header_compiles(tmp_path):
    src = tmp_path / "use_shims.cpp"
    src.write_text(
        '#include "qmm_launchers.hpp"\n'
        "void (*p0)(const void*, const void*, void*, int, int, int) = &launch_matmul_q4_k_device;\n"
        "void (*p1)(const void*, const void*, void*, int, int, int) = &launch_matmul_q6_k;\n"
        "void (*p2)(const void*, void*, int) = &launch_dequantize_q8_0;\n"
        "static_assert(BLOCK_Q6_K_BYTES == 210, \"\");\n")
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", f"-I{os.path.join(REPO, 'include')}", str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_cpp_caller_links_and_loads():
    """The C++ caller of qmm_launchers.hpp (built by build(), tests/cpp/Makefile) resolves every
    symbol it uses from libqmm_gfx950.so at load time; without arguments it prints its usage and
    exits with 2 before any HIP call."""
    exe = os.path.join(REPO, "tests", "cpp", "_build", "launchers_caller")
    assert os.path.exists(exe), "run __graft_entry__.build() (make -C tests/cpp)"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=60, env={**os.environ, "LD_BIND_NOW": "1"})
    assert r.returncode == 2 and "usage" in r.stderr, (r.returncode, r.stderr)


def test_c_header_is_plain_c(tmp_path):
    src = tmp_path / "use_c.c"
    src.write_text('#include "qmm.h"\nint f(void) { return qmm_version(); }\n')
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only",
                        f"-I{os.path.join(REPO, 'include')}", str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
