"""Build recipe for the in-tree native artefacts (gfx950 only).

* ``libqmm_gfx950.so`` - the HIP kernels and the C ABI declared in ``include/qmm.h``
  (hipcc, ``--offload-arch=gfx950``);
* ``matmul_module<EXT_SUFFIX>`` - the drop-in pybind11 module, host-only C++ linked against
  ``libqmm_gfx950.so`` with an ``$ORIGIN`` rpath.

Both land next to this file, so they travel with the source tree.  Run as
``python gfx1150-inference_amd/build_ext.py`` or through ``__graft_entry__.build()``.
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libqmm_gfx950.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)

HIP_SOURCES = ["qmm_api.hip", "qmm_gemv.hip", "qmm_gemv_mfma.hip", "qmm_dequant.hip", "qmm_prefill.hip", "qmm_embed.hip", "qmm_upload.hip", "qmm_layer.hip",
               "qmm_host.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}")
    return proc.stdout


def build_libqmm(extra_flags=None) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    flags = HIP_FLAGS + list(extra_flags or [])

    def compile_one(src):
        obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
        _run([HIPCC, *flags, "-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    with ThreadPoolExecutor(max_workers=min(8, len(HIP_SOURCES))) as pool:
        objs = list(pool.map(compile_one, HIP_SOURCES))
    tmp = LIB_PATH + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def matmul_module_path() -> str:
    return os.path.join(PKG_DIR, "matmul_module" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_matmul_module() -> str:
    import pybind11

    out = matmul_module_path()
    tmp = out + ".tmp"
    cmd = [
        "g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-fvisibility=hidden",
        f"-I{pybind11.get_include()}", f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}",
        os.path.join(CSRC, "matmul_module.cpp"),
        f"-L{PKG_DIR}", "-l:" + LIB_NAME, "-Wl,-rpath,$ORIGIN",
        "-o", tmp,
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_libqmm()
    build_matmul_module()


if __name__ == "__main__":
    build_all()
    print(LIB_PATH)
    print(matmul_module_path())
    sys.exit(0)
