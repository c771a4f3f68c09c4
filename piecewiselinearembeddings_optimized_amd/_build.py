"""In-tree build of the native parts of the package.

* ``libple_hip.so`` -- the HIP kernels and the C ABI of ``include/ple_hip.h``,
  compiled by ``hipcc`` for gfx950 only.
* ``_C<ext-suffix>`` -- the CPython extension that registers the
  ``torch.ops.rtdl_num_embeddings_cuda`` operators (host C++, ``g++``), linked
  against ``libple_hip.so`` with an ``$ORIGIN`` rpath.

Both land next to this file, so a copy of the source tree (as shipped to a GPU
box) carries them.  No hipify step and no CUDA headers are involved.

Usage: ``python -m piecewiselinearembeddings_optimized_amd._build``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
KERNEL_LIB = os.path.join(PKG_DIR, "libple_hip.so")
EXT_SUFFIX = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
EXT_PATH = os.path.join(PKG_DIR, "_C" + EXT_SUFFIX)

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
OFFLOAD_ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Packed fp32 VALU ops stay off (the compiler would otherwise form them
    # from ordinary float code).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in res.stdout.splitlines()
        # hipcc's host pass does not know the device-only feature name
        if "packed-fp32-ops" not in line and "is not a recognized feature" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def _hipcc() -> str:
    p = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found; set ROCM_PATH")
    return p


KERNEL_SOURCES = ("ple_capi.hip", "ple_forward.hip", "ple_backward.hip", "ple_encode.hip", "ple_noalloc.hip")


def build_kernels(verbose: bool = False) -> str:
    """One hipcc process per translation unit (in parallel), then the link."""
    import concurrent.futures as cf
    import tempfile

    hipcc = _hipcc()
    with tempfile.TemporaryDirectory(prefix="ple_build_") as tmpdir:
        objs = [os.path.join(tmpdir, os.path.splitext(s)[0] + ".o") for s in KERNEL_SOURCES]
        cmds = [[hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", "-c", "-o", o, os.path.join(CSRC, s)]
                for s, o in zip(KERNEL_SOURCES, objs)]
        with cf.ThreadPoolExecutor(max_workers=len(cmds)) as ex:
            for fut in [ex.submit(_run, c, verbose) for c in cmds]:
                fut.result()
        tmp = KERNEL_LIB + ".tmp"
        _run([hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-Wl,-soname,libple_hip.so",
              "-o", tmp, *objs], verbose)
    os.replace(tmp, KERNEL_LIB)
    return KERNEL_LIB


def build_extension(verbose: bool = False) -> str:
    import torch
    from torch.utils import cpp_extension

    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], os.path.join(ROCM, "include"), INCLUDE]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    src = os.path.join(CSRC, "ple_ops.cpp")
    tmp = EXT_PATH + ".tmp"
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-function",
        "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *[f"-I{i}" for i in incs],
        "-o", tmp, src,
        f"-L{PKG_DIR}", "-lple_hip",
        f"-L{torch_lib}", "-lc10", "-ltorch_cpu", "-ltorch", "-lc10_hip", "-lamdhip64",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}",
    ]
    _run(cmd, verbose)
    os.replace(tmp, EXT_PATH)
    return EXT_PATH


def build(verbose: bool = False) -> None:
    build_kernels(verbose)
    build_extension(verbose)


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
