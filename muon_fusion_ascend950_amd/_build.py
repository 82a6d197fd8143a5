"""In-tree build of the native libraries (gfx950 only).

Two shared objects land next to this file:

* ``libmuon_polar.so`` — the HIP kernels and the C ABI of ``include/muon_polar.h``
  (``hipcc --offload-arch=gfx950``; no torch dependency).
* ``_C.so`` — the torch operator ``muon_ascend950::polar_step`` (g++ against the
  torch headers), linked to ``libmuon_polar.so``.

This mirrors the reference build (``setup.py:46-153``: an accelerator compiler
turns the kernel source into an object, then a C++ extension links it), with
``hipcc`` in place of ``bisheng``.  Run ``python -m muon_fusion_ascend950_amd._build``
or ``python setup.py build_ext --inplace``.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
BUILD_DIR = PKG_DIR / "_build_obj"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

# Packed-FP32 VALU forms are disabled for all device code.
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    exe = ROCM / "bin" / "hipcc"
    return str(exe) if exe.exists() else "hipcc"


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout)
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd[:2])} ...")
    if verbose and proc.stdout.strip():
        # hipcc's host pass warns about the device-only target feature: harmless.
        lines = [ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln]
        if lines:
            print("\n".join(lines), flush=True)


def _torch_paths() -> tuple[list[str], Path]:
    import torch  # noqa: WPS433 (build-time only)

    root = Path(torch.__file__).resolve().parent
    incs = [str(root / "include"), str(root / "include" / "torch" / "csrc" / "api" / "include")]
    return incs, root / "lib"


def build_hip_library(verbose: bool = True) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    common = HIP_FLAGS + [f"-I{INCLUDE}", f"-I{CSRC}"]
    sources = ["polar_kernels.hip", "polar_stream.hip", "polar_norm.hip", "polar_noalloc.hip",
               "polar_capi.cpp"]
    objects = [BUILD_DIR / (Path(src).stem + ".o") for src in sources]
    jobs = [[_hipcc(), "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)] + common
            for src, obj in zip(sources, objects)]
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(jobs)) as pool:
        for fut in [pool.submit(_run, cmd, verbose) for cmd in jobs]:
            fut.result()
    out = PKG_DIR / "libmuon_polar.so"
    tmp = out.with_suffix(".so.tmp")
    _run([_hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}"] + [str(o) for o in objects]
         + ["-Wl,-soname,libmuon_polar.so", "-o", str(tmp)], verbose)
    os.replace(tmp, out)
    return out


def build_torch_binding(verbose: bool = True) -> Path:
    incs, torch_lib = _torch_paths()
    import torch

    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    out = PKG_DIR / "_C.so"
    tmp = out.with_suffix(".so.tmp")
    cxx = shutil.which("g++") or "g++"
    cmd = [
        cxx, "-O2", "-std=c++17", "-fPIC", "-shared",
        str(CSRC / "muon_polar_step_binding.cpp"),
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        f"-I{INCLUDE}", f"-I{ROCM / 'include'}",
        f"-I{sysconfig.get_paths()['include']}",
    ]
    cmd += [f"-I{p}" for p in incs]
    cmd += [
        f"-L{PKG_DIR}", "-lmuon_polar",
        f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
        f"-L{ROCM / 'lib'}", "-lamdhip64",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}",
        "-o", str(tmp),
    ]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = True) -> None:
    """Compile both native libraries in place (always recompiles)."""
    build_hip_library(verbose)
    build_torch_binding(verbose)


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
