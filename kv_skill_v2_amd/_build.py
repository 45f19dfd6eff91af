"""Build recipe for libxenc_hip.so (hand-written HIP kernels for gfx950 + the C ABI).

Compiled in-tree with hipcc so the built library travels with the source tree:
    python -m kv_skill_v2_amd._build
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "_lib"
LIB = LIBDIR / "libxenc_hip.so"
TORCH_LIB = LIBDIR / "libxenc_torch.so"
TORCH_OPS_SRC = CSRC / "torch_ops.cpp"
ARCH = "gfx950"

# Packed fp32 VALU ops are disabled: the kernels here are written for scalar/float4 math.
HIPFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with exit code {res.returncode}")


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source into one shared library (always rebuilds).  Each source is
    compiled to an object file in parallel (every translation unit carries its own device code),
    then the objects are linked."""
    LIBDIR.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cc = hipcc()
    inc = ["-I", str(PKG.parent / "include")]
    jobs = jobs or min(len(sources()), max(1, min(os.cpu_count() or 1, 16)))
    with tempfile.TemporaryDirectory(prefix="xenc_build_") as td:
        objs = [str(Path(td) / (src.stem + ".o")) for src in sources()]
        cmds = [[cc, *HIPFLAGS, *inc, "-c", str(src), "-o", obj] for src, obj in zip(sources(), objs)]
        with ThreadPoolExecutor(max_workers=jobs) as ex:
            list(ex.map(lambda c: _run(c, verbose), cmds))
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)], verbose)
    os.replace(tmp, LIB)
    build_torch_ops(verbose)
    return LIB


def build_torch_ops(verbose: bool = False) -> Path:
    """The per-token operators registered in torch's dispatcher from C++ (csrc/torch_ops.cpp):
    host code only, compiled by the system C++ compiler against torch's headers and linked to
    libxenc_hip.so (found next to it at load time)."""
    import torch

    tdir = Path(torch.__file__).resolve().parent
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cxx = os.environ.get("CXX") or shutil.which("g++") or "c++"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = TORCH_LIB.with_suffix(".so.tmp")
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-I", str(tdir / "include"), "-I", str(tdir / "include" / "torch" / "csrc" / "api" / "include"),
           "-I", str(Path(rocm) / "include"), "-I", str(PKG.parent / "include"),
           str(TORCH_OPS_SRC), "-o", str(tmp),
           "-L", str(tdir / "lib"), "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
           "-L", str(LIBDIR), "-lxenc_hip", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tdir / 'lib'}"]
    _run(cmd, verbose)
    os.replace(tmp, TORCH_LIB)
    return TORCH_LIB


if __name__ == "__main__":
    print(build(verbose=True))
