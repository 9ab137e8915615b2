"""Build ``libtokenforge_hip.so`` (the C-ABI library of the gfx950 kernels) in-tree.

    python -m tokenforge_amd.build [--jobs N] [--verbose]

Every ``csrc/*.hip`` file is compiled separately with ``hipcc --offload-arch=gfx950`` (in
parallel), then linked into ``tokenforge_amd/lib/libtokenforge_hip.so``. The library
depends only on the HIP runtime; it has no PyTorch headers or symbols.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD_DIR = PKG.parent / "_build"
LIB_DIR = PKG / "lib"
LIB_NAME = "libtokenforge_hip.so"
ARCH = "gfx950"

# Packed-FP32 VALU forms are disabled: hipcc -O3 would otherwise emit v_pk_{add,mul,fma}_f32
# from scalar float code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; that is benign.
    noise = ("packed-fp32-ops", "not a recognized feature")
    err = "\n".join(
        line for line in proc.stderr.splitlines() if not any(n in line for n in noise)
    ).strip()
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if err and verbose:
        print(err, file=sys.stderr)


def _link(cc: str, objects: list[Path], out: Path, verbose: bool) -> None:
    tmp = out.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)], verbose)
    os.replace(tmp, out)


def build_library(sources: list[Path], out: Path, jobs: int | None = None, verbose: bool = False,
                  tag: str = "") -> Path:
    """Compile ``sources`` (in parallel, objects under ``_build/`` prefixed with ``tag``) and
    link them into the shared library ``out``."""
    cc = hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    out.parent.mkdir(parents=True, exist_ok=True)
    objects = [BUILD_DIR / (tag + s.stem + ".o") for s in sources]
    cmds = [[cc, *HIPCC_FLAGS, "-c", str(s), "-o", str(o)] for s, o in zip(sources, objects)]
    with ThreadPoolExecutor(max_workers=jobs or min(8, os.cpu_count() or 1)) as pool:
        list(pool.map(lambda c: _run(c, verbose), cmds))
    _link(cc, objects, out, verbose)
    return out


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every kernel source and link the product library, then the torch operator
    extension. Returns the kernel library's path."""
    out = build_library(sorted(CSRC.glob("*.hip")), LIB_DIR / LIB_NAME, jobs, verbose)
    build_torch_ops(verbose)
    return out


TORCH_OPS_SRC = PKG / "ext" / "torch_ops.cpp"
TORCH_OPS_NAME = "libtokenforge_torch.so"


def build_torch_ops(verbose: bool = False) -> Path:
    """The torch.ops.tokenforge extension (``ext/torch_ops.cpp``): host C++ against PyTorch's
    headers and libraries, no device code. It calls the kernel library through its C ABI, bound
    at run time, so it has no link-time dependency on it. The HIP headers that PyTorch's ROCm
    stream and guard headers include need ``__HIP_PLATFORM_AMD__`` and ``USE_ROCM`` defined."""
    import torch

    torch_dir = Path(torch.__file__).resolve().parent
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    out = LIB_DIR / TORCH_OPS_NAME
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    cxx = os.environ.get("CXX", "g++")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = out.with_suffix(".so.tmp")
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
          "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM", f"-I{torch_dir / 'include'}",
          f"-I{torch_dir / 'include' / 'torch' / 'csrc' / 'api' / 'include'}", f"-I{rocm / 'include'}",
          str(TORCH_OPS_SRC), "-o", str(tmp), f"-L{torch_dir / 'lib'}", f"-Wl,-rpath,{torch_dir / 'lib'}",
          "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ldl"], verbose)
    os.replace(tmp, out)
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
