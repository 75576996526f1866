"""Build libmcop_norm.so (the gfx950 kernels and their C ABI) in-tree with hipcc, and the C++
torch extension _torch_ops.so (the mcoplib.op / torch.ops._C surfaces over that ABI) with g++.

Usage: python mcoplib_amd/_build.py [--jobs N]
(run as a script: importing the package would load the library this builds)

Each csrc/*.hip translation unit is compiled for gfx950 only, in parallel, then linked into
mcoplib_amd/libmcop_norm.so next to this file. Objects go to mcoplib_amd/_build/.
csrc/torch_ops.cpp is host C++ against torch's headers (ROCm build) and links
libmcop_norm.so through an $ORIGIN run path.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libmcop_norm.so"
EXT = PKG / "_torch_ops.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: the arithmetic is specified operation by operation (each fp32 product is
#   rounded before it is used); explicit __builtin_fma is used where a fused op is intended.
# -packed-fp32-ops disabled: no v_pk_*_f32 is emitted.
COMPILE_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-gpu-rdc",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, build_dir: Path = BUILD, defines: tuple = ()) -> Path:
    obj = build_dir / (src.stem + ".o")
    cmd = [HIPCC, *COMPILE_FLAGS, *[f"-D{d}" for d in defines], "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = True, out: Path = LIB,
          defines: tuple = ()) -> Path:
    """Compile every kernel source and link libmcop_norm.so (or `out`, with extra -D
    `defines`, for tuning builds). Always rebuilds."""
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    build_dir = BUILD if out == LIB else BUILD / out.stem
    build_dir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, build_dir, defines), srcs))
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", f"-Wl,-soname,{LIB.name}", "-o",
           str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} from {len(srcs)} sources", file=sys.stderr)
    return out


def build_extension(verbose: bool = True) -> Path:
    """Compile csrc/torch_ops.cpp into mcoplib_amd/_torch_ops.so (always rebuilds)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    tdir = Path(torch.__file__).resolve().parent
    cxx = os.environ.get("CXX", "g++")
    abi = int(torch.compiled_with_cxx11_abi())
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"]]
    if "/opt/rocm/include" not in incs:
        incs.append("/opt/rocm/include")
    tmp = EXT.with_suffix(".so.tmp")
    cmd = [cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Wno-unused-function",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_torch_ops",
           "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *[f"-I{p}" for p in incs], str(CSRC / "torch_ops.cpp"), "-o", str(tmp),
           f"-L{tdir / 'lib'}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
           "-ltorch_python", f"-L{PKG}", "-lmcop_norm", "-Wl,-rpath,$ORIGIN",
           f"-Wl,-rpath,{tdir / 'lib'}"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"{cxx} failed for torch_ops.cpp:\n{proc.stderr}")
    os.replace(tmp, EXT)
    if verbose:
        print(f"built {EXT}", file=sys.stderr)
    return EXT


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    build(args.jobs)
    build_extension()


if __name__ == "__main__":
    main()
