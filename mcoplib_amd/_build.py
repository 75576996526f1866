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
import json
import os
import re
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


# Kernels that ask for four waves per SIMD (amdgpu_waves_per_eu(4), i.e. at most 128 VGPRs): each
# must meet that bound without spilling registers to scratch.  Patterns match demangled names.
FOUR_WAVE_KERNELS = (
    r"^void mcop::k_rms_norm_quant<mcop::BF16, 8, 8, false, (true|false), [0-9], (true|false)>\(",
    r"^void mcop::k_fused_add_rms_norm<mcop::BF16, 8, 8, (true|false)>\(",
    r"^void mcop::k_rms_norm_quant_split<mcop::BF16, 8, 8, false, (true|false), [0-9]>\(",
)
RESOURCES = "resource_usage.json"


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _remarks(text: str, tu: str) -> list[dict]:
    """Per-kernel records of hipcc's -Rpass-analysis=kernel-resource-usage remarks."""
    out, cur = [], None
    for line in text.splitlines():
        m = re.search(r"remark: (?:\s*)Function Name: (\S+)", line)
        if m:
            cur = {"tu": tu, "mangled": m.group(1)}
            out.append(cur)
            continue
        m = re.search(r"remark:\s+([A-Za-z ]+?)(?: \[[^\]]*\])?: (\S+) \[-Rpass", line)
        if m and cur is not None:
            key = {"VGPRs": "vgprs", "AGPRs": "agprs", "ScratchSize": "scratch",
                   "Occupancy": "occupancy", "LDS Size": "lds", "TotalSGPRs": "sgprs"}.get(
                       m.group(1).strip())
            if key:
                cur[key] = int(m.group(2)) if m.group(2).isdigit() else m.group(2)
    return out


def _compile(src: Path, build_dir: Path = BUILD, defines: tuple = ()) -> tuple[Path, list]:
    obj = build_dir / (src.stem + ".o")
    cmd = [HIPCC, *COMPILE_FLAGS, "-Rpass-analysis=kernel-resource-usage",
           *[f"-D{d}" for d in defines], "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    return obj, _remarks(proc.stderr, src.name)


def _demangle(records: list[dict]) -> None:
    names = [r["mangled"] for r in records]
    try:
        proc = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True,
                              text=True, check=True)
        dem = proc.stdout.split("\n")
    except (OSError, subprocess.CalledProcessError):
        dem = names
    for r, d in zip(records, dem):
        r["kernel"] = d


def check_resources(records: list[dict]) -> list[str]:
    """Problems with the compiled kernels' resources (empty = fine):
    - a multi-pass kernel (k_*_wide) that spills (they are launched without a resource check);
    - a kernel built with the four-waves request that spills or misses four waves per SIMD;
    - no kernel matching one of those requests (a renamed kernel would escape the check).
    Register-resident kernels may spill at 8 or 16 vectors per lane: the launch code skips
    spilling kernels and sends such rows to the operator's multi-pass kernel."""
    bad = []
    for r in records:
        k = r.get("kernel", r["mangled"])
        if "_wide<" in k and r.get("scratch", 0) != 0:
            bad.append(f"multi-pass kernel spills {r['scratch']} B/lane: {k}")
    for pat in FOUR_WAVE_KERNELS:
        hits = [r for r in records if re.search(pat, r.get("kernel", ""))]
        if not hits:
            bad.append(f"no kernel matches the four-waves pattern {pat}")
        for r in hits:
            if r.get("scratch", 0) != 0 or r.get("occupancy", 0) < 4:
                bad.append(f"four-waves kernel spills {r.get('scratch')} B/lane or runs "
                           f"{r.get('occupancy')} waves/SIMD: {r['kernel']}")
    return bad


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
        done = list(ex.map(lambda s: _compile(s, build_dir, defines), srcs))
    objs = [o for o, _ in done]
    records = [r for _, rs in done for r in rs]
    _demangle(records)
    (build_dir / RESOURCES).write_text(json.dumps(records, indent=0))
    problems = check_resources(records)
    if problems:
        raise RuntimeError("kernel resource check failed:\n  " + "\n  ".join(problems))
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
