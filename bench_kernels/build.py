"""Build bench_kernels/libmcop_pattern.so: the compute-free access-pattern kernels (and the empty
kernel) that bench.py times beside the operators.  Measurement tooling, not part of the operator
library: it shares the operators' device helpers (mcoplib_amd/csrc/rowkern.h) and their hipcc
flags (mcoplib_amd/_build.py), and fails if a pattern kernel spills registers.

Usage: python bench_kernels/build.py   (also run by __graft_entry__.build())
"""

from __future__ import annotations

import importlib.util
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
LIB = HERE / "libmcop_pattern.so"
BUILD = HERE / "_build"


def _package_build():
    # loaded by path: importing mcoplib_amd would load the operator library
    spec = importlib.util.spec_from_file_location("mcoplib_amd_build",
                                                  ROOT / "mcoplib_amd" / "_build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def build(verbose: bool = True) -> Path:
    """Compile pattern.hip for gfx950 and link libmcop_pattern.so next to it (always rebuilds)."""
    pb = _package_build()
    BUILD.mkdir(parents=True, exist_ok=True)
    obj, records = pb._compile(HERE / "pattern.hip", BUILD)
    pb._demangle(records)
    spills = [r["kernel"] for r in records if r.get("scratch", 0) != 0]
    if spills:
        raise RuntimeError("pattern kernels spill: " + "; ".join(spills))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [pb.HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", f"-Wl,-soname,{LIB.name}",
           "-o", str(tmp), str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
