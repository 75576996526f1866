#!/usr/bin/env python3
"""Benchmark of the fused add + RMSNorm + per-token quantization path on one MI355X.

Headline workload ("cfg3"): x and residual bf16 [8192, 8192] (1% of channels scaled x20 as
outliers), weight bf16 ~N(1, 0.1), eps 1e-5; output int8 [8192, 8192] + fp32 scales [8192, 1] +
the bf16 residual written in place.  One step = one call of
mcoplib.op.rms_norm_dynamic_per_token_quant_custom (one kernel launch) over one batch already
resident in HBM; copies of the input are rotated so consecutive steps do not hit the 256 MB
last-level cache.

The default run prints ONE JSON line: the headline (value = algorithmic GB/s, bytes = every
input read once + every output written once) with
  - roofline: the kernel's average launch time from HIP events around the timed launches, next
    to the rocprofv3 kernel-trace mean and the HBM traffic of the committed profile summary;
  - guard: whether the headline stays at >= 75% of peak with traffic <= 1.01x the algorithmic
    bytes, measured by a profile taken on the current kernel sources (`regressed` true when
    not, `profile_stale` true when the profile's recorded source hash differs);
  - device_copy / ceilings: a non-temporal streaming copy, read-only and write-only kernels, and
    compute-free kernels with each timed operator's exact access pattern
    (bench_kernels/libmcop_pattern.so), also run over the same elements reshaped to 2048-wide
    rows (the operator's traffic mix at the fastest streaming shape);
  - cpu_baseline / cpu_torch: the C oracle and a vectorized torch restatement on a row sample of
    the same inputs, on this host's cores, with a bit-for-bit check of the GPU's first call;
  - configs: the other configurations -- cfg1 (CPU only), cfg2, cfg4, cfg5 large (GB/s, fraction
    of peak, traffic, pattern ceiling, CPU baseline, parity of the sampled rows), cfg5 decode
    (us per call in fixed batches, eager and replayed from a HIP graph, beside the empty kernel
    and the compute-free pattern at the same launch shape), and published_h1: the reference's
    one published measurement (fused_add_rms_norm, 1024 x 512 fp16) timed at its own shape.
Every configuration's inputs are generated on the CPU from torch.Generator().manual_seed(k) for
configuration k and copied to the GPU, so the GPU, the oracle and the torch legs see the same bits
(and the parity tests build the same inputs: tests import `config_inputs`).

  python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--workload cfg3] [--no-configs] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
HBM_PEAK_GBS = 8000.0
METRIC = "HBM GB/s & % of peak: fused add-RMSNorm+per-token int8 quant, 8192x8192"
FRAC_GUARD, TRAFFIC_GUARD = 0.75, 1.01
PAD_SIZE = 3840  # padded workload: bf16 elements per padded row (2 * 3840 bytes)
BLOCK_GROUP = 128  # block-fp8 workload: elements per scale group
HEADS = 8  # head-norm workload: heads per token (all normalized, per-head weights)
DECODE_T = (1, 4, 16, 64)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="cfg3", choices=sorted(WORKLOADS))
    ap.add_argument("--sets", type=int, default=0,
                    help="rotated input copies (default: enough for > 1 GiB, at least 3)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU legs")
    ap.add_argument("--no-configs", action="store_true",
                    help="time the chosen workload only (no other configs, ceilings or copy)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="CPU time of the headline's CPU legs (the other configs take a third)")
    ap.add_argument("--warmup-seconds", type=float, default=2.0)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run three 1 GiB device-to-device copies (a kernel of known "
                         "traffic, used to scale rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    ap.add_argument("--multi-pass", action="store_true",
                    help="run rows wider than the registers on the multi-pass kernels (the "
                         "split-row kernels' fallback under graph capture), for comparison")
    ap.add_argument("--pattern", default=None, choices=["natural", "4", "3", "2"],
                    help="time only the workload's compute-free access-pattern kernel, at its "
                         "natural occupancy or capped to 4, 3 or 2 workgroups per CU (for "
                         "profiling the ceilings on their own); prints one JSON line")
    return ap.parse_args()


# ------------------------------------------------------------------------------ inputs
def config_inputs(name: str) -> dict:
    """Seeded CPU inputs of a configuration (bf16 unless stated; torch.Generator seeded with the
    configuration number, draws in the order listed):
      cfg1        x [256, 4096] ~N(0,1); w [4096] ~N(1, 0.1); no residual; eps 1e-6
      cfg2        x, r [4096, 4096]; w; eps 1e-6
      cfg3        82 = round(1% of 8192) outlier channels idx = randperm(8192)[:82];
                  x [8192, 8192] ~N(0,1) with x[:, idx] *= 20 before the bf16 cast; r; w; eps 1e-5
      cfg4        x [16384, 7168]; w; smooth fp32 [7168] ~U(0.5, 2); eps 1e-6
      cfg5-decodeT x, r [T, 5120] (T in 1, 4, 16, 64); w; eps 1e-6
      cfg5-large  x, r [32768, 16384]; w; eps 1e-6
      published-h1 x, r, w fp16 [1024, 512] (seed 6): the shape of the reference's only
                  published measurement (fused_add_rms_norm, mxbench/README_MXBENCH.md:160-177)
    Returns a dict of CPU tensors (x, r or None, w, sm or None) and eps."""
    import torch

    spec = {"cfg1": (1, 256, 4096, False, 1e-6), "cfg2": (2, 4096, 4096, True, 1e-6),
            "cfg3": (3, 8192, 8192, True, 1e-5), "cfg4": (4, 16384, 7168, False, 1e-6),
            "cfg5-large": (5, 32768, 16384, True, 1e-6),
            **{f"cfg5-decode{t}": (5, t, 5120, True, 1e-6) for t in DECODE_T},
            "published-h1": (6, 1024, 512, True, 1e-6)}
    seed, T, H, res, eps = spec[name]
    dt = torch.float16 if name == "published-h1" else torch.bfloat16
    g = torch.Generator().manual_seed(seed)
    idx = torch.randperm(H, generator=g)[: round(0.01 * H)] if name == "cfg3" else None
    x = torch.randn(T, H, generator=g)
    if idx is not None:
        x[:, idx] *= 20.0
    x = x.to(dt)
    r = torch.randn(T, H, generator=g).to(dt) if res else None
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(dt)
    sm = (0.5 + 1.5 * torch.rand(H, generator=g)) if name == "cfg4" else None
    return {"x": x, "r": r, "w": w, "sm": sm, "eps": eps}


# ------------------------------------------------------------------------------ workloads
class Workload:
    """Inputs, a launcher and the byte model of one benchmark configuration."""

    def __init__(self, name, T, H, eps, kind):
        self.name, self.T, self.H, self.eps, self.kind = name, T, H, eps, kind

    @property
    def seeded(self) -> bool:
        """Inputs come from config_inputs (the configurations and the reference's published
        shape) rather than the device RNG."""
        return self.name.startswith("cfg") or self.name == "published-h1"

    @property
    def pad(self) -> int:
        """Padded row size in bf16 elements (padded workloads): PAD_SIZE, or enough for H + 4."""
        return PAD_SIZE if 2 * PAD_SIZE >= self.H + 4 else (self.H + 4 + 63) // 64 * 32

    @property
    def bytes(self) -> int:
        return self.bytes_for(self.T)

    def bytes_for(self, T: int) -> int:
        H = self.H
        if self.kind == "add_norm_int8":   # read x, r (2H each), w; write r (2H), q (H), s
            return 7 * T * H + 2 * H + 4 * T
        if self.kind == "norm_int8":       # read x, w; write q, s
            return 3 * T * H + 2 * H + 4 * T
        if self.kind == "fused_add":       # read x, r; write x, r; read w
            return 8 * T * H + 2 * H
        if self.kind == "smooth_fp8":      # read x; write q, after_res, after_norm; w, smooth, s
            return 2 * T * H + T * H + 4 * T * H + 2 * H + 4 * H + 4 * T
        if self.kind == "sdq":             # read h, smooth (fp32); write q, s
            return 3 * T * H + 4 * H + 4 * T
        if self.kind in ("ptq_int8", "ptq_fp8"):  # read x; write q, s
            return 3 * T * H + 4 * T
        if self.kind == "ptq_int8_azp":    # read x; write q, s, azp
            return 3 * T * H + 8 * T
        if self.kind == "padded":          # read x, r; write r, rms, q, padded q + scale, s; w
            return 10 * T * H + 8 * T + 2 * H
        if self.kind == "block_fp8":       # read x, r, w; write r, q, one scale per group
            return 7 * T * H + 2 * H + 4 * T * (H // BLOCK_GROUP)
        if self.kind == "norm_res":        # read x, r, w; write out, after_res
            return 8 * T * H + 2 * H
        if self.kind == "vllm_norm":       # read x, w; write out
            return 4 * T * H + 2 * H
        if self.kind == "head_norm":       # T rows of HEADS heads: read x, per-head w; write out
            return 4 * T * H + 2 * HEADS * H
        raise ValueError(self.kind)

    def device_sets(self, torch, dev, n_sets, cpu=None):
        """n_sets input sets on the device: copies of the seeded CPU inputs for the
        configurations (rotation only changes addresses), device-RNG draws otherwise."""
        if self.seeded:
            cpu = cpu or config_inputs(self.name)
            return [self._alloc(torch, dev, {k: (v.to(dev) if hasattr(v, "to") and v is not None
                                                 else v) for k, v in cpu.items()})
                    for _ in range(n_sets)]
        return [self._alloc(torch, dev, self._draw(torch, dev, 100 + i)) for i in range(n_sets)]

    def _draw(self, torch, dev, seed):
        T, H = self.T, self.H
        g = torch.Generator(device=dev).manual_seed(seed)
        x = torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16)
        w = (1 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
        d = {"x": x, "w": w, "r": None, "sm": None}
        if self.kind == "head_norm":       # x [T/HEADS tokens, HEADS, H], per-head weights
            d["x"] = x.view(T // HEADS, HEADS, H)
            d["w"] = (1 + 0.1 * torch.randn(HEADS, H, generator=g, device=dev)).to(torch.bfloat16)
        if self.kind in ("add_norm_int8", "fused_add", "padded", "block_fp8", "norm_res"):
            d["r"] = torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16)
        if self.kind in ("sdq", "smooth_fp8"):
            d["sm"] = 0.5 + 1.5 * torch.rand(H, generator=g, device=dev)
        return d

    def _alloc(self, torch, dev, d):
        """Output buffers of one set."""
        T, H, x = self.T, self.H, d["x"]
        if self.kind in ("norm_res", "vllm_norm", "head_norm"):
            d["out"] = torch.empty_like(x)
        if self.kind in ("add_norm_int8", "norm_int8"):
            d["q"] = torch.empty(T, H, dtype=torch.int8, device=dev)
            d["s"] = torch.empty(T, 1, dtype=torch.float32, device=dev)
        if self.kind == "block_fp8":
            d["q"] = torch.empty(T, H, dtype=torch.float8_e4m3fn, device=dev)
            d["s"] = torch.empty(T, H // BLOCK_GROUP, dtype=torch.float32, device=dev)
        if self.kind == "padded":
            d["p"] = torch.empty(T, 2 * self.pad, dtype=torch.int8, device=dev)
            d["rms"] = torch.empty_like(x)
            d["q"] = torch.empty(T, H, dtype=torch.int8, device=dev)
            d["s"] = torch.empty(T, 1, dtype=torch.float32, device=dev)
        if self.kind.startswith("ptq_"):
            qdt = torch.float8_e4m3fn if self.kind == "ptq_fp8" else torch.int8
            d["q"] = torch.empty(T, H, dtype=qdt, device=dev)
            d["s"] = torch.empty(T, 1, dtype=torch.float32, device=dev)
            d["azp"] = (torch.empty(T, 1, dtype=torch.int32, device=dev)
                        if self.kind == "ptq_int8_azp" else None)
        if self.kind == "smooth_fp8":
            d["q"] = torch.empty(T, H, dtype=torch.float8_e4m3fn, device=dev)
            d["s"] = torch.empty(T, dtype=torch.float32, device=dev)
            d["ar"] = torch.empty_like(x)
            d["an"] = torch.empty_like(x)
        return d

    def launcher(self, torch, d):
        from mcoplib import op
        import mcoplib._C  # noqa: F401
        if self.kind == "add_norm_int8":
            return lambda: op.rms_norm_dynamic_per_token_quant_custom(
                d["q"], d["x"], d["w"], d["s"], self.eps, None, d["r"])
        if self.kind == "norm_int8":
            return lambda: torch.ops._C.rms_norm_dynamic_per_token_quant(
                d["q"], d["x"], d["w"], d["s"], self.eps, None, None)
        if self.kind == "fused_add":
            return lambda: torch.ops._C.fused_add_rms_norm(d["x"], d["r"], d["w"], self.eps)
        if self.kind == "norm_res":
            d["ares"] = torch.empty_like(d["x"])
            return lambda: op.rms_norm(d["out"], d["x"], d["w"], self.eps, d["ares"], d["r"], True)
        if self.kind == "vllm_norm":
            return lambda: torch.ops._C.rms_norm(d["out"], d["x"], d["w"], self.eps)
        if self.kind == "head_norm":
            return lambda: op.head_rms_norm(d["out"], d["x"], d["w"], self.eps, 0, HEADS)
        if self.kind == "block_fp8":
            return lambda: torch.ops._C.rms_norm_per_block_quant(
                d["q"], d["x"], d["w"], d["s"], self.eps, None, d["r"], BLOCK_GROUP, False)
        if self.kind == "padded":
            return lambda: op.fused_add_rms_norm_dynamic_per_token_quant_padding_output(
                d["p"], d["rms"], d["q"], d["s"], d["x"], d["r"], d["w"], self.pad, self.eps)
        if self.kind == "sdq":  # returns new tensors, as the reference's op does
            return lambda: op.scale_dynamic_quant(d["x"], d["sm"], torch.int8)
        if self.kind == "ptq_fp8":
            return lambda: torch.ops._C.dynamic_per_token_scaled_fp8_quant(d["q"], d["x"], d["s"],
                                                                         None)
        if self.kind.startswith("ptq_int8"):
            return lambda: torch.ops._C.dynamic_scaled_int8_quant(d["q"], d["x"], d["s"], d["azp"])
        return lambda: op.rms_norm_dynamic_per_token_quant(
            d["q"], d["x"], d["w"], d["sm"], d["s"], self.eps, d["ar"], d["an"], None)


WORKLOADS = {
    "cfg1": Workload("cfg1", 256, 4096, 1e-6, "norm_int8"),
    "cfg2": Workload("cfg2", 4096, 4096, 1e-6, "fused_add"),
    "cfg3": Workload("cfg3", 8192, 8192, 1e-5, "add_norm_int8"),
    "cfg4": Workload("cfg4", 16384, 7168, 1e-6, "smooth_fp8"),
    "cfg5-large": Workload("cfg5-large", 32768, 16384, 1e-6, "add_norm_int8"),
    **{f"cfg5-decode{t}": Workload(f"cfg5-decode{t}", t, 5120, 1e-6, "add_norm_int8")
       for t in DECODE_T},
    # the reference's only published measurement: fused_add_rms_norm, 1024 x 512 fp16
    # (mxbench/README_MXBENCH.md:160-177; byte model benchmark/fused_add_rms_norm_simple.py:57-61,
    # 8TH + 2H = 4,195,328 B, the same as this workload's)
    "published-h1": Workload("published-h1", 1024, 512, 1e-6, "fused_add"),
    # the standalone quantizers, at the headline shape (the step after an unfused norm)
    "ptq-int8": Workload("ptq-int8", 8192, 8192, 0.0, "ptq_int8"),
    "ptq-int8-azp": Workload("ptq-int8-azp", 8192, 8192, 0.0, "ptq_int8_azp"),
    "ptq-fp8": Workload("ptq-fp8", 8192, 8192, 0.0, "ptq_fp8"),
    # the padded wire format at DeepSeek's width (H 7168, rows of 2 * 3840 bytes)
    "padded": Workload("padded", 8192, 7168, 1e-6, "padded"),
    # per-group (128) fp8 scales for block-scaled GEMMs, at the headline shape with residual
    "block-fp8": Workload("block-fp8", 8192, 8192, 1e-6, "block_fp8"),
    # RMSNorms without quantization: mcoplib rms_norm with residual (after_res), vLLM rms_norm,
    # and q/k head norm (T rows = tokens x heads of 128)
    "norm-res": Workload("norm-res", 8192, 8192, 1e-6, "norm_res"),
    "vllm-norm": Workload("vllm-norm", 8192, 8192, 1e-6, "vllm_norm"),
    "head-norm": Workload("head-norm", 65536 * 8, 128, 1e-6, "head_norm"),
    # the un-normed SmoothQuant sibling (scale_dynamic_quant) at SmoothQuant's shape
    "sdq": Workload("sdq", 16384, 7168, 0.0, "sdq"),
    # rows wider than the registers hold: the split-row kernels of H1, H2/H3, H4 and H5 (the row
    # shared by several workgroups, read once), each other operator's multi-pass kernel
    "wide-int8": Workload("wide-int8", 2048, 131072, 1e-6, "add_norm_int8"),
    "wide-fused": Workload("wide-fused", 2048, 131072, 1e-6, "fused_add"),
    "wide-fp8": Workload("wide-fp8", 2048, 131072, 1e-6, "smooth_fp8"),
    "wide-sdq": Workload("wide-sdq", 2048, 131072, 0.0, "sdq"),
    "wide-norm": Workload("wide-norm", 2048, 131072, 1e-6, "norm_res"),
    "wide-ptq": Workload("wide-ptq", 2048, 131072, 0.0, "ptq_int8"),
    "wide-padded": Workload("wide-padded", 2048, 131072, 1e-6, "padded"),
    "wide-block": Workload("wide-block", 2048, 131072, 1e-6, "block_fp8"),
}
KERNEL_NAME = {"add_norm_int8": "k_rms_norm_quant", "norm_int8": "k_rms_norm_quant",
               "fused_add": "k_fused_add_rms_norm",
               "smooth_fp8": "k_rms_norm_smooth_quant", "ptq_int8": "k_per_token_quant",
               "ptq_int8_azp": "k_per_token_quant", "ptq_fp8": "k_per_token_quant",
               "padded": "k_add_rms_norm_quant_padded", "block_fp8": "k_rms_norm_group_quant",
               "norm_res": "k_rms_norm", "vllm_norm": "k_rms_norm", "head_norm": "k_rms_norm",
               "sdq": "k_scale_dynamic_quant"}


# kinds whose wide rows take a split-row kernel (the others a multi-pass kernel); --multi-pass
# sends them to the multi-pass kernels too
SPLIT_KINDS = {"add_norm_int8", "fused_add", "smooth_fp8", "sdq", "norm_res", "vllm_norm",
               "ptq_int8", "ptq_int8_azp", "ptq_fp8", "padded", "block_fp8"}
MULTI_PASS = False


def kernel_name(wl) -> str:
    if not wl.name.startswith("wide-"):
        return KERNEL_NAME[wl.kind]
    split = wl.kind in SPLIT_KINDS and not MULTI_PASS
    return KERNEL_NAME[wl.kind] + ("_split" if split else "_wide")


# Compute-free kernels with a configuration's access pattern (bench_kernels/mcop_pattern.h), at the
# launch shape the operator picks for it (vectors per lane, lanes per row).
PATTERN_OF = {"cfg2": (1, 2, 256), "cfg3": (0, 2, 512), "cfg4": (2, 4, 256),
              "cfg5-large": (0, 4, 512)}
PATTERN_COPY, PATTERN_READ, PATTERN_WRITE, PATTERN_EMPTY, PATTERN_EXACT = 3, 4, 5, 6, 7
MIX_H = 2048  # row width of the reshaped ("mix") pattern: one 16-byte vector a lane, 256 lanes
# LDS of a CU (bytes): a pattern launched with LDS_PER_CU // n - 1024 bytes of unused dynamic LDS
# per workgroup (the 1 KiB margin covers the kernel's own reduction slots) has at most n
# workgroups on a CU
LDS_PER_CU = 163840


# ------------------------------------------------------------------------------ profiles
# The files whose text decides each kernel's code: its translation units (mcoplib_amd/csrc), the
# device helpers and the launch-shape choice every kernel shares, and the hipcc flags.  A
# profile summary records the hash of these at the time it was taken (kernel_source_sha16), so
# a figure measured on other code is reported as stale instead of vouching for the current one.
KERNEL_SOURCES = {
    "k_rms_norm_quant": ["rms_norm_quant.hip"],
    "k_fused_add_rms_norm": ["fused_add_rms_norm.hip"],
    "k_rms_norm_smooth_quant": ["smooth_quant_kernel.h", "rms_norm_smooth_quant.hip",
                                "rms_norm_smooth_quant_bf16.hip", "rms_norm_smooth_quant_f16.hip"],
    "k_scale_dynamic_quant": ["scale_dynamic_quant.hip"],
    "k_per_token_quant": ["per_token_quant.hip"],
    "k_add_rms_norm_quant_padded": ["padded_quant.hip"],
    "k_rms_norm_group_quant": ["group_quant.hip"],
    "k_rms_norm": ["norm_kernel.h", "rms_norm.hip", "rms_norm_bf16.hip", "rms_norm_f16.hip"],
}
SHARED_SOURCES = ["rowkern.h", "numerics.h", "abi.hip", "split_row.h"]


def kernel_source_hash(kernel: str, root: Path = ROOT) -> str:
    """First 16 hex digits of the SHA-256 over a kernel's source files (name and text, in name
    order) and the hipcc flags of mcoplib_amd/_build.py (`kernel` may carry the _wide or _split
    suffix of the multi-pass or split-row form, which live in the same files)."""
    import hashlib

    base = re.sub(r"_(wide|split)$", "", kernel)
    h = hashlib.sha256()
    for name in sorted(KERNEL_SOURCES[base] + SHARED_SOURCES):
        h.update(name.encode() + b"\0")
        h.update((root / "mcoplib_amd" / "csrc" / name).read_bytes())
    build = (root / "mcoplib_amd" / "_build.py").read_text()
    flags = re.search(r"^COMPILE_FLAGS = \[.*?^\]", build, re.M | re.S)
    h.update(flags.group(0).encode() if flags else b"")
    return h.hexdigest()[:16]


def profile_summary(wl: Workload, root: Path = ROOT):
    """Figures of the committed rocprofv3 summary profiles/<kernel>_<workload>.txt: HBM bytes per
    dispatch (FETCH_SIZE + WRITE_SIZE passes, each scaled by a copy kernel's reading), the
    kernel-trace mean of the timed launches, and whether the summary was taken on the current
    sources (`stale`: its recorded kernel_source_sha16 differs from the current hash, or it has
    none); None where absent."""
    p = root / "profiles" / f"{kernel_name(wl)}_{wl.name}.txt"
    if not p.exists():
        return None
    t = p.read_text()
    m = re.search(r"^hbm_bytes_per_dispatch:\s*([0-9.eE+]+)", t, re.M)
    k = re.search(r"^timed legs \((\d+) dispatches\): mean ([0-9.]+) us", t, re.M)
    h = re.search(r"^kernel_source_sha16:\s*([0-9a-f]{16})\s*$", t, re.M)
    current = kernel_source_hash(kernel_name(wl), root)
    return {"file": str(p.relative_to(root)),
            "hbm_bytes_per_dispatch": float(m.group(1)) if m else None,
            "trace_mean_us": float(k.group(2)) if k else None,
            "source_sha16": h.group(1) if h else None, "current_source_sha16": current,
            "stale": h is None or h.group(1) != current}


def guard_of(frac: float, prof, traffic_bytes: int) -> dict:
    """The headline's regression guard: `regressed` when the fraction of the 8 TB/s peak falls
    under FRAC_GUARD, when the committed profile's traffic exceeds TRAFFIC_GUARD times the
    algorithmic bytes, or when that profile is missing or stale (taken on other sources, so its
    traffic figure says nothing about the code that ran)."""
    tr = (round(prof["hbm_bytes_per_dispatch"] / traffic_bytes, 4)
          if prof and prof["hbm_bytes_per_dispatch"] else None)
    stale = prof is None or prof["stale"]
    return {"frac_min": FRAC_GUARD, "traffic_ratio_max": TRAFFIC_GUARD, "frac": frac,
            "traffic_ratio": tr, "profile_stale": stale,
            "profile_source_sha16": prof["source_sha16"] if prof else None,
            "current_source_sha16": prof["current_source_sha16"] if prof else None,
            "regressed": bool(frac < FRAC_GUARD or tr is None or tr > TRAFFIC_GUARD or stale)}


# ------------------------------------------------------------------------------ GPU timing
def _ev(torch):
    return torch.cuda.Event(enable_timing=True)


def time_launches(torch, launches, K, warmup, warmup_seconds):
    """Warm up (the requested launches, continued until the GPU has been busy for
    `warmup_seconds`), then time K back-to-back launches between two HIP events on torch's
    current stream (the stream the operators launch on).  Returns (ms per launch, host seconds)."""
    i, t_w = 0, time.perf_counter()
    while i < warmup or time.perf_counter() - t_w < warmup_seconds:
        launches[i % len(launches)]()
        i += 1
        if i % 64 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    e0, e1 = _ev(torch), _ev(torch)
    t0 = time.perf_counter()
    e0.record()
    for i in range(K):
        launches[i % len(launches)]()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / K, time.perf_counter() - t0


def graph_us(torch, launches, K):
    """us per call of the same K launches replayed from a HIP graph (best of 5 replays)."""
    g = torch.cuda.CUDAGraph()
    s_cap = torch.cuda.Stream()
    s_cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s_cap):
        with torch.cuda.graph(g, stream=s_cap):
            for i in range(K):
                launches[i % len(launches)]()
    torch.cuda.current_stream().wait_stream(s_cap)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(5):
        e0, e1 = _ev(torch), _ev(torch)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / K)
    return best


class Pattern:
    """ctypes binding of bench_kernels/libmcop_pattern.so (compute-free access-pattern kernels
    and an empty kernel; bench_kernels/mcop_pattern.h)."""

    def __init__(self):
        import ctypes
        path = ROOT / "bench_kernels" / "libmcop_pattern.so"
        if not path.exists():
            raise RuntimeError(f"{path} is not built (python bench_kernels/build.py)")
        self.lib = ctypes.CDLL(str(path))
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        self.lib.mcop_pattern.argtypes = [I, P, P, P, P, P, P, P, P, I64, I64, I, I, I, P]
        self.lib.mcop_pattern.restype = I
        self.lib.mcop_pattern_last_error.restype = ctypes.c_char_p

    def launcher(self, torch, pattern, d, T, H, nv, tpr, lds=0):
        """A launch of `pattern` on torch's current stream at call time (so it can be captured
        into a HIP graph like the operators)."""
        def p(t):
            return None if t is None else t.data_ptr()
        args = (pattern, p(d.get("x")), p(d.get("r")), p(d.get("w")), p(d.get("sm")),
                p(d.get("o0")), p(d.get("o1")), p(d.get("q")), p(d.get("s")), T, H, nv, tpr, lds)

        def run():
            rc = self.lib.mcop_pattern(*args, torch.cuda.current_stream().cuda_stream)
            if rc != 0:
                raise RuntimeError(self.lib.mcop_pattern_last_error().decode())
        return run


def pattern_us(torch, pat, pattern, T, H, nv, tpr, dev, K, with_w=False, with_sm=False, lds=0):
    """us per launch of a pattern kernel over [T, H] bf16 tensors (rotated copies to defeat the
    last-level cache), at the given launch shape (and `lds` bytes of LDS per workgroup)."""
    per_set = T * H * 7
    n_sets = max(2, -(-(1 << 30) // per_set))
    sets = []
    for _ in range(n_sets):
        d = {"x": torch.zeros(T, H, dtype=torch.bfloat16, device=dev),
             "r": torch.zeros(T, H, dtype=torch.bfloat16, device=dev),
             "o0": torch.empty(T, H, dtype=torch.bfloat16, device=dev),
             "o1": torch.empty(T, H, dtype=torch.bfloat16, device=dev),
             "q": torch.empty(T, H, dtype=torch.uint8, device=dev),
             "s": torch.empty(T, dtype=torch.float32, device=dev)}
        if pattern == 1:  # in place, as the operator writes x and r
            d["o0"], d["o1"] = d["x"], d["r"]
        if with_w:
            d["w"] = torch.ones(H, dtype=torch.bfloat16, device=dev)
        if with_sm:
            d["sm"] = torch.ones(H, dtype=torch.float32, device=dev)
        sets.append(d)
    launches = [pat.launcher(torch, pattern, d, T, H, nv, tpr, lds) for d in sets]
    ms, _ = time_launches(torch, launches, K, 5, 0.3)
    del sets, launches
    torch.cuda.empty_cache()
    return ms * 1e3


def mix_us(torch, pat, wl: Workload, dev, K):
    """us per launch of a configuration's pattern kernel over the same elements reshaped to
    MIX_H-wide rows, at one vector a lane and 256 lanes (the shape at which the streaming kernels
    run fastest): the same input and output streams and per-row reductions, with the smallest
    workgroup footprint.  No row kernel of the configuration's width can have that footprint (a
    row's reductions need the whole row in one workgroup), so this bounds what any launch shape of
    a one-pass kernel could reach on the configuration's traffic mix."""
    p = PATTERN_OF[wl.name][0]
    return pattern_us(torch, pat, p, wl.T * wl.H // MIX_H, MIX_H, 1, 256, dev, K, with_w=True,
                      with_sm=wl.kind == "smooth_fp8")


# ------------------------------------------------------------------------------ CPU legs
def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def _time_cpu(fn, seconds, min_runs=3):
    fn()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < min_runs:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def oracle_call(wl: Workload, c: dict):
    """The C oracle (oracle/mcop_oracle.c) on the rows in c: the operation the workload's GPU
    launch performs.  Returns its outputs in the order the GPU check compares them."""
    import torch
    import oracle  # CPU baseline leg only
    if wl.kind == "add_norm_int8":
        q, s, r = oracle.rms_norm_dynamic_per_token_quant_custom(c["x"], c["w"], wl.eps,
                                                                 residual=c["r"])
        return {"q": q, "s": s, "r": r}
    if wl.kind == "norm_int8":
        q, s, _ = oracle.rms_norm_dynamic_per_token_quant(c["x"], c["w"], wl.eps, torch.int8)
        return {"q": q, "s": s}
    if wl.kind == "fused_add":
        x, r = oracle.fused_add_rms_norm(c["x"], c["r"], c["w"], wl.eps)
        return {"x": x, "r": r}
    if wl.kind == "smooth_fp8":
        q, s, ar, an = oracle.rms_norm_smooth_quant(c["x"], c["w"], c["sm"], wl.eps,
                                                    torch.float8_e4m3fn)
        return {"q": q, "s": s, "ar": ar, "an": an}
    raise ValueError(wl.kind)


def cpu_baseline(wl: Workload, cpu: dict, rows: int, seconds: float, gpu_out=None,
                 threads=None) -> dict:
    """The C oracle (OpenMP over rows) on the first `rows` rows of the workload's seeded inputs,
    on this host's cores (or `threads`), in the metric's unit; with gpu_out (the GPU's outputs of
    its first call on the same rows) also whether the GPU matched it bit for bit."""
    import torch
    import oracle  # CPU baseline leg only

    cores = threads or len(os.sched_getaffinity(0))
    oracle.set_threads(cores)
    c = {k: (v[:rows] if (torch.is_tensor(v) and v.dim() == 2) else v) for k, v in cpu.items()}
    med, n = _time_cpu(lambda: oracle_call(wl, c), seconds, 5)
    oracle.set_threads(len(os.sched_getaffinity(0)))  # the OpenMP runtime may be torch's too
    out = {"value": round(wl.bytes_for(rows) / med / 1e9, 3), "unit": "GB/s", "cores": cores,
           "kind": "port", "us_per_call": round(med * 1e6, 2),
           "sample": f"first {rows} of {wl.T} rows x {wl.H} of the same seeded inputs (same "
                     f"byte model), median of {n} runs over ~{seconds:.0f} s, "
                     f"oracle/mcop_oracle.c with {cores} OpenMP threads, {_cpu_model()}",
           "tokens_per_s": round(rows / med, 1)}
    if gpu_out is not None:
        n_chk = next(iter(gpu_out.values())).shape[0]
        ref = oracle_call(wl, {k: (v[:n_chk] if (torch.is_tensor(v) and v.dim() == 2) else v)
                               for k, v in cpu.items()})
        diffs = {}
        for k, g in gpu_out.items():
            a, b = g.view(-1), ref[k].reshape(-1)
            if a.dtype in (torch.bfloat16, torch.float16, torch.float8_e4m3fn):
                a, b = a.view(torch.uint8 if a.element_size() == 1 else torch.int16), \
                    b.view(torch.uint8 if b.element_size() == 1 else torch.int16)
            elif a.dtype == torch.float32:
                a, b = a.view(torch.int32), b.view(torch.int32)
            diffs[k] = int((a != b).sum())
        out["gpu_first_call_vs_oracle"] = {"rows": n_chk, "differing_values": diffs,
                                           "bit_exact": all(v == 0 for v in diffs.values())}
    return out


def torch_cpu_add_norm_int8(x, r, w, eps: float, floor=None, lo=-128):
    """(Residual add +) RMSNorm + per-token int8 restated in vectorized torch (the form of the
    reference's own torch-native test oracles), following the reference's rounding points
    (op/vllm/quantization/fused_kernels/layernorm_utils.cuh:245-276, 436-447, 503-531 and
    fused_layernorm_dynamic_per_token_quant.cu:37): residual b(x + r), rho on the unrounded sum,
    y = b(b(a * rho) * w), s = max(A / 127, floor), q = sat[lo, 127](rne(y * (1/s))).  The floor
    is FLT_EPSILON for vLLM's operator; mcoplib's own (op/rms_norm_dynamic_per_token_quant.cu,
    kernel/rms_norm_vllm.cuh:382 and kernel/utils.h:219-226) uses 1.5e-6 and lo = -127.
    r may be None (no residual).  Returns (q, s, residual or None)."""
    import torch

    bf, H = torch.bfloat16, x.shape[-1]
    floor = torch.finfo(torch.float32).eps if floor is None else floor
    a = x.float() + (r.float() if r is not None else 0.0)
    res = a.to(bf) if r is not None else None
    ss = (a.double() * a.double()).sum(-1, keepdim=True)
    rho = 1.0 / torch.sqrt((ss / H).float() + eps)
    y = ((a * rho).to(bf).float() * w.float()).to(bf).float()
    s = torch.clamp(y.abs().amax(-1, keepdim=True) / 127.0, min=floor)
    q = torch.round(y * (1.0 / s)).clamp(lo, 127).to(torch.int8)
    return q, s, res


def cpu_torch(wl: Workload, cpu: dict, rows: int, seconds: float):
    """torch_cpu_add_norm_int8 timed on this host (torch's intra-op threads) on the first `rows`
    rows of the seeded inputs, beside the C oracle (add_norm_int8 and norm_int8 kinds only)."""
    import torch

    if wl.kind == "add_norm_int8":
        fn = lambda: torch_cpu_add_norm_int8(cpu["x"][:rows], cpu["r"][:rows], cpu["w"],  # noqa
                                             wl.eps, floor=1.5e-6, lo=-127)
    elif wl.kind == "norm_int8":
        fn = lambda: torch_cpu_add_norm_int8(cpu["x"][:rows], None, cpu["w"], wl.eps)  # noqa
    else:
        return None
    torch.set_num_threads(len(os.sched_getaffinity(0)))
    med, n = _time_cpu(fn, seconds, 3)
    threads = torch.get_num_threads()
    return {"value": round(wl.bytes_for(rows) / med / 1e9, 3), "unit": "GB/s", "cores": threads,
            "us_per_call": round(med * 1e6, 2),
            "sample": f"first {rows} of {wl.T} rows x {wl.H} of the same seeded inputs, median "
                      f"of {n} runs over ~{seconds:.0f} s, vectorized torch on the CPU with "
                      f"{threads} intra-op threads (bench.py torch_cpu_add_norm_int8)",
            "tokens_per_s": round(rows / med, 1)}


# ------------------------------------------------------------------------------ one config
def first_call_outputs(torch, wl: Workload, d: dict, rows: int):
    """The outputs of one launch on a fresh set, first `rows` rows, on the CPU."""
    keys = {"add_norm_int8": ("q", "s", "r"), "norm_int8": ("q", "s"), "fused_add": ("x", "r"),
            "smooth_fp8": ("q", "s", "ar", "an")}[wl.kind]
    wl.launcher(torch, d)()
    torch.cuda.synchronize()
    return {k: d[k][:rows].cpu() for k in keys}


def measure(torch, wl: Workload, args, dev, cpu=None, check_rows=0, hot=True, warmup_s=None):
    """Time K launches of a workload over rotated input sets; returns a dict of figures (and
    the GPU's first-call outputs of `check_rows` rows when asked)."""
    K = args.steps
    # > 1 GiB of rotated copies for the bandwidth-bound shapes; decode-sized calls are latency
    # bound (their inputs sit in the caches whatever the rotation): three copies
    n_sets = args.sets or (3 if wl.T <= 256 else max(3, -(-(1 << 30) // wl.bytes)))
    if wl.seeded and cpu is None:
        cpu = config_inputs(wl.name)
    sets = wl.device_sets(torch, dev, n_sets, cpu)
    first = first_call_outputs(torch, wl, sets[0], check_rows) if check_rows else None
    launches = [wl.launcher(torch, d) for d in sets]
    ms, wall = time_launches(torch, launches, K, args.warmup,
                             args.warmup_seconds if warmup_s is None else warmup_s)
    res = {"ms": ms, "wall": wall, "sets": len(sets), "first": first}
    if hot:
        # single-launch spread (an event pair around every launch: also times the event
        # packets, so its mean sits above the back-to-back figure) and one set only (hot caches)
        ev = [(_ev(torch), _ev(torch)) for _ in range(K)]
        for i in range(K):
            ev[i][0].record()
            launches[i % len(launches)]()
            ev[i][1].record()
        torch.cuda.synchronize()
        per = sorted(a.elapsed_time(b) for a, b in ev)
        res["p10_p50_p90_us"] = [round(per[int(q * (K - 1))] * 1e3, 3) for q in (0.1, 0.5, 0.9)]
        h0, h1 = _ev(torch), _ev(torch)
        h0.record()
        for _ in range(K):
            launches[0]()
        h1.record()
        torch.cuda.synchronize()
        res["hot_ms"] = h0.elapsed_time(h1) / K
    if wl.T <= 256:
        res["graph_us"] = graph_us(torch, launches, K)
    del sets, launches
    torch.cuda.empty_cache()
    return res


def config_entry(torch, wl: Workload, args, dev, pat, entry: str):
    """The figures of one GPU configuration for the `configs` object."""
    cpu = config_inputs(wl.name)
    check = min(wl.T, 256)
    m = measure(torch, wl, args, dev, cpu, check_rows=check, hot=False, warmup_s=0.5)
    us = m["ms"] * 1e3
    gbs = wl.bytes / (m["ms"] * 1e-3) / 1e9
    out = {"entry": entry, "kernel": kernel_name(wl),
           "shape": [wl.T, wl.H], "algorithmic_bytes": wl.bytes, "us_per_call": round(us, 3),
           "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
           "tokens_per_s": round(wl.T / (m["ms"] * 1e-3), 1), "rotated_input_sets": m["sets"]}
    prof = profile_summary(wl)
    if prof:
        out["profile"] = prof["file"]
        out["rocprof_trace_mean_us"] = prof["trace_mean_us"]
        out["profile_stale"] = prof["stale"]
        if prof["hbm_bytes_per_dispatch"]:
            out["traffic_ratio"] = round(prof["hbm_bytes_per_dispatch"] / wl.bytes, 4)
    if pat is not None and wl.name in PATTERN_OF:
        p, nv, tpr = PATTERN_OF[wl.name]
        pus = pattern_us(torch, pat, p, wl.T, wl.H, nv, tpr, dev, args.steps, with_w=True,
                         with_sm=wl.kind == "smooth_fp8")
        out["pattern_us"] = round(pus, 3)
        out["kernel_vs_pattern"] = round(pus / us, 4)
        mus = mix_us(torch, pat, wl, dev, args.steps)
        out["mix_us"] = round(mus, 3)
        out["kernel_vs_mix"] = round(mus / us, 4)
        if wl.name == "cfg4":
            # cfg 4's compute-free pattern streams faster with fewer workgroups per CU (capped by
            # unused LDS) while the kernel, at four per CU by its registers, needs its waves to
            # hide its arithmetic: the pattern at the kernel's occupancy and below it
            caps = {}
            for per_cu in (4, 3):
                cu = pattern_us(torch, pat, p, wl.T, wl.H, nv, tpr, dev, args.steps,
                                with_w=True, with_sm=True, lds=LDS_PER_CU // per_cu - 1024)
                caps[f"{per_cu}_per_cu"] = {"us": round(cu, 3),
                                            "kernel_vs_pattern": round(cu / us, 4)}
            out["pattern_capped_occupancy"] = caps
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(wl, cpu, min(wl.T, 512), args.cpu_seconds / 3,
                                           m["first"])
    return out


# Latency-bound calls are timed in fixed batches, independent of --steps: DECODE_CALLS calls per
# batch, DECODE_BATCHES batches, the median batch reported with the fastest and slowest.
DECODE_CALLS, DECODE_BATCHES = 500, 7


def _batches(run_batch, batches=DECODE_BATCHES) -> dict:
    """us per call over `batches` runs of run_batch(): median, min and max (3 decimals)."""
    v = sorted(run_batch() for _ in range(batches))
    return {"median": round(v[len(v) // 2], 3), "min": round(v[0], 3), "max": round(v[-1], 3)}


def eager_batch(torch, launches, n=DECODE_CALLS):
    """A batch of n back-to-back eager launches between two events; returns us per call."""
    def run():
        torch.cuda.synchronize()
        e0, e1 = _ev(torch), _ev(torch)
        e0.record()
        for i in range(n):
            launches[i % len(launches)]()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / n
    return run


def graph_batch(torch, launches, n=DECODE_CALLS):
    """n launches captured into one HIP graph; each run replays it between two events and
    returns us per call."""
    g = torch.cuda.CUDAGraph()
    s_cap = torch.cuda.Stream()
    s_cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s_cap):
        with torch.cuda.graph(g, stream=s_cap):
            for i in range(n):
                launches[i % len(launches)]()
    torch.cuda.current_stream().wait_stream(s_cap)
    g.replay()
    torch.cuda.synchronize()

    def run():
        e0, e1 = _ev(torch), _ev(torch)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / n
    run.graph = g  # keep the graph alive with the closure
    return run


def decode_floor_launches(torch, pat, T, H, dev, n_sets=3):
    """Launchers of the decode floor kernels at the operator's exact-row launch shape (two
    vectors a lane over H/16 lanes, one row per workgroup): the empty kernel (the launch floor)
    and the compute-free add-norm-quant pattern in the exact-row form (loads of x, r, w; the
    residual store; two row reductions; codes and scale stores)."""
    nv, tpr = 2, H // 16
    sets = []
    for _ in range(n_sets):
        sets.append({"x": torch.zeros(T, H, dtype=torch.bfloat16, device=dev),
                     "r": torch.zeros(T, H, dtype=torch.bfloat16, device=dev),
                     "w": torch.ones(H, dtype=torch.bfloat16, device=dev),
                     "o0": torch.empty(T, H, dtype=torch.bfloat16, device=dev),
                     "q": torch.empty(T, H, dtype=torch.uint8, device=dev),
                     "s": torch.empty(T, dtype=torch.float32, device=dev)})
    empty = [pat.launcher(torch, PATTERN_EMPTY, {}, T, H, nv, tpr)]
    exact = [pat.launcher(torch, PATTERN_EXACT, d, T, H, nv, tpr) for d in sets]
    return empty, exact, sets


def decode_entry(torch, args, dev, pat):
    """cfg5 decode, T in DECODE_T at H = 5120: us per call in fixed batches (eager: back-to-back
    calls through the operator surface; graph: the same calls replayed from a HIP graph), next to
    the floor of what one such call can cost on this GPU -- the empty kernel at the operator's
    launch shape and the compute-free exact-row pattern of its loads, reductions and stores, both
    graph-replayed the same way -- and the C oracle on one thread.  The batches of every shape and
    kind are interleaved (round r runs batch r of each), so slow phases of the host affect every
    figure alike rather than whichever shape was running."""
    out = {"entry": "mcoplib.op.rms_norm_dynamic_per_token_quant_custom with residual",
           "hidden": 5120, "timing": f"{DECODE_BATCHES} interleaved batches of {DECODE_CALLS} "
                                     "calls per figure, median batch (min, max) in us per call",
           "launch_shape": "two 16-byte vectors a lane, 320 lanes, one row per workgroup"}
    runs, keep = {}, []
    for t in DECODE_T:
        wl = WORKLOADS[f"cfg5-decode{t}"]
        cpu = config_inputs(wl.name)
        sets = wl.device_sets(torch, dev, 3, cpu)
        first = first_call_outputs(torch, wl, sets[0], t)
        launches = [wl.launcher(torch, d) for d in sets]
        for i in range(200):
            launches[i % 3]()
        runs[(t, "eager")] = eager_batch(torch, launches)
        runs[(t, "graph")] = graph_batch(torch, launches)
        if pat is not None:
            empty, exact, psets = decode_floor_launches(torch, pat, t, wl.H, dev)
            runs[(t, "floor")] = graph_batch(torch, empty)
            runs[(t, "pattern")] = graph_batch(torch, exact)
            keep.append(psets)
        keep.append(sets)
        e = {"algorithmic_bytes": wl.bytes}
        if not args.no_cpu:
            cb = cpu_baseline(wl, cpu, t, 1.0, first, threads=1)
            e["cpu_us"] = cb["us_per_call"]
            e["cpu_cores"] = 1
            e["gpu_first_call_vs_oracle"] = cb["gpu_first_call_vs_oracle"]
        out[f"T{t}"] = e
    got = {k: [] for k in runs}
    for _ in range(DECODE_BATCHES):
        for k, run in runs.items():
            got[k].append(run())
    for (t, kind), v in got.items():
        v = sorted(v)
        e = out[f"T{t}"]
        e[f"{kind}_us"] = round(v[len(v) // 2], 3)
        e[f"{kind}_us_min_max"] = [round(v[0], 3), round(v[-1], 3)]
    for t in DECODE_T:
        e = out[f"T{t}"]
        if "floor_us" in e:
            e["kernel_vs_floor"] = round(e["floor_us"] / e["graph_us"], 4)
            e["kernel_vs_pattern"] = round(e["pattern_us"] / e["graph_us"], 4)
    eagers = [out[f"T{t}"]["eager_us"] for t in DECODE_T]
    out["eager_spread"] = round(max(eagers) / min(eagers) - 1, 4)
    del runs, keep
    torch.cuda.empty_cache()
    return out


# The reference's only published figure for this path: fused_add_rms_norm, T = 1024, H = 512,
# fp16, "GPU time (cold)" on four MetaX C280 devices (56 SMs, 1843 GB/s bus peak), measured by
# benchmark/fused_add_rms_norm_simple.py under its nvbench fork.
PUBLISHED_H1 = {"device": "MetaX C280", "gpu_us_cold": [62.880, 55.262, 41.581, 41.773],
                "bytes_per_call": 4195328,
                "source": "mxbench/README_MXBENCH.md:162,167,172,177 (bytes: "
                          "benchmark/fused_add_rms_norm_simple.py:57-61)"}


def published_entry(torch, args, dev):
    """torch.ops._C.fused_add_rms_norm at the reference's published shape (1024 x 512 fp16,
    eps 1e-6), timed as nvbench times its samples: one launch between an event pair, with the
    stream held busy while the host enqueues them (so the pair measures the GPU, not the host's
    launch latency).  Cold: each sample follows a 512 MiB fill, which evicts the inputs from L2
    and the 256 MB Infinity Cache (nvbench's cold samples flush the L2 the same way); hot: each
    sample follows a clock-bounded spin kernel (torch.cuda._sleep) on inputs already in cache.
    Also back to back and replayed from a HIP graph; GB/s on the reference's byte model; the
    ratio of the reference's published GPU times to this cold median; the GPU's first call
    against the C oracle."""
    wl = WORKLOADS["published-h1"]
    cpu = config_inputs(wl.name)
    ref = oracle_call(wl, cpu) if not args.no_cpu else None
    sets = wl.device_sets(torch, dev, 4, cpu)
    first = first_call_outputs(torch, wl, sets[0], wl.T)
    launches = [wl.launcher(torch, d) for d in sets]
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
    for i in range(64):
        launches[i % len(launches)]()
    torch.cuda.synchronize()
    n = 256

    def samples(before):
        ev = [(_ev(torch), _ev(torch)) for _ in range(n)]
        for i in range(n):
            before()
            ev[i][0].record()
            launches[i % len(launches)]()
            ev[i][1].record()
        torch.cuda.synchronize()
        v = sorted(a.elapsed_time(b) * 1e3 for a, b in ev)
        return {"median": round(v[n // 2], 3), "p10": round(v[n // 10], 3),
                "p90": round(v[9 * n // 10], 3)}
    cold = samples(lambda: flush.zero_())
    hot = samples(lambda: torch.cuda._sleep(100000))
    b2b = _batches(eager_batch(torch, launches, 1024), 5)
    graph = _batches(graph_batch(torch, launches, 1024), 5)
    props = torch.cuda.get_device_properties(0)
    pub = PUBLISHED_H1["gpu_us_cold"]
    out = {"entry": "torch.ops._C.fused_add_rms_norm (in place), fp16", "kernel": kernel_name(wl),
           "shape": [wl.T, wl.H], "dtype": "fp16", "bytes_per_call": wl.bytes,
           "device": f"{torch.cuda.get_device_name(0)} ({props.gcnArchName.split(':')[0]}, "
                     f"{props.multi_processor_count} CUs)",
           "cold_us": cold, "hot_us": hot,
           "back_to_back_us": b2b["median"], "graph_us": graph["median"],
           "GBs_cold": round(wl.bytes / (cold["median"] * 1e-6) / 1e9, 1),
           "GBs_graph": round(wl.bytes / (graph["median"] * 1e-6) / 1e9, 1),
           "published": PUBLISHED_H1,
           "vs_published": {"what": "reference GPU time (cold) / this GPU's cold median, per "
                                    "published device (higher = faster here); different GPUs "
                                    "and vendors, so context rather than a like-for-like target",
                            "ratios": [round(p / cold["median"], 2) for p in pub],
                            "min": round(min(pub) / cold["median"], 2),
                            "max": round(max(pub) / cold["median"], 2)},
           "timing": f"{n} samples of one launch between an event pair (cold: after a 512 MiB "
                     f"fill; hot: after a spin kernel); back-to-back and graph: median of 5 "
                     f"batches of 1024 calls"}
    if ref is not None:
        diffs = {k: int((first[k].view(torch.int16) != ref[k].view(torch.int16)).sum())
                 for k in ("x", "r")}
        out["gpu_first_call_vs_oracle"] = {"rows": wl.T, "differing_values": diffs,
                                           "bit_exact": all(v == 0 for v in diffs.values())}
    prof = profile_summary(wl)
    if prof:
        out["profile"] = prof["file"]
        out["rocprof_trace_mean_us"] = prof["trace_mean_us"]
        out["profile_stale"] = prof["stale"]
    del sets, launches, flush
    torch.cuda.empty_cache()
    return out


def cfg1_entry(args):
    """cfg1 runs on the CPU only: the C oracle (all cores, and one) and the torch restatement."""
    import torch

    wl = WORKLOADS["cfg1"]
    cpu = config_inputs("cfg1")
    out = {"entry": "rms_norm_dynamic_per_token_quant (vLLM), no residual, int8", "cpu_only": True,
           "shape": [wl.T, wl.H], "algorithmic_bytes": wl.bytes}
    if args.no_cpu:
        return out
    secs = args.cpu_seconds / 3
    out["oracle"] = cpu_baseline(wl, cpu, wl.T, secs)
    out["oracle_1_thread"] = cpu_baseline(wl, cpu, wl.T, secs, threads=1)
    out["torch"] = cpu_torch(wl, cpu, wl.T, secs)
    # the torch restatement and the oracle agree bit for bit on this input
    q, s, _ = torch_cpu_add_norm_int8(cpu["x"], None, cpu["w"], wl.eps)
    ref = oracle_call(wl, cpu)
    out["torch_equals_oracle"] = bool(torch.equal(q, ref["q"]) and
                                      torch.equal(s.view(-1), ref["s"].view(-1)))
    return out


# ------------------------------------------------------------------------------ main
def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "rows are independent, so N GPUs would each run this kernel on T/N rows with no "
              "communication -- run with --gpus 1", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    sys.path.insert(0, str(ROOT))
    import mcoplib  # noqa: F401  (fails loudly if libmcop_norm.so is missing)

    if args.multi_pass:
        global MULTI_PASS
        from mcoplib_amd import _lib
        _lib.set_split_rows(False)
        MULTI_PASS = True
    dev = "cuda:0"
    torch.cuda.set_device(0)
    wl = WORKLOADS[args.workload]
    if args.copy_calibration:
        src = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if wl.kind == "norm_int8":
        print("bench.py: cfg1 is measured on the CPU only (it is part of the default run's "
              "`configs`)", file=sys.stderr)
        return 2
    if args.pattern is not None:
        if wl.name not in PATTERN_OF:
            print(f"bench.py: {wl.name} has no access-pattern kernel (those of "
                  f"{sorted(PATTERN_OF)} do)", file=sys.stderr)
            return 2
        p, nv, tpr = PATTERN_OF[wl.name]
        lds = 0 if args.pattern == "natural" else LDS_PER_CU // int(args.pattern) - 1024
        pus = pattern_us(torch, Pattern(), p, wl.T, wl.H, nv, tpr, dev, args.steps, with_w=True,
                         with_sm=wl.kind == "smooth_fp8", lds=lds)
        print(json.dumps({"workload": wl.name, "pattern": p, "vectors_per_lane": nv,
                          "lanes_per_row": tpr, "workgroups_per_cu": args.pattern,
                          "lds_bytes": lds, "us": round(pus, 3),
                          "GBs": round(wl.bytes / (pus * 1e-6) / 1e9, 1)}), flush=True)
        return 0

    cpu = config_inputs(wl.name) if wl.seeded else None
    check_rows = min(wl.T, 1024) if (wl.seeded and not args.no_cpu) else 0
    m = measure(torch, wl, args, dev, cpu, check_rows=check_rows)
    K, ms = args.steps, m["ms"]
    value = wl.bytes / (ms * 1e-3) / 1e9
    # one step is exactly one launch of the kernel and nothing else runs on the stream, so the
    # kernel's average launch duration over the timed region is total / K
    kernel_us = ms * 1e3
    prof = profile_summary(wl)
    traffic = prof["hbm_bytes_per_dispatch"] if prof else None
    roof = {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic,
            "traffic_ratio": round(traffic / wl.bytes, 4) if traffic else None,
            "kernel": kernel_name(wl), "kernel_avg_us": round(kernel_us, 3),
            "kernel_avg_us_from": "HIP events around the K timed launches on the launch stream",
            "rocprof_trace_mean_us": prof["trace_mean_us"] if prof else None,
            "profile": prof["file"] if prof else None,
            "single_launch_us_p10_p50_p90": m.get("p10_p50_p90_us"),
            "algorithmic_bytes_per_launch": wl.bytes}
    out = {
        "metric": METRIC if wl.name == "cfg3" else f"HBM GB/s: {wl.name} ({wl.kind}, {wl.T}x{wl.H})",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded CPU inputs copied to the GPU, the same bits in every leg"
                if wl.seeded else "synthetic: device-RNG inputs",
        "config": {"workload": f"{wl.name}: {wl.kind} T={wl.T} H={wl.H} "
                               f"{'fp16' if wl.name == 'published-h1' else 'bf16'} in"
                               + ("" if wl.kind.startswith("ptq_") or wl.kind == "sdq" else f", eps={wl.eps}")
                               + (", 1% outlier channels x20" if wl.name == "cfg3" else ""),
                   "tokens": wl.T, "hidden": wl.H, "io": "bf16 -> int8/fp8 + fp32 scales",
                   "rotated_input_sets": m["sets"]},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "tokens_per_s": round(wl.T / (ms * 1e-3), 1),
        "roofline": roof,
        "hot_value": round(wl.bytes / (m["hot_ms"] * 1e-3) / 1e9, 2),
        "hot_note": "the same steps on one input set (not rotated)",
        "host_wall_s": round(m["wall"], 4),
        "us_per_call": round(kernel_us, 3),
        "us_per_call_graph": None if "graph_us" not in m else round(m["graph_us"], 3),
    }
    roof["profile_stale"] = prof["stale"] if prof else None
    if wl.name == "cfg3":
        out["guard"] = guard_of(roof["frac"], prof, wl.bytes)
    pat = None
    if not args.no_configs:
        pat = Pattern()
        # streaming ceilings over 1 GiB of bf16 (read-only and write-only: 1 GiB moved; copy:
        # 1 GiB read + 1 GiB written) at the launch shape that streams fastest on this GPU (one
        # 16-byte vector a lane, 2048-element rows of 256 lanes: measured best of 1-8 vectors a
        # lane and 64-1024 lanes)
        T1, H1 = 262144, 2048
        cu = pattern_us(torch, pat, PATTERN_COPY, T1, H1, 1, 256, dev, K)
        ru = pattern_us(torch, pat, PATTERN_READ, T1, H1, 1, 256, dev, K)
        wu = pattern_us(torch, pat, PATTERN_WRITE, T1, H1, 1, 256, dev, K)
        copy_gbs = 2 * T1 * H1 * 2 / (cu * 1e-6) / 1e9
        out["device_copy"] = {"GBs": round(copy_gbs, 1), "frac": round(value / copy_gbs, 4),
                              "what": "non-temporal streaming copy kernel (libmcop_pattern.so), "
                                      "1 GiB read + 1 GiB written, one 16-byte vector a lane"}
        ceil = {"read_only_GBs": round(T1 * H1 * 2 / (ru * 1e-6) / 1e9, 1),
                "write_only_GBs": round(T1 * H1 * 2 / (wu * 1e-6) / 1e9, 1),
                "copy_GBs": round(copy_gbs, 1)}
        if wl.name in PATTERN_OF:
            p, nv, tpr = PATTERN_OF[wl.name]
            pus = pattern_us(torch, pat, p, wl.T, wl.H, nv, tpr, dev, K, with_w=True,
                             with_sm=wl.kind == "smooth_fp8")
            ceil[f"{wl.name}_pattern"] = {
                "us": round(pus, 3), "GBs": round(wl.bytes / (pus * 1e-6) / 1e9, 1),
                "kernel_vs_pattern": round(pus / kernel_us, 4),
                "what": "compute-free kernel with the operator's loads, stores and launch shape"}
            mus = mix_us(torch, pat, wl, dev, K)
            ceil[f"{wl.name}_mix"] = {
                "us": round(mus, 3), "GBs": round(wl.bytes / (mus * 1e-6) / 1e9, 1),
                "kernel_vs_mix": round(mus / kernel_us, 4),
                "what": f"the same compute-free kernel over the same elements reshaped to "
                        f"{MIX_H}-wide rows (one vector a lane, 256 lanes): the operator's "
                        f"traffic mix at the fastest streaming shape"}
        out["ceilings"] = ceil
    if not args.no_cpu and wl.seeded:
        out["cpu_baseline"] = cpu_baseline(wl, cpu, min(wl.T, 1024), args.cpu_seconds,
                                           m["first"])
        out["cpu_torch"] = cpu_torch(wl, cpu, min(wl.T, 512), min(args.cpu_seconds, 10.0))
    if not args.no_configs and wl.name == "cfg3":
        cfgs = {"cfg1": cfg1_entry(args)}
        cfgs["cfg2"] = config_entry(torch, WORKLOADS["cfg2"], args, dev, pat,
                                    "torch.ops._C.fused_add_rms_norm (in place)")
        cfgs["cfg4"] = config_entry(torch, WORKLOADS["cfg4"], args, dev, pat,
                                    "mcoplib.op.rms_norm_dynamic_per_token_quant (SmoothQuant, "
                                    "fp8-e4m3fn, after_res + after_norm)")
        cfgs["cfg5_decode"] = decode_entry(torch, args, dev, pat)
        cfgs["cfg5_large"] = config_entry(torch, WORKLOADS["cfg5-large"], args, dev, pat,
                                          "mcoplib.op.rms_norm_dynamic_per_token_quant_custom "
                                          "with residual")
        # the reference's one published number sits on another GPU and another shape than the
        # headline metric, so `vs_baseline` stays null; the comparison at its own shape is here
        cfgs["published_h1"] = published_entry(torch, args, dev)
        out["configs"] = cfgs
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
