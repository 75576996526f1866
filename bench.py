#!/usr/bin/env python3
"""Benchmark of the fused add + RMSNorm + per-token int8 quantization path on one MI355X.

Default workload ("cfg3", the headline configuration): x and residual bf16 [8192, 8192] (1% of channels scaled x20
as outliers), weight bf16 ~N(1, 0.1), eps 1e-5; output int8 [8192, 8192] + fp32 scales [8192, 1]
+ the bf16 residual written in place.  One step = one call of
mcoplib_amd.custom_ops.rms_norm_dynamic_per_token_quant (one kernel launch) over one batch that
is already resident in HBM; three input sets are rotated so consecutive steps do not hit the
256 MB last-level cache.

Prints ONE JSON line:  value = algorithmic GB/s of the whole job (bytes = every input read once
+ every output written once, 7*T*H + 2*H + 4*T for config 3), plus `roofline` (the kernel's
average launch duration from HIP events recorded around every launch inside the timed region)
and `cpu_baseline` (the C oracle on a bounded row sample on this host's cores), with
`cpu_torch` beside it (the same operation in vectorized torch on the CPU).

  python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--workload cfg3]
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
PAD_SIZE = 3840  # padded workload: bf16 elements per padded row (2 * 3840 bytes)
BLOCK_GROUP = 128  # block-fp8 workload: elements per scale group
HEADS = 8  # head-norm workload: heads per token (all normalized, per-head weights)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="cfg3",
                    choices=["cfg2", "cfg3", "cfg4", "cfg5-large", "cfg5-decode1",
                             "cfg5-decode4", "cfg5-decode16", "cfg5-decode64", "ptq-int8",
                             "ptq-int8-azp", "ptq-fp8", "padded", "block-fp8", "norm-res",
                             "vllm-norm", "head-norm", "sdq", "wide-int8", "wide-fused",
                             "wide-fp8", "wide-sdq", "wide-norm", "wide-ptq", "wide-padded",
                             "wide-block"])
    ap.add_argument("--sets", type=int, default=0,
                    help="rotated input sets (default: enough for > 1 GiB, at least 3)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--warmup-seconds", type=float, default=2.0)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run three 1 GiB device-to-device copies (a kernel of known "
                         "traffic, used to scale rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    return ap.parse_args()


# ------------------------------------------------------------------------------ workloads
class Workload:
    """Inputs, a launcher and the byte model of one benchmark configuration."""

    def __init__(self, name, T, H, eps, kind):
        self.name, self.T, self.H, self.eps, self.kind = name, T, H, eps, kind

    @property
    def pad(self) -> int:
        """Padded row size in bf16 elements (padded workloads): PAD_SIZE, or enough for H + 4."""
        return PAD_SIZE if 2 * PAD_SIZE >= self.H + 4 else (self.H + 4 + 63) // 64 * 32

    @property
    def bytes(self) -> int:
        T, H = self.T, self.H
        if self.kind == "add_norm_int8":   # read x, r (2H each), w; write r (2H), q (H), s
            return 7 * T * H + 2 * H + 4 * T
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

    def make(self, torch, dev, seed):
        T, H = self.T, self.H
        g = torch.Generator(device=dev).manual_seed(seed)
        x = torch.randn(T, H, generator=g, device=dev)
        if self.name == "cfg3":
            idx = torch.randperm(H, generator=torch.Generator().manual_seed(3))[: round(0.01 * H)]
            x[:, idx.to(dev)] *= 20.0
        x = x.to(torch.bfloat16)
        w = (1 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
        d = {"x": x, "w": w}
        if self.kind == "head_norm":       # x [T/HEADS tokens, HEADS, H], per-head weights
            d["x"] = x.view(T // HEADS, HEADS, H)
            d["w"] = (1 + 0.1 * torch.randn(HEADS, H, generator=g, device=dev)).to(torch.bfloat16)
        if self.kind in ("norm_res", "vllm_norm", "head_norm"):
            d["out"] = torch.empty_like(d["x"])
        if self.kind in ("add_norm_int8", "fused_add", "padded", "block_fp8", "norm_res"):
            d["r"] = torch.randn(T, H, generator=g, device=dev).to(torch.bfloat16)
        if self.kind == "add_norm_int8":
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
        if self.kind == "sdq":
            d["sm"] = 0.5 + 1.5 * torch.rand(H, generator=g, device=dev)
        if self.kind == "smooth_fp8":
            d["sm"] = 0.5 + 1.5 * torch.rand(H, generator=g, device=dev)
            d["q"] = torch.empty(T, H, dtype=torch.float8_e4m3fn, device=dev)
            d["s"] = torch.empty(T, dtype=torch.float32, device=dev)
            d["ar"] = torch.empty_like(x)
            d["an"] = torch.empty_like(x)
        return d

    def launcher(self, torch, d):
        from mcoplib_amd import op
        import mcoplib_amd._C  # noqa: F401
        if self.kind == "add_norm_int8":
            return lambda: op.rms_norm_dynamic_per_token_quant_custom(
                d["q"], d["x"], d["w"], d["s"], self.eps, None, d["r"])
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
    "cfg2": Workload("cfg2", 4096, 4096, 1e-6, "fused_add"),
    "cfg3": Workload("cfg3", 8192, 8192, 1e-5, "add_norm_int8"),
    "cfg4": Workload("cfg4", 16384, 7168, 1e-6, "smooth_fp8"),
    "cfg5-large": Workload("cfg5-large", 32768, 16384, 1e-6, "add_norm_int8"),
    **{f"cfg5-decode{t}": Workload(f"cfg5-decode{t}", t, 5120, 1e-6, "add_norm_int8")
       for t in (1, 4, 16, 64)},
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
    # rows wider than the registers hold: the headline operator's multi-pass kernel
    "wide-int8": Workload("wide-int8", 2048, 131072, 1e-6, "add_norm_int8"),
    "wide-fused": Workload("wide-fused", 2048, 131072, 1e-6, "fused_add"),
    "wide-fp8": Workload("wide-fp8", 2048, 131072, 1e-6, "smooth_fp8"),
    "wide-sdq": Workload("wide-sdq", 2048, 131072, 0.0, "sdq"),
    "wide-norm": Workload("wide-norm", 2048, 131072, 1e-6, "norm_res"),
    "wide-ptq": Workload("wide-ptq", 2048, 131072, 0.0, "ptq_int8"),
    "wide-padded": Workload("wide-padded", 2048, 131072, 1e-6, "padded"),
    "wide-block": Workload("wide-block", 2048, 131072, 1e-6, "block_fp8"),
}
KERNEL_NAME = {"add_norm_int8": "k_rms_norm_quant", "fused_add": "k_fused_add_rms_norm",
               "smooth_fp8": "k_rms_norm_smooth_quant", "ptq_int8": "k_per_token_quant",
               "ptq_int8_azp": "k_per_token_quant", "ptq_fp8": "k_per_token_quant",
               "padded": "k_add_rms_norm_quant_padded", "block_fp8": "k_rms_norm_group_quant",
               "norm_res": "k_rms_norm", "vllm_norm": "k_rms_norm", "head_norm": "k_rms_norm",
               "sdq": "k_scale_dynamic_quant"}
# workloads whose kernel is not their kind's register-resident one
KERNEL_NAME_OF_WORKLOAD = {"wide-int8": "k_rms_norm_quant_wide",
                           "wide-fused": "k_fused_add_rms_norm_wide",
                           "wide-fp8": "k_rms_norm_smooth_quant_wide",
                           "wide-sdq": "k_scale_dynamic_quant_wide",
                           "wide-norm": "k_rms_norm_wide", "wide-ptq": "k_per_token_quant_wide",
                           "wide-padded": "k_add_rms_norm_quant_padded_wide",
                           "wide-block": "k_rms_norm_group_quant_wide"}


def kernel_name(wl) -> str:
    return KERNEL_NAME_OF_WORKLOAD.get(wl.name, KERNEL_NAME[wl.kind])


# ------------------------------------------------------------------------------ pieces
def traffic_from_profiles(wl: Workload):
    """HBM bytes per dispatch measured with rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, scaled by
    a copy kernel's reading), from the committed summary, or None."""
    p = ROOT / "profiles" / f"{kernel_name(wl)}_{wl.name}.txt"
    if not p.exists():
        return None
    m = re.search(r"^hbm_bytes_per_dispatch:\s*([0-9.eE+]+)", p.read_text(), re.M)
    return float(m.group(1)) if m else None


def cpu_baseline(wl: Workload, seconds: float) -> dict:
    """The C oracle (oracle/mcop_oracle.c, OpenMP over rows) on a bounded row sample of the same
    workload, on this host's cores; reported in the metric's unit."""
    import torch
    import oracle  # CPU baseline leg only

    cores = len(os.sched_getaffinity(0))
    oracle.set_threads(cores)
    rows = min(wl.T, 1024)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(rows, wl.H, generator=g).to(torch.bfloat16)
    r = torch.randn(rows, wl.H, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(wl.H, generator=g)).to(torch.bfloat16)
    sm = 0.5 + 1.5 * torch.rand(wl.H, generator=g)

    def run():
        if wl.kind == "add_norm_int8":
            oracle.rms_norm_dynamic_per_token_quant(x, w, wl.eps, torch.int8, residual=r)
        elif wl.kind == "fused_add":
            oracle.fused_add_rms_norm(x, r, w, wl.eps)
        elif wl.kind == "norm_res":
            oracle.rms_norm(x, w, wl.eps, residual=r)
        elif wl.kind == "vllm_norm":
            oracle.vllm_rms_norm(x, w, wl.eps)
        elif wl.kind == "head_norm":
            xs = x.reshape(-1, HEADS, wl.H)
            oracle.head_rms_norm(xs, xs, w.repeat(HEADS).view(HEADS, wl.H), wl.eps, 0, HEADS)
        elif wl.kind == "block_fp8":
            oracle.rms_norm_per_block_quant(x, w, wl.eps, torch.float8_e4m3fn, BLOCK_GROUP,
                                            residual=r)
        elif wl.kind == "padded":
            oracle.add_rms_norm_quant_padded(x, r, w, wl.pad, wl.eps)
        elif wl.kind == "sdq":
            oracle.scale_dynamic_quant(x, sm)
        elif wl.kind == "ptq_fp8":
            oracle.dynamic_per_token_scaled_fp8_quant(x)
        elif wl.kind.startswith("ptq_int8"):
            oracle.dynamic_scaled_int8_quant(x, use_azp=wl.kind == "ptq_int8_azp")
        else:
            oracle.rms_norm_smooth_quant(x, w, sm, wl.eps, torch.float8_e4m3fn)

    run()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    sample_bytes = Workload(wl.name, rows, wl.H, wl.eps, wl.kind).bytes
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(sample_bytes / med / 1e9, 3), "unit": "GB/s", "cores": cores,
            "kind": "port",
            "sample": f"{rows} of {wl.T} rows x {wl.H} (same byte model), median of {len(times)} "
                      f"runs over ~{seconds:.0f} s, oracle/mcop_oracle.c with {cores} OpenMP "
                      f"threads, {cpu_model}",
            "tokens_per_s": round(rows / med, 1)}


def torch_cpu_add_norm_int8(x, r, w, eps: float):
    """Add + RMSNorm + per-token int8 restated in vectorized torch (the form of the reference's
    own torch-native test oracles), following the reference's rounding points
    (op/vllm/quantization/fused_kernels/layernorm_utils.cuh:245-276, 436-447, 503-531 and
    fused_layernorm_dynamic_per_token_quant.cu:37): residual b(x + r), rho on the unrounded sum,
    y = b(b(a * rho) * w), s = max(A / 127, FLT_EPSILON), q = sat(rne(y * (1/s))).
    Returns (q, s, residual)."""
    import torch

    bf, H = torch.bfloat16, x.shape[-1]
    a = x.float() + r.float()
    res = a.to(bf)
    ss = (a.double() * a.double()).sum(-1, keepdim=True)
    rho = 1.0 / torch.sqrt((ss / H).float() + eps)
    y = ((a * rho).to(bf).float() * w.float()).to(bf).float()
    s = torch.clamp(y.abs().amax(-1, keepdim=True) / 127.0, min=torch.finfo(torch.float32).eps)
    q = torch.round(y * (1.0 / s)).clamp(-128, 127).to(torch.int8)
    return q, s, res


def cpu_torch(wl: Workload, seconds: float):
    """torch_cpu_add_norm_int8 timed on this host (torch's intra-op threads) on a bounded row
    sample, beside the C oracle.  Only the headline operation (kind add_norm_int8) has this leg;
    None otherwise."""
    if wl.kind != "add_norm_int8":
        return None
    import torch

    rows = min(wl.T, 512)
    g = torch.Generator().manual_seed(7)
    x = torch.randn(rows, wl.H, generator=g).to(torch.bfloat16)
    r = torch.randn(rows, wl.H, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(wl.H, generator=g)).to(torch.bfloat16)
    torch_cpu_add_norm_int8(x, r, w, wl.eps)
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        torch_cpu_add_norm_int8(x, r, w, wl.eps)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    sample_bytes = Workload(wl.name, rows, wl.H, wl.eps, wl.kind).bytes
    threads = torch.get_num_threads()
    return {"value": round(sample_bytes / med / 1e9, 3), "unit": "GB/s", "cores": threads,
            "sample": f"{rows} of {wl.T} rows x {wl.H}, median of {len(times)} runs over "
                      f"~{seconds:.0f} s, vectorized torch on the CPU with {threads} intra-op "
                      "threads (bench.py torch_cpu_add_norm_int8)",
            "tokens_per_s": round(rows / med, 1)}


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
    import mcoplib_amd  # noqa: F401  (fails loudly if libmcop_norm.so is missing)

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
    n_sets = args.sets or max(3, -(-(1 << 30) // wl.bytes))
    sets = [wl.make(torch, dev, 100 + i) for i in range(n_sets)]
    launches = [wl.launcher(torch, d) for d in sets]
    # warm-up: the requested steps, continued until the GPU has been busy for ~2 s so that
    # clocks and power state have settled before the timed region
    i, t_w = 0, time.perf_counter()
    while i < args.warmup or time.perf_counter() - t_w < args.warmup_seconds:
        launches[i % len(launches)]()
        i += 1
        if i % 64 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()

    K = args.steps
    # (1) whole-job throughput: K back-to-back steps between two events
    t_start, t_stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    t_start.record()
    for i in range(K):
        launches[i % len(launches)]()
    t_stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total_ms = t_start.elapsed_time(t_stop)
    ms_per_step = total_ms / K
    # (2) a second pass with an event pair around every launch: the spread of single-launch
    # times (each pair also times the event packets themselves, so its mean sits above the
    # back-to-back figure, which is what rocprofv3's kernel trace reports)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(K)]
    for i in range(K):
        ev[i][0].record()
        launches[i % len(launches)]()
        ev[i][1].record()
    torch.cuda.synchronize()
    per_launch_ms = sorted(a.elapsed_time(b) for a, b in ev)
    # one step is exactly one launch of the kernel and nothing else runs on the stream, so the
    # kernel's average launch duration over the timed region is total / K
    kernel_ms = ms_per_step

    # (2b) the same K steps on one input set only (hot: small sets stay in the 256 MB MALL)
    h0, h1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    h0.record()
    for i in range(K):
        launches[0]()
    h1.record()
    torch.cuda.synchronize()
    hot_ms = h0.elapsed_time(h1) / K
    # (2c) this GPU's device-copy bandwidth (1 GiB copy_, read + write bytes): the practical
    # ceiling of a streaming kernel, reported next to the 8 TB/s peak
    csrc = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    cdst = torch.empty_like(csrc)
    for _ in range(3):
        cdst.copy_(csrc)
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record()
    for _ in range(5):
        cdst.copy_(csrc)
    c1.record()
    torch.cuda.synchronize()
    copy_gbs = 2 * 5 * (1 << 30) / (c0.elapsed_time(c1) * 1e-3) / 1e9
    del csrc, cdst

    # (3) decode shapes are launch-bound: also time the same steps replayed from a HIP graph
    graph_us = None
    if wl.T <= 256:
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
        g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 5
        g0.record()
        for _ in range(reps):
            g.replay()
        g1.record()
        torch.cuda.synchronize()
        graph_us = g0.elapsed_time(g1) * 1e3 / (reps * K)

    value = wl.bytes / (ms_per_step * 1e-3) / 1e9
    achieved = wl.bytes / (kernel_ms * 1e-3) / 1e9
    traffic = traffic_from_profiles(wl)
    out = {
        "metric": METRIC if wl.name == "cfg3" else f"HBM GB/s: {wl.name} ({wl.kind}, {wl.T}x{wl.H})",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{wl.name}: {wl.kind} T={wl.T} H={wl.H} bf16 in"
                               + ("" if wl.kind.startswith("ptq_") or wl.kind == "sdq" else f", eps={wl.eps}")
                               + (", 1% outlier channels x20" if wl.name == "cfg3" else ""),
                   "tokens": wl.T, "hidden": wl.H, "io": "bf16 -> int8/fp8 + fp32 scales",
                   "rotated_input_sets": len(sets)},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "tokens_per_s": round(wl.T / (ms_per_step * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "kernel": kernel_name(wl),
                     "kernel_avg_us": round(kernel_ms * 1e3, 3),
                     "single_launch_us_p10_p50_p90": [
                         round(per_launch_ms[int(q * (K - 1))] * 1e3, 3) for q in (0.1, 0.5, 0.9)],
                     "algorithmic_bytes_per_launch": wl.bytes},
        "device_copy": {"GBs": round(copy_gbs, 1), "frac": round(value / copy_gbs, 4),
                        "what": "1 GiB torch copy_ on this GPU, read + write bytes"},
        "hot_value": round(wl.bytes / (hot_ms * 1e-3) / 1e9, 2),
        "hot_note": "the same steps on one input set (not rotated)",
        "host_wall_s": round(wall, 4),
        "us_per_call": round(ms_per_step * 1e3, 3),
        "us_per_call_graph": None if graph_us is None else round(graph_us, 3),
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(wl, args.cpu_seconds)
        out["cpu_torch"] = cpu_torch(wl, min(args.cpu_seconds, 10.0))
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
