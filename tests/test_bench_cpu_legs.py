"""The CPU legs and inputs of bench.py: the vectorized torch restatement (the `cpu_torch` figure)
equals the C oracle bit for bit for both operators it restates, and the seeded inputs follow the
stated recipe (the same builder feeds the GPU parity tests, so the benchmarked bits are the
parity-checked bits)."""

import torch

import bench
import oracle


def _rows(seed, T, H):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g)
    x[:, :40] *= 20.0  # outlier channels, as in the headline workload
    x = x.to(torch.bfloat16)
    r = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    return x, r, w


def test_torch_cpu_leg_equals_the_oracle():
    x, r, w = _rows(3, 64, 4096)
    q, s, res = bench.torch_cpu_add_norm_int8(x, r, w, 1e-5)
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-5, torch.int8,
                                                                  residual=r)
    assert torch.equal(res, r_ref)
    assert torch.equal(s.view(-1), s_ref.view(-1))
    assert torch.equal(q, q_ref)
    # without a residual (cfg1)
    q, s, res = bench.torch_cpu_add_norm_int8(x, None, w, 1e-6)
    q_ref, s_ref, _ = oracle.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.int8)
    assert res is None and torch.equal(q, q_ref) and torch.equal(s.view(-1), s_ref.view(-1))


def test_torch_cpu_leg_of_the_mcoplib_operator_equals_the_oracle():
    # the benchmarked surface is mcoplib's own operator (1.5e-6 scale floor, codes +-127)
    x, r, w = _rows(4, 64, 8192)
    x[3].zero_()
    r[3].zero_()  # a zero row: the floor decides the scale
    q, s, res = bench.torch_cpu_add_norm_int8(x, r, w, 1e-5, floor=1.5e-6, lo=-127)
    q_ref, s_ref, r_ref = oracle.rms_norm_dynamic_per_token_quant_custom(x, w, 1e-5, residual=r)
    assert torch.equal(res, r_ref)
    assert torch.equal(s.view(-1), s_ref.view(-1))
    assert s[3].item() == torch.tensor(1.5e-6, dtype=torch.float32).item()
    assert torch.equal(q, q_ref)


def test_config_inputs_follow_the_recipe():
    c = bench.config_inputs("cfg3")
    x, r, w = c["x"], c["r"], c["w"]
    assert x.shape == r.shape == (8192, 8192) and w.shape == (8192,) and c["eps"] == 1e-5
    assert x.dtype == r.dtype == w.dtype == torch.bfloat16
    # 82 outlier channels: column RMS ~20 there, ~1 elsewhere
    col = x.float().pow(2).mean(0).sqrt()
    assert int((col > 10).sum()) == 82 and float(col[col < 10].max()) < 1.2
    g = torch.Generator().manual_seed(3)
    assert set(torch.nonzero(col > 10).view(-1).tolist()) == \
        set(torch.randperm(8192, generator=g)[:82].tolist())
    # residual and weight statistics
    assert abs(float(r.float().std()) - 1) < 0.01 and abs(float(w.float().mean()) - 1) < 0.01
    c4 = bench.config_inputs("cfg4")
    assert c4["r"] is None and c4["sm"].dtype == torch.float32
    assert 0.5 <= float(c4["sm"].min()) and float(c4["sm"].max()) <= 2.0
    # deterministic: the same bits every time
    assert torch.equal(bench.config_inputs("cfg5-decode4")["x"],
                       bench.config_inputs("cfg5-decode4")["x"])


def _guard_tree(tmp_path):
    """A copy of the sources the headline kernel's hash covers, with a profile summary of the
    headline workload that records their current hash."""
    import shutil
    from pathlib import Path

    src = Path(bench.ROOT)
    (tmp_path / "mcoplib_amd").mkdir()
    shutil.copytree(src / "mcoplib_amd" / "csrc", tmp_path / "mcoplib_amd" / "csrc")
    shutil.copy(src / "mcoplib_amd" / "_build.py", tmp_path / "mcoplib_amd" / "_build.py")
    (tmp_path / "profiles").mkdir()
    wl = bench.WORKLOADS["cfg3"]
    h = bench.kernel_source_hash("k_rms_norm_quant", tmp_path)
    (tmp_path / "profiles" / "k_rms_norm_quant_cfg3.txt").write_text(
        "# k_rms_norm_quant on cfg3\n"
        f"kernel_source_sha16: {h}\n"
        "timed legs (200 dispatches): mean 76.310 us, median 76.151 us\n"
        f"hbm_bytes_per_dispatch: {int(wl.bytes * 1.0009)}\n")
    return tmp_path, wl


def test_guard_flags_a_profile_of_other_sources(tmp_path):
    """The headline guard trusts the committed profile's traffic only while the kernel's sources
    are the ones it was taken on: editing rms_norm_quant.hip (or a header every kernel shares, or
    the compile flags) without re-profiling marks the profile stale and the run regressed."""
    root, wl = _guard_tree(tmp_path)
    prof = bench.profile_summary(wl, root)
    assert prof["stale"] is False
    g = bench.guard_of(0.7651, prof, wl.bytes)
    assert g["regressed"] is False and g["profile_stale"] is False
    assert g["traffic_ratio"] == 1.0009
    # an edit to the kernel's own source
    k = root / "mcoplib_amd" / "csrc" / "rms_norm_quant.hip"
    k.write_text(k.read_text() + "\n// edited after the profile was taken\n")
    prof = bench.profile_summary(wl, root)
    assert prof["stale"] is True
    g = bench.guard_of(0.7651, prof, wl.bytes)
    assert g["regressed"] is True and g["profile_stale"] is True
    # re-profiling (a summary recording the new hash) clears it; a shared header edit sets it
    p = root / "profiles" / "k_rms_norm_quant_cfg3.txt"
    p.write_text(p.read_text().replace(prof["source_sha16"], prof["current_source_sha16"]))
    assert bench.profile_summary(wl, root)["stale"] is False
    hdr = root / "mcoplib_amd" / "csrc" / "rowkern.h"
    hdr.write_text(hdr.read_text() + "\n")
    assert bench.profile_summary(wl, root)["stale"] is True
    # an unrelated kernel's source does not touch the headline's hash
    p.write_text(p.read_text().replace(
        bench.profile_summary(wl, root)["source_sha16"],
        bench.kernel_source_hash("k_rms_norm_quant", root)))
    other = root / "mcoplib_amd" / "csrc" / "scale_dynamic_quant.hip"
    other.write_text(other.read_text() + "\n")
    assert bench.profile_summary(wl, root)["stale"] is False


def test_guard_without_a_profile_or_below_the_bar():
    wl = bench.WORKLOADS["cfg3"]
    assert bench.guard_of(0.77, None, wl.bytes)["regressed"] is True
    prof = {"hbm_bytes_per_dispatch": wl.bytes * 1.0009, "stale": False, "source_sha16": "x",
            "current_source_sha16": "x"}
    assert bench.guard_of(0.7499, prof, wl.bytes)["regressed"] is True
    assert bench.guard_of(0.7501, prof, wl.bytes)["regressed"] is False
    prof["hbm_bytes_per_dispatch"] = wl.bytes * 1.02
    assert bench.guard_of(0.77, prof, wl.bytes)["regressed"] is True


def test_every_benched_workload_names_a_profiled_kernel():
    """Each bandwidth workload's kernel name (the split-row kernel for the wide workloads of
    every operator that has one, the multi-pass kernel under --multi-pass) has its committed
    rocprofv3 summary, so the bench never attributes a workload to a kernel that does not run.
    (Whether a summary is current is the bench's own guard: profile_stale.)"""
    from pathlib import Path
    missing = []
    for name, wl in bench.WORKLOADS.items():
        if name.startswith("cfg5-decode") or name == "cfg1":
            continue
        for mp in ((False, True) if name.startswith("wide-") else (False,)):
            bench.MULTI_PASS = mp
            try:
                kn = bench.kernel_name(wl)
            finally:
                bench.MULTI_PASS = False
            p = Path(bench.ROOT) / "profiles" / f"{kn}_{name}.txt"
            if not p.exists():
                missing.append(str(p.name))
    assert not missing, missing
