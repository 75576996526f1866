"""Compiled resources of the gfx950 kernels, from the hipcc resource-usage remarks that the build
records (mcoplib_amd/_build/resource_usage.json): the build's own check passes on them, and the
check catches the problems it is there for."""

import json

import pytest

from conftest import ROOT


def _build_module():
    import importlib.util

    spec = importlib.util.spec_from_file_location("mcoplib_amd_build",
                                                  ROOT / "mcoplib_amd" / "_build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _records():
    p = ROOT / "mcoplib_amd" / "_build" / "resource_usage.json"
    if not p.exists():
        pytest.skip("the library has not been built here (python mcoplib_amd/_build.py)")
    return json.loads(p.read_text())


def test_built_kernels_pass_the_resource_check():
    b = _build_module()
    recs = _records()
    assert len(recs) > 100
    assert b.check_resources(recs) == []
    # the kernels of the configured shapes keep every register in registers
    # (both forms of the norm-quant kernel: generic and exact-row)
    for pat in (r"k_rms_norm_quant<mcop::BF16, 8, 2, false, true, 1, ",      # cfg 3 (custom op)
                r"k_rms_norm_quant<mcop::BF16, 8, 4, false, true, 0, ",      # cfg 5 large
                r"k_fused_add_rms_norm<mcop::BF16, 8, 2, ",                  # cfg 2
                r"k_rms_norm_smooth_quant<mcop::BF16, mcop::BF16, mcop::F32, 8, 4, true, false, "):
        hits = [r for r in recs if pat in r["kernel"]]
        assert hits and all(r["scratch"] == 0 for r in hits), pat


def test_resource_check_catches_spills():
    b = _build_module()
    ok_four = {"kernel": "void mcop::k_rms_norm_quant<mcop::BF16, 8, 8, false, true, 1, "
                         "false>(...)", "mangled": "x", "scratch": 0, "occupancy": 4}
    ok_h1 = {"kernel": "void mcop::k_fused_add_rms_norm<mcop::BF16, 8, 8, false>(...)",
             "mangled": "y", "scratch": 0, "occupancy": 4}
    ok_split = {"kernel": "void mcop::k_rms_norm_quant_split<mcop::BF16, 8, 8, false, true, "
                          "0>(...)", "mangled": "s", "scratch": 0, "occupancy": 4}
    oks = [ok_four, ok_h1, ok_split]
    assert b.check_resources(oks) == []
    wide = {"kernel": "void mcop::k_rms_norm_quant_wide<mcop::F16, 8, true, false, 0>(...)",
            "mangled": "z", "scratch": 16, "occupancy": 4}
    assert any("multi-pass" in p for p in b.check_resources(oks + [wide]))
    spilled = dict(ok_four, scratch=20)
    assert any("four-waves" in p for p in b.check_resources([spilled, ok_h1, ok_split]))
    three = dict(ok_h1, occupancy=3)
    assert any("four-waves" in p for p in b.check_resources([ok_four, three, ok_split]))
    three_split = dict(ok_split, occupancy=3)
    assert any("four-waves" in p for p in b.check_resources([ok_four, ok_h1, three_split]))
    assert any("no kernel matches" in p for p in b.check_resources([ok_four]))
