"""The C-ABI library and the Python surfaces, without a GPU: the library loads, exports every
entry point include/mcop_norm.h declares, and rejects bad arguments before touching the device;
the Python surfaces reproduce the reference's argument checks."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

import mcoplib_amd
from mcoplib_amd import _lib, op, custom_ops

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mcop_norm.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mcop_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = _declared()
    assert "mcop_rms_norm_dynamic_per_token_quant" in names and len(names) >= 8
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for n in names:
        assert hasattr(lib, n), f"{n} declared in {HEADER.name} but not exported"


def test_every_header_is_served_by_a_built_library():
    """include/ holds the operator header only; it and the two non-operator headers (the test
    hooks of the operator library, the bench's pattern kernels) each belong to one in-tree
    library, which exports all the header declares."""
    assert sorted(p.name for p in (ROOT / "include").glob("*.h")) == ["mcop_norm.h"]
    libs = {ROOT / "include" / "mcop_norm.h": _lib.LIB_PATH,
            ROOT / "mcoplib_amd" / "csrc" / "mcop_testing.h": _lib.LIB_PATH,
            ROOT / "bench_kernels" / "mcop_pattern.h":
                ROOT / "bench_kernels" / "libmcop_pattern.so"}
    for header, path in libs.items():
        if not path.exists():
            pytest.skip(f"{path.name} not built")
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names = sorted(set(re.findall(r"\b(mcop_[a-z0-9_]+)\s*\(", text)))
        lib = ctypes.CDLL(str(path))
        assert names
        for n in names:
            assert hasattr(lib, n), f"{n} declared in {header.name} but not exported by {path.name}"


def test_operator_header_entries_cite_the_reference():
    """Every entry point of include/mcop_norm.h names the reference interface it replaces, or
    says why the reference has none (the error and version queries)."""
    text = HEADER.read_text()
    decls = [m.start() for m in re.finditer(r"^(?:int|const char\*) (mcop_[a-z0-9_]+)\s*\(",
                                             text, re.M)]
    assert len(decls) >= 12
    prev = 0
    for start in decls:
        comment = text[prev:start]
        prev = start
        assert ("Replaces" in comment or "reference" in comment), text[start:start + 80]


def test_abi_version_and_error_channel():
    assert _lib.lib.mcop_abi_version() == 2
    assert mcoplib_amd.LIBRARY_PATH.endswith("libmcop_norm.so")


def _err():
    return _lib.lib.mcop_last_error().decode()


def test_c_abi_rejects_bad_arguments_without_a_device():
    L = _lib.lib
    # zero rows: nothing to do
    assert L.mcop_rms_norm_dynamic_per_token_quant(None, 3, None, None, None, None, None, 0, 64,
                                                   0, 1e-6, None) == 0
    assert L.mcop_fused_add_rms_norm(None, 64, None, None, 0, 64, 0, 1e-6, None) == 0
    # bad shapes
    assert L.mcop_rms_norm_dynamic_per_token_quant(None, 3, None, None, None, None, None, 4, 0,
                                                   0, 1e-6, None) == -1
    assert "bad shape" in _err()
    assert L.mcop_fused_add_rms_norm(None, 32, None, None, 4, 64, 0, 1e-6, None) == -1
    assert "input_row_stride" in _err()
    assert L.mcop_scale_dynamic_quant(None, None, None, None, -1, 8, None) == -1
    # null pointers
    assert L.mcop_rms_norm_dynamic_per_token_quant(None, 3, None, None, None, None, None, 4, 64,
                                                   0, 1e-6, None) == -1
    assert "null pointer" in _err()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    # output dtype must be int8 / fp8
    assert L.mcop_rms_norm_dynamic_per_token_quant(p, 0, p, p, p, None, None, 4, 64, 0, 1e-6,
                                                   None) == -1
    assert "out dtype" in _err()
    # input dtype must be bf16 / fp16 / fp32
    assert L.mcop_rms_norm_dynamic_per_token_quant(p, 3, p, p, p, None, None, 4, 64, 3, 1e-6,
                                                   None) == -1
    assert "input dtype" in _err()
    assert L.mcop_fused_add_rms_norm(p, 64, p, p, 4, 64, 4, 1e-6, None) == -1
    # smooth quant: weight / smooth dtype combinations
    assert L.mcop_rms_norm_smooth_quant(p, 3, p, p, p, 1, p, 2, None, None, None, 4, 64, 0, 1e-6,
                                        0, None) == -1
    assert "weight dtype" in _err()
    assert L.mcop_rms_norm_smooth_quant(p, 3, p, p, p, 0, p, 2, None, None, None, 4, 64, 2, 1e-6,
                                        0, None) == -1
    assert "fp32 input" in _err()
    # launch override validation
    assert L.mcop_debug_set_launch_override(2, 100) == -1
    assert L.mcop_debug_set_launch_override(0, 0) == 0


def test_c_abi_rejects_shapes_beyond_the_kernels_without_a_device():
    """The launch limit is decided on the host before any HIP call: more rows than one
    launch's 2^31 - 1 workgroups, for register-resident and multi-pass launches."""
    L = _lib.lib
    p = ctypes.c_void_p(16)  # never dereferenced: every call below fails before a launch
    # 8-element rows: 16 lanes per row, 16 rows per workgroup; 2^36 rows need 2^32 workgroups
    assert L.mcop_scale_dynamic_quant(p, p, p, p, 1 << 36, 8, None) == -2
    assert "4294967296 workgroups" in _err()
    # multi-pass rows (one workgroup each): 2^31 rows
    assert L.mcop_scale_dynamic_quant(p, p, p, p, 1 << 31, 131072, None) == -2
    assert "2147483648 rows need more than" in _err()
    assert L.mcop_rms_norm_dynamic_per_token_quant(p, 3, p, p, p, None, None, 1 << 31, 131072,
                                                   0, 1e-6, None) == -2


def test_reference_checks_on_the_operator_surfaces():
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    w = torch.ones(64, dtype=torch.bfloat16)
    s = torch.zeros(4, 1)
    with pytest.raises(RuntimeError, match=r"Expected out.dtype\(\) == torch::kInt8"):
        op.rms_norm_dynamic_per_token_quant_custom(torch.empty(4, 64, dtype=torch.float16), x, w,
                                                   s, 1e-6)
    with pytest.raises(RuntimeError, match="scales.dtype"):
        op.rms_norm_dynamic_per_token_quant_custom(torch.empty(4, 64, dtype=torch.int8), x, w,
                                                   s.double(), 1e-6)
    with pytest.raises(RuntimeError, match="is_contiguous"):
        op.rms_norm_dynamic_per_token_quant_custom(torch.empty(64, 4, dtype=torch.int8).t(), x,
                                                   w, s, 1e-6)
    with pytest.raises(RuntimeError, match="not implemented for 'Int'"):
        op.rms_norm_dynamic_per_token_quant_custom(torch.empty(4, 64, dtype=torch.int8),
                                                   x.int(), w, s, 1e-6)
    # CPU tensors never reach the library
    with pytest.raises(RuntimeError, match="CUDA"):
        op.rms_norm_dynamic_per_token_quant_custom(torch.empty(4, 64, dtype=torch.int8), x, w, s,
                                                   1e-6)
    with pytest.raises(RuntimeError, match="CUDA"):
        custom_ops.rms_norm_dynamic_per_token_quant(x, w, 1e-6, torch.int8)
    with pytest.raises(RuntimeError):
        op.scale_dynamic_quant(x, torch.ones(64), torch.int8)
    sm = torch.ones(64)
    with pytest.raises(RuntimeError, match=r"out.dtype\(\) == torch::kInt8"):
        op.rms_norm_dynamic_per_token_quant(torch.empty(4, 64), x, w, sm, torch.zeros(4), 1e-6,
                                            torch.empty_like(x), torch.empty_like(x))


def test_torch_library_schemas_registered():
    import mcoplib_amd._C  # noqa: F401

    fa = torch.ops._C.fused_add_rms_norm.default._schema
    assert [a.name for a in fa.arguments] == ["input", "residual", "weight", "epsilon"]
    assert [a.alias_info is not None and a.alias_info.is_write for a in fa.arguments] == [
        True, True, False, False]
    assert len(fa.returns) == 0
    rq = torch.ops._C.rms_norm_dynamic_per_token_quant.default._schema
    assert [a.name for a in rq.arguments] == ["result", "input", "weight", "scale", "epsilon",
                                              "scale_ub", "residual"]
    assert [a.alias_info is not None and a.alias_info.is_write for a in rq.arguments] == [
        True, False, False, True, False, False, True]
    assert len(rq.returns) == 0
    # no CPU implementation: the dispatcher refuses CPU tensors
    x = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        torch.ops._C.fused_add_rms_norm(x, x.clone(), torch.ones(64, dtype=torch.bfloat16), 1e-6)
    # the CUDA implementations apply the reference's checks before any device work
    from mcoplib_amd import _C
    with pytest.raises(RuntimeError, match="weight.scalar_type"):
        _C.fused_add_rms_norm(x, x.clone(), torch.ones(64), 1e-6)
    with pytest.raises(RuntimeError, match="kFp8Type"):
        _C.rms_norm_dynamic_per_token_quant(
            torch.empty(4, 64, dtype=torch.int8), x, torch.ones(64, dtype=torch.bfloat16),
            torch.zeros(4, 1), 1e-6, torch.ones(1), None)


def test_c_caller_library_links_the_abi():
    """tests/c_caller/libabi_example.so (the plain C caller the GPU tests drive) loads without a
    device, exports its four examples and binds the operator entry points of libmcop_norm.so."""
    path = ROOT / "tests" / "c_caller" / "libabi_example.so"
    if not path.exists():
        pytest.skip("tests/c_caller is not built (make -C tests/c_caller)")
    lib = ctypes.CDLL(str(path))
    for n in ("example_fused_add_rms_norm", "example_rms_norm_quant",
              "example_rms_norm_smooth_quant", "example_scale_dynamic_quant"):
        assert hasattr(lib, n), n
    import subprocess
    syms = subprocess.run(["nm", "-D", "--undefined-only", str(path)], capture_output=True,
                          text=True, check=True).stdout
    for n in ("mcop_fused_add_rms_norm", "mcop_rms_norm_dynamic_per_token_quant",
              "mcop_rms_norm_smooth_quant", "mcop_scale_dynamic_quant", "mcop_last_error",
              "hipStreamCreate", "hipMalloc"):
        assert n in syms, n
