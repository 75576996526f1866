"""The reference's own caller lines run verbatim against this package (CPU: imports, schemas and
the surfaces' argument checks; the GPU suites exercise the same names on a device)."""

import subprocess
import sys

from conftest import ROOT

# README.md:149,155 and unit_test/test_rms_norm_custom.py:2 of the reference, then the schemas
# of op/vllm/torch_bindings.cpp:155-164,216-229,359-364,374-379 as this torch prints them
_SCRIPT = r'''
from mcoplib import op as ops
import mcoplib._C
from mcoplib.custom_ops import rms_norm_dynamic_per_token_quant
import torch
import mcoplib, mcoplib_amd
assert ops is mcoplib_amd.op and mcoplib.op is ops
assert mcoplib._C is mcoplib_amd._C
assert rms_norm_dynamic_per_token_quant is mcoplib_amd.custom_ops.rms_norm_dynamic_per_token_quant
for name in ("rms_norm_dynamic_per_token_quant", "rms_norm_dynamic_per_token_quant_custom",
             "scale_dynamic_quant", "fused_add_rms_norm_dynamic_per_token_quant_padding_output",
             "rms_norm", "head_rms_norm"):
    assert callable(getattr(ops, name)), name
for name in ("rms_norm", "fused_add_rms_norm", "rms_norm_dynamic_per_token_quant",
             "rms_norm_per_block_quant", "dynamic_scaled_int8_quant",
             "dynamic_per_token_scaled_fp8_quant"):
    print(name, "|", getattr(torch.ops._C, name).default._schema)
'''

_SCHEMA_ARGS = {
    "rms_norm": "result, Tensor input, Tensor weight, float epsilon) -> ()",
    "fused_add_rms_norm": "input, Tensor($1! -> ) residual, Tensor weight, float epsilon) -> ()",
    "rms_norm_dynamic_per_token_quant": "Tensor weight, Tensor($1! -> ) scale, float epsilon, "
                                        "Tensor? scale_ub, Tensor($2! -> )? residual) -> ()",
    "rms_norm_per_block_quant": "Tensor? scale_ub, Tensor($2! -> )? residual, int group_size, "
                                "bool is_scale_transposed) -> ()",
    "dynamic_scaled_int8_quant": "scale, Tensor($2! -> )? azp) -> ()",
    "dynamic_per_token_scaled_fp8_quant": "scale, Tensor? scale_ub) -> ()",
}


def test_reference_caller_lines_import_this_package():
    out = subprocess.run([sys.executable, "-c", _SCRIPT], cwd=str(ROOT), capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    got = dict(line.split(" | ", 1) for line in out.stdout.strip().splitlines())
    for name, tail in _SCHEMA_ARGS.items():
        assert got[name].startswith(f"_C::{name}("), got[name]
        assert got[name].endswith(tail), got[name]
