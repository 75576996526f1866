"""The kernels' per-element division by a per-row constant (mcop_fdiv_const, Markstein's
correction with guards) must be the IEEE binary32 quotient bit for bit.  The helper is plain
IEEE arithmetic, so it is compiled for the host with gcc and swept exhaustively over bf16
numerators and randomly over fp32 numerators (tests/fdiv_check.c)."""

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent


def test_fdiv_const_is_correctly_rounded(tmp_path):
    exe = tmp_path / "fdiv_check"
    subprocess.run(["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
                    "-Wall", "-o", str(exe), str(HERE / "fdiv_check.c"), "-lm"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    checked = int(out.stdout.split()[1])
    assert checked > 200_000_000
