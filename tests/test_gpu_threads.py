"""The library keeps no per-call state: two host threads, each launching on its own stream
(default priority), interleave calls of the headline operator and of fused_add_rms_norm on
different inputs, and every result equals the one computed alone beforehand."""

import threading

import pytest
import torch

import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C.*)
from mcoplib_amd import op
from gpu_util import DEV, randn, say, weight

pytestmark = pytest.mark.gpu


def _case(seed, T, H):
    x = randn((T, H), seed, torch.bfloat16).to(DEV)
    r = randn((T, H), seed + 1, torch.bfloat16).to(DEV)
    w = weight(H, seed + 2, torch.bfloat16).to(DEV)
    return x, r, w


def _run(x, r, w):
    q = torch.empty(x.shape, dtype=torch.int8, device=DEV)
    s = torch.empty(x.shape[0], 1, device=DEV)
    rr = r.clone()
    op.rms_norm_dynamic_per_token_quant_custom(q, x, w, s, 1e-6, None, rr)
    x2, r2 = x.clone(), r.clone()
    torch.ops._C.fused_add_rms_norm(x2, r2, w, 1e-6)
    return q, s, rr, x2, r2


def test_two_threads_two_streams():
    say("threads: two host threads, two streams, interleaved calls")
    cases = [_case(10, 96, 5120), _case(20, 33, 7168)]
    expected = [_run(*c) for c in cases]
    torch.cuda.synchronize()
    errors = []

    def worker(i):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                for _ in range(30):
                    got = _run(*cases[i])
                    stream.synchronize()
                    for a, b in zip(got, expected[i]):
                        if not torch.equal(a, b):
                            errors.append(f"thread {i}: result differs")
                            return
        except Exception as e:  # reported by the main thread
            errors.append(f"thread {i}: {e!r}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads), "a thread did not finish"
    assert not errors, errors
