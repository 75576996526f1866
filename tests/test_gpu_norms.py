"""GPU parity of the RMSNorms without quantization against the CPU oracle, bit for bit:
``mcoplib_amd.op.rms_norm`` and ``op.head_rms_norm`` (both reference rounding chains, both sides
of the reference's vectorized / element-wise switch) and ``torch.ops._C.rms_norm`` (2-D, 3-D and
4-D inputs with strided rows); plus the reference's own asserting tests
(unit_test/test_rms_norm.py, unit_test/test_head_rms_norm.py) run on the GPU output."""

import pytest
import torch

import oracle
import mcoplib_amd._C  # noqa: F401  (registers torch.ops._C.*)
from mcoplib_amd import _lib, op
from gpu_util import DEV, assert_exact, say

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _mc_case(T, H, dtype, wdtype, with_res, rms_div, seed, x_scale=2.0):
    tag = f"rms_norm T={T} H={H} {dtype} w={wdtype} res={with_res} div={rms_div}"
    g = _gen(seed)
    x = (torch.randn(T, H, generator=g) * x_scale).to(dtype)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(wdtype)
    r = torch.randn(T, H, generator=g).to(dtype) if with_res else None
    out_ref, ares_ref = oracle.rms_norm(x, w, 1e-6, residual=r, rms_div=rms_div)
    out = torch.empty((T, H), dtype=dtype, device=DEV)
    ares = torch.empty((T, H), dtype=dtype, device=DEV) if with_res else None
    op.rms_norm(out, x.to(DEV), w.to(DEV), 1e-6, ares, None if r is None else r.to(DEV), rms_div)
    torch.cuda.synchronize()
    assert_exact(out, out_ref, tag + " out")
    if with_res:
        assert_exact(ares, ares_ref, tag + " after_res")


@pytest.mark.parametrize("dtype,wdtype,H", [
    (torch.bfloat16, torch.bfloat16, 4096), (torch.bfloat16, torch.bfloat16, 1030),
    (torch.bfloat16, torch.bfloat16, 24576), (torch.bfloat16, torch.bfloat16, 32768),
    (torch.bfloat16, torch.float32, 7168), (torch.float16, torch.float16, 5120),
    (torch.float16, torch.float32, 12296), (torch.float32, torch.float32, 4096),
    (torch.float32, torch.float32, 1026), (torch.float32, torch.float32, 16384),
    (torch.bfloat16, torch.bfloat16, 64), (torch.float16, torch.float16, 1),
])
@pytest.mark.parametrize("T", [1, 83, 1024])
def test_mc_rms_norm(dtype, wdtype, H, T):
    say(f"mc rms_norm T={T} H={H} {dtype} w={wdtype}")
    for with_res in (False, True):
        for rms_div in (True, False):
            _mc_case(T, H, dtype, wdtype, with_res, rms_div, T * 13 + H)


def test_reference_rms_norm_test():
    say("reference unit_test/test_rms_norm.py (fp32 4096 x 4096)")
    m = n = 4096
    torch.manual_seed(42)
    h = torch.randn(m, n, device=DEV)
    r = torch.randn(m, n, device=DEV)
    w = torch.randn(n, device=DEV)
    after_ref = h + r
    rms = torch.rsqrt(torch.mean(after_ref * after_ref, dim=-1, keepdim=True) + 1e-5)
    norm_ref = after_ref / rms * w
    norm = torch.empty(m, n, device=DEV)
    ares = torch.empty(m, n, device=DEV)
    op.rms_norm(norm, h, w, 1e-5, ares, r, True)
    torch.testing.assert_close(norm_ref, norm, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(after_ref.reshape(-1), ares.reshape(-1), atol=1e-5, rtol=1e-5)


def _head_case(T, NH, D, off, hn, dtype, wdtype, seed):
    tag = f"head_rms_norm T={T} NH={NH} D={D} heads [{off},{off + hn}) {dtype} w={wdtype}"
    g = _gen(seed)
    hs = torch.randn(T, NH, D, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(NH, D, generator=g)).to(wdtype)
    base = torch.randn(T, NH, D, generator=g).to(dtype)
    ref = oracle.head_rms_norm(base, hs, w, 1e-6, off, hn)
    out = base.to(DEV)
    op.head_rms_norm(out, hs.to(DEV), w.to(DEV), 1e-6, off, hn)
    torch.cuda.synchronize()
    assert_exact(out, ref, tag)


@pytest.mark.parametrize("T,NH,D,off,hn", [(128, 32, 128, 0, 8), (7, 64, 128, 32, 32),
                                           (3, 8, 4096, 2, 4), (2, 4, 12288, 1, 2),
                                           (2, 4, 24584, 0, 4), (5, 6, 100, 1, 5),
                                           (1, 1, 64, 0, 1)])
@pytest.mark.parametrize("dtype,wdtype", [(torch.bfloat16, torch.bfloat16),
                                          (torch.bfloat16, torch.float32),
                                          (torch.float16, torch.bfloat16),
                                          (torch.float32, torch.float32),
                                          (torch.float32, torch.bfloat16)])
def test_head_rms_norm(T, NH, D, off, hn, dtype, wdtype):
    say(f"head_rms_norm T={T} NH={NH} D={D} {dtype} {wdtype}")
    _head_case(T, NH, D, off, hn, dtype, wdtype, T * NH + D)


@pytest.mark.parametrize("D", [4096, 4096 * 2, 4096 * 3])
def test_reference_head_rms_norm_test(D):
    say(f"reference unit_test/test_head_rms_norm.py D={D}")
    T, NH, hn = 128, 128, 64
    torch.manual_seed(42)
    hs = torch.randn(T, NH, D, device=DEV)
    w = torch.randn(NH, D, device=DEV)
    ref = hs.clone()
    for h in range(hn):
        sel = hs[:, h, :]
        var = sel.pow(2).mean(-1, keepdim=True)
        ref[:, h, :] = w[h, :] * (sel / torch.rsqrt(var + 1e-5))
    out = hs.clone()
    op.head_rms_norm(out, hs, w, 1e-5, 0, hn)
    torch.testing.assert_close(ref, out, atol=1e-5, rtol=1e-5)


def _vllm_case(x_dev, w, tag):
    x_cpu = x_dev.cpu()
    ref = oracle.vllm_rms_norm(x_cpu.contiguous(), w, 1e-6)
    out = torch.empty(x_dev.shape, dtype=x_dev.dtype, device=DEV)
    torch.ops._C.rms_norm(out, x_dev, w.to(DEV), 1e-6)
    torch.cuda.synchronize()
    assert_exact(out, ref, tag)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_vllm_rms_norm_exact_row_layouts(dtype):
    """Rows that fill their workgroup exactly (4096-wide, at most 256 of them) take the kernel's
    exact-row form: 2-D row-strided and 3-D views of a fused buffer."""
    say(f"vllm rms_norm exact-row layouts {dtype}")
    g = _gen(6)
    H = 4096
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype)
    wide = (torch.randn(64, 3 * H, generator=g)).to(dtype).to(DEV)
    _vllm_case(wide[:, H:2 * H], w, "2-D strided rows")
    qkv = torch.randn(16, 3 * 8 * H, generator=g).to(dtype).to(DEV)
    _vllm_case(qkv[:, : 8 * H].view(16, 8, H), w, "3-D q view of qkv")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_vllm_rms_norm_layouts(dtype):
    say(f"vllm rms_norm layouts {dtype}")
    g = _gen(5)
    H = 128
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype)
    # 2-D contiguous and row-strided
    x = (torch.randn(300, H, generator=g) * 2).to(dtype).to(DEV)
    _vllm_case(x, w, "2-D contiguous")
    wide = (torch.randn(300, 3 * H, generator=g)).to(dtype).to(DEV)
    _vllm_case(wide[:, H:2 * H], w, "2-D strided rows")
    # 3-D [batch, heads, head_size] viewed out of a fused qkv buffer
    qkv = torch.randn(40, 3 * 8 * H, generator=g).to(dtype).to(DEV)
    q = qkv[:, : 8 * H].view(40, 8, H)
    _vllm_case(q, w, "3-D q view of qkv")
    # 4-D [batch, seq, head, head_dim] with a permuted (non-contiguous) layout
    base = torch.randn(2, 8, 5, H, generator=g).to(dtype).to(DEV)  # [b, head, seq, d]
    _vllm_case(base.permute(0, 2, 1, 3), w, "4-D permuted")
    # last dimension not contiguous: the reference copies it first
    t = torch.randn(H, 50, generator=g).to(dtype).to(DEV)
    _vllm_case(t.t(), w, "transposed (copied)")


@pytest.mark.parametrize("T,H", [(1, 4096), (83, 5120), (2048, 8192), (5, 16384), (7, 1029),
                                 (4096, 64)])
def test_vllm_rms_norm_shapes(T, H):
    say(f"vllm rms_norm T={T} H={H}")
    for dtype in (torch.bfloat16, torch.float32):
        g = _gen(T + H)
        x = torch.randn(T, H, generator=g).to(dtype)
        w = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype)
        _vllm_case(x.to(DEV), w, f"vllm T={T} H={H} {dtype}")


@pytest.mark.parametrize("nv", [1, 2, 4, 8, 16])
def test_launch_shape_does_not_change_bits(nv):
    say(f"norms launch override nv={nv}")
    try:
        _lib.set_launch_override(nv, 0)
        _mc_case(129, 4096, torch.bfloat16, torch.bfloat16, True, True, 3)
        _mc_case(129, 4096, torch.float16, torch.float32, False, False, 4)
        _head_case(9, 16, 4096, 4, 8, torch.bfloat16, torch.float32, 5)
        g = _gen(6)
        x = torch.randn(129, 4096, generator=g).to(torch.bfloat16)
        w = (1 + 0.1 * torch.randn(4096, generator=g)).to(torch.bfloat16)
        _vllm_case(x.to(DEV), w, "vllm override")
    finally:
        _lib.set_launch_override(0, 0)


def test_argument_errors():
    say("norm argument checks")
    x = torch.randn(4, 64, device=DEV, dtype=torch.bfloat16)
    w = torch.ones(64, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError):  # residual without after_res
        op.rms_norm(torch.empty_like(x), x, w, 1e-6, None, x.clone(), True)
    with pytest.raises(RuntimeError):  # fp16 weight for head norm
        op.head_rms_norm(torch.empty(2, 4, 64, device=DEV, dtype=torch.float16),
                         torch.empty(2, 4, 64, device=DEV, dtype=torch.float16),
                         torch.ones(4, 64, device=DEV, dtype=torch.float16), 1e-6, 0, 2)
    with pytest.raises(RuntimeError):  # heads out of range
        op.head_rms_norm(torch.empty(2, 4, 64, device=DEV, dtype=torch.bfloat16),
                         torch.empty(2, 4, 64, device=DEV, dtype=torch.bfloat16),
                         torch.ones(4, 64, device=DEV, dtype=torch.bfloat16), 1e-6, 3, 2)
    with pytest.raises(RuntimeError):  # rank 1
        torch.ops._C.rms_norm(torch.empty(64, device=DEV, dtype=torch.bfloat16),
                              torch.ones(64, device=DEV, dtype=torch.bfloat16), w, 1e-6)
