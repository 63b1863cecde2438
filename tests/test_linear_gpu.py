"""skv_linear (hipBLASLt with a plan cached per shape) against torch's linear and a float64 product.

The decoder step's projections (speech_serving/models.py:127-207 in the reference, the LM head :416/:486)
run through it: the large-v3 decode shapes must give torch's linear bit for bit (same algorithm), every
shape must stay within the rounding of the output dtype of the float64 product, and a captured graph must
replay what the eager calls gave.
"""
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from speech_serving import models, native

pytestmark = pytest.mark.gpu

# (n, k, bias): the large-v3 decoder's projections (fused q/k/v, output, MLP in and out, LM head).
LARGE_V3 = [(3840, 1280, False), (1280, 1280, False), (5120, 1280, True), (1280, 5120, True), (51866, 1280, False)]


def _data(m, n, k, dt, bias, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(m, k, generator=g, device="cuda").to(dt)
    w = (torch.randn(n, k, generator=g, device="cuda") * 0.02).to(dt)
    b = torch.randn(n, generator=g, device="cuda").to(dt) if bias else None
    return x, w, b


def _within_rounding(y, x, w, b):
    """|y - float64 product| within half an output ulp plus the fp32 accumulation's error bound."""
    ref = x.double() @ w.double().t()
    if b is not None:
        ref = ref + b.double()
    k = x.shape[-1]
    eps_out = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -24}[y.dtype]
    mag = x.double().abs() @ w.double().abs().t() + (b.double().abs() if b is not None else 0)
    tol = eps_out * ref.abs() + k * 2.0 ** -24 * mag + 1e-30
    err = (y.double() - ref).abs()
    assert bool((err <= tol).all()), f"max excess {float((err - tol).max()):.3g}"


@pytest.mark.parametrize("m", [1, 8, 64, 128])
@pytest.mark.parametrize("n,k,bias", LARGE_V3)
def test_linear_large_v3_equals_torch_linear(cuda, m, n, k, bias):
    x, w, b = _data(m, n, k, torch.bfloat16, bias, 100 + m)
    y = native.linear(x, w, b)
    assert torch.equal(y, F.linear(x, w, b))
    _within_rounding(y, x, w, b)


@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,n,k,bias", [(4, 384, 384, False), (4, 1536, 384, True), (3, 384, 1536, True),
                                        (4, 51865, 384, False), (5, 512, 768, True), (2, 4096, 256, False)])
def test_linear_within_rounding_of_float64(cuda, dt, m, n, k, bias):
    x, w, b = _data(m, n, k, dt, bias, 7)
    y = native.linear(x, w, b)
    assert y.shape == (m, n) and y.dtype == dt
    _within_rounding(y, x, w, b)


def test_linear_strided_rows_batch_dims_and_empty(cuda):
    x, w, b = _data(24, 512, 256, torch.bfloat16, True, 3)
    big = torch.zeros(24, 300, device="cuda", dtype=torch.bfloat16)
    big[:, :256] = x
    xs = big[:, :256]  # rows 300 elements apart
    assert xs.stride(0) == 300
    assert torch.equal(native.linear(xs, w, b), native.linear(x, w, b))
    x3 = x.view(4, 6, 256)
    y3 = native.linear(x3, w, b)
    assert y3.shape == (4, 6, 512) and torch.equal(y3.view(24, 512), native.linear(x, w, b))
    assert native.linear(x[:0], w, b).shape == (0, 512)
    xb = x[:1].expand(24, 256)  # rows broadcast from one (row stride 0)
    assert torch.equal(native.linear(xb, w, b), F.linear(xb.contiguous(), w, b))


def test_linear_graph_replays_equal_eager(cuda):
    x, w, b = _data(64, 1280, 1280, torch.bfloat16, True, 11)
    xin = x.clone()
    native.linear(xin, w, b)  # plan built outside capture
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        native.linear(xin, w, b)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        yg = native.linear(xin, w, b)
    for seed in range(4):
        xn, _, _ = _data(64, 1280, 1280, torch.bfloat16, False, 50 + seed)
        xin.copy_(xn)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, native.linear(xn, w, b))


def test_linear_rejects_mismatches(cuda):
    x, w, b = _data(4, 64, 32, torch.bfloat16, True, 1)
    with pytest.raises(RuntimeError):
        native.linear(x, w.float(), b)
    with pytest.raises(RuntimeError):
        native.linear(x, w[:, :16], b)
    with pytest.raises(RuntimeError):
        native.linear(x, w, b[:8])
    with pytest.raises(RuntimeError):
        native.linear(x.cpu(), w, b)
    with pytest.raises(RuntimeError):
        native.linear(x, w.t(), None)  # weight rows not contiguous


def test_proj_runs_hooks_and_other_modules_as_modules(cuda):
    lin = nn.Linear(32, 16).cuda().to(torch.bfloat16)
    x = torch.randn(4, 32, device="cuda", dtype=torch.bfloat16)
    assert torch.equal(models.proj(lin, x), lin(x))
    seen = []
    h = lin.register_forward_hook(lambda mod, inp, out: seen.append(out.shape))
    try:
        models.proj(lin, x)
    finally:
        h.remove()
    assert seen == [torch.Size([4, 16])]  # the hooked module was called as a module
    seq = nn.Sequential(nn.Linear(32, 64), nn.GELU(), nn.Linear(64, 32)).cuda().to(torch.bfloat16)
    assert torch.equal(models.mlp(seq, x), seq(x))
