"""skv_add_layernorm: residual add (bit-exact to the tensor-type add) + LayerNorm.

The sum is compared bit for bit with torch's x + y in the same dtype. The norm is
compared with float64 LayerNorm of that sum (population variance, eps) to one
rounding of the output type, and with torch's own LayerNorm of the same tensor.
"""
import pytest
import torch
import torch.nn.functional as F

from speech_serving import native

pytestmark = pytest.mark.gpu

ULP = {torch.float32: 2.0 ** -23, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}


def ln64(s, w, b, eps):
    s = s.double()
    mean = s.mean(-1, keepdim=True)
    var = ((s - mean) ** 2).mean(-1, keepdim=True)
    return (s - mean) / torch.sqrt(var + eps) * w.double() + b.double()


def check_norm(got, want, dtype, what):
    err = (got.double() - want).abs()
    tol = 1e-5 + 2 * ULP[dtype] * want.abs() + (1e-3 if dtype != torch.float32 else 1e-5)
    assert bool((err <= tol).all()), f"{what}: max err {float(err.max()):.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hidden", [32, 384, 768, 1280, 2048])
def test_add_layernorm_matches_reference(cuda, dtype, hidden):
    gen = torch.Generator().manual_seed(hidden)
    for rows in (1, 7, 64, 130):
        x = (torch.randn(rows, 1, hidden, generator=gen) * 3 + 0.5).to(cuda, dtype)
        y = torch.randn(rows, 1, hidden, generator=gen).to(cuda, dtype)
        w = (1 + 0.2 * torch.randn(hidden, generator=gen)).to(cuda, dtype)
        b = (0.2 * torch.randn(hidden, generator=gen)).to(cuda, dtype)
        s, n = native.add_layernorm(x, y, w, b, 1e-5)
        torch.cuda.synchronize()
        want_s = x + y
        assert torch.equal(s, want_s), f"sum rows={rows} hidden={hidden}"
        check_norm(n.cpu(), ln64(want_s.cpu(), w.cpu(), b.cpu(), 1e-5), dtype, f"norm rows={rows} hidden={hidden}")
        torch_n = F.layer_norm(want_s, (hidden,), w, b, 1e-5)
        err = (n.double() - torch_n.double()).abs().max().item()
        assert err <= 4 * ULP[dtype] * max(1.0, torch_n.abs().max().item()), f"vs torch layer_norm {err}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_layernorm_without_add_and_in_place_sum(cuda, dtype):
    gen = torch.Generator().manual_seed(5)
    rows, hidden = 48, 1280
    x = torch.randn(rows, hidden, generator=gen).to(cuda, dtype)
    y = torch.randn(rows, hidden, generator=gen).to(cuda, dtype)
    w = torch.randn(hidden, generator=gen).to(cuda, dtype)
    b = torch.randn(hidden, generator=gen).to(cuda, dtype)
    s0, n0 = native.add_layernorm(x, None, w, b, 1e-5)
    assert s0 is x
    check_norm(n0.cpu(), ln64(x.cpu(), w.cpu(), b.cpu(), 1e-5), dtype, "no add")
    want_s = x + y
    s1, n1 = native.add_layernorm(x, y, w, b, 1e-5, sum_out=x)  # in place
    torch.cuda.synchronize()
    assert s1 is x and torch.equal(x, want_s)
    check_norm(n1.cpu(), ln64(want_s.cpu(), w.cpu(), b.cpu(), 1e-5), dtype, "in place")


def test_add_layernorm_in_graph_replays(cuda):
    gen = torch.Generator().manual_seed(9)
    rows, hidden, dt = 64, 1280, torch.bfloat16
    x = torch.zeros(rows, hidden, dtype=dt, device=cuda)
    y = torch.zeros(rows, hidden, dtype=dt, device=cuda)
    w = torch.randn(hidden, generator=gen).to(cuda, dt)
    b = torch.randn(hidden, generator=gen).to(cuda, dt)
    s = torch.empty_like(x)
    native.add_layernorm(x, y, w, b, 1e-5, sum_out=s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _, n = native.add_layernorm(x, y, w, b, 1e-5, sum_out=s)
    for it in range(3):
        x.copy_(torch.randn(rows, hidden, generator=gen).to(cuda, dt))
        y.copy_(torch.randn(rows, hidden, generator=gen).to(cuda, dt))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(s, x + y)
        check_norm(n.cpu(), ln64((x + y).cpu(), w.cpu(), b.cpu(), 1e-5), dt, f"replay {it}")
