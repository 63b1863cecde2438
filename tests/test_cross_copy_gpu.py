"""skv_copy_cross_kv: a request's encoder K/V for every decoder layer into its decode slot, one launch.

The bar is bit-exact: the slot region after the call must hold the same bytes as the reference's per-layer
copies (graph_decode_buffers.py:317-327, `g_cross_kv[slot, l, 0, :, :n].copy_(ck[0, :, :n])`), and every
byte outside the copied positions must be unchanged.
"""
import pytest
import torch

from speech_serving import native

pytestmark = pytest.mark.gpu


def reference_copy(dst, ks, vs, n):
    for l, (k, v) in enumerate(zip(ks, vs)):
        dst[l, 0, :, :n].copy_(k[:, :n])
        dst[l, 1, :, :n].copy_(v[:, :n])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("layers,heads,t_src,t_max,n,d", [
    (32, 20, 1500, 1500, 1500, 64),   # large-v3 shape, whole encoder
    (6, 8, 1500, 1500, 731, 64),      # base shape, shorter valid length
    (4, 4, 1600, 1500, 1500, 64),     # source longer than the slot: truncated to the slot
    (2, 3, 17, 40, 17, 128),
    (3, 2, 9, 9, 1, 32),
])
def test_copy_matches_per_layer_copies(cuda, dtype, layers, heads, t_src, t_max, n, d):
    gen = torch.Generator(device=cuda).manual_seed(layers * 100 + n)
    slots = 2
    g = torch.randn(slots, layers, 2, heads, t_max, d, generator=gen, device=cuda).to(dtype)
    want = g.clone()
    ks = [torch.randn(1, heads, t_src, d, generator=gen, device=cuda).to(dtype)[0] for _ in range(layers)]
    vs = [torch.randn(1, heads, t_src, d, generator=gen, device=cuda).to(dtype)[0] for _ in range(layers)]
    native.copy_cross_kv(ks, vs, g[1], n)
    reference_copy(want[1], ks, vs, n)
    torch.cuda.synchronize()
    assert torch.equal(g.view(torch.uint8), want.view(torch.uint8))


def test_strided_and_mixed_sources(cuda):
    """Sources with other strides (a transposed cache view, a sliced tensor, another dtype) give the same bytes."""
    gen = torch.Generator().manual_seed(7)
    layers, heads, t, d = 5, 4, 300, 64
    g = torch.zeros(2, layers, 2, heads, t, d, dtype=torch.bfloat16, device=cuda)
    want = g.clone()
    base = torch.randn(layers, t, heads, d, generator=gen).to(cuda, torch.bfloat16)
    ks = [base[l].transpose(0, 1) for l in range(layers)]                      # [H, T, D] with head stride D
    vs = [torch.randn(heads, t + 50, d, generator=gen).to(cuda, torch.float32)[:, 25:25 + t] for _ in range(layers)]
    native.copy_cross_kv(ks, vs, g[0], 257)
    reference_copy(want[0], ks, vs, 257)
    torch.cuda.synchronize()
    assert torch.equal(g.view(torch.int16), want.view(torch.int16))


def test_more_layers_than_one_launch_holds(cuda):
    gen = torch.Generator().manual_seed(8)
    layers, heads, t, d = native.MAX_CROSS_LAYERS + 6, 2, 33, 64
    g = torch.zeros(1, layers, 2, heads, t, d, dtype=torch.float16, device=cuda)
    want = g.clone()
    ks = [torch.randn(heads, t, d, generator=gen).to(cuda, torch.float16) for _ in range(layers)]
    vs = [torch.randn(heads, t, d, generator=gen).to(cuda, torch.float16) for _ in range(layers)]
    native.copy_cross_kv(ks, vs, g[0], t)
    reference_copy(want[0], ks, vs, t)
    torch.cuda.synchronize()
    assert torch.equal(g.view(torch.int16), want.view(torch.int16))


def test_copy_inside_a_graph_replays(cuda):
    """The launch records into a HIP graph; every replay copies the sources' current contents."""
    gen = torch.Generator().manual_seed(9)
    layers, heads, t, d = 4, 4, 100, 64
    g = torch.zeros(1, layers, 2, heads, t, d, dtype=torch.bfloat16, device=cuda)
    ks = [torch.zeros(heads, t, d, dtype=torch.bfloat16, device=cuda) for _ in range(layers)]
    vs = [torch.zeros(heads, t, d, dtype=torch.bfloat16, device=cuda) for _ in range(layers)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        native.copy_cross_kv(ks, vs, g[0], t)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        native.copy_cross_kv(ks, vs, g[0], t)
    for rep in range(3):
        for x in ks + vs:
            x.copy_(torch.randn(heads, t, d, generator=gen).to(cuda, torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = torch.zeros_like(g)
        reference_copy(want[0], ks, vs, t)
        assert torch.equal(g.view(torch.int16), want.view(torch.int16)), f"replay {rep}"
