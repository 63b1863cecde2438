"""skv_paged_attention_noalloc — the allocation-free variant of skv_paged_attention (split-K partials
in the library's fixed per-device scratch) — against skv_paged_attention on the same inputs, through
the C ABI: two calls in a row, the second smaller, both bit-equal to the workspace entry point and
within the attention bar of the float64 oracle; a call whose partials exceed the scratch is refused
before anything launches."""
import math

import numpy as np
import pytest
import torch

from oracle import paged_kv as O
from speech_serving import native

pytestmark = pytest.mark.gpu


def problem(cuda, dtype, batch, heads, d, bs, nb, max_ctx, seed, fused):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(1, max_ctx + 1, (batch,), generator=g)
    ctx[0] = max_ctx
    maxblk = math.ceil(max_ctx / bs)
    tables = torch.randperm(nb, generator=g)[: batch * maxblk].view(batch, maxblk).to(torch.int32)
    kp = torch.randn(nb, bs, heads, d, generator=g).to(cuda, dtype)
    vp = torch.randn(nb, bs, heads, d, generator=g).to(cuda, dtype)
    q = torch.randn(batch, heads, d, generator=g).to(cuda, dtype)
    kn = vn = None
    if fused:
        kn = torch.randn(batch, heads, d, generator=g).to(cuda, dtype)
        vn = torch.randn(batch, heads, d, generator=g).to(cuda, dtype)
    return dict(q=q, kp=kp, vp=vp, tables=tables, ctx=ctx, kn=kn, vn=vn, max_ctx=max_ctx)


def run(p, cuda, noalloc):
    kp, vp = p["kp"].clone(), p["vp"].clone()
    out = torch.empty_like(p["q"])
    native.paged_attention(p["q"], kp, vp, p["tables"].to(cuda), p["ctx"].to(torch.int32).to(cuda), p["max_ctx"],
                           1.0 / math.sqrt(p["q"].shape[-1]), out=out, k_new=p["kn"], v_new=p["vn"],
                           noalloc=noalloc)
    torch.cuda.synchronize()
    return out, kp, vp


def test_noalloc_graph_replays_equal_eager_calls(cuda):
    """A split-K call captured into a HIP graph (run alone, this file makes the device's first
    allocation-free call inside the capture, where the scratch address is looked up): replays with new
    queries, with eager work and a sync between them, are bit-equal to eager calls of both entry points."""
    dtype = torch.bfloat16
    p = problem(cuda, dtype, 4, 8, 64, 16, 512, 1500, 5, fused=False)
    assert native.attention_workspace_bytes(4, 8, 64, p["max_ctx"], dtype) > 0  # split-K is exercised
    tables, ctx = p["tables"].to(cuda), p["ctx"].to(torch.int32).to(cuda)
    scale = 1.0 / 8.0
    q_static = p["q"].clone()
    out_static = torch.empty_like(q_static)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        native.paged_attention(q_static, p["kp"], p["vp"], tables, ctx, p["max_ctx"], scale, out=out_static,
                               noalloc=True)
    gen = torch.Generator().manual_seed(6)
    for i in range(4):
        q_new = torch.randn(q_static.shape, generator=gen).to(cuda, dtype)
        q_static.copy_(q_new)
        g.replay()
        torch.cuda.synchronize()
        got = out_static.clone()
        eager_noalloc = native.paged_attention(q_new, p["kp"], p["vp"], tables, ctx, p["max_ctx"], scale,
                                               noalloc=True)
        eager_ws = native.paged_attention(q_new, p["kp"], p["vp"], tables, ctx, p["max_ctx"], scale)
        torch.cuda.synchronize()
        assert torch.equal(got, eager_noalloc), f"replay {i}"
        assert torch.equal(got, eager_ws), f"replay {i}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_noalloc_matches_the_workspace_entry_point_twice(cuda, dtype):
    # A few (row, head) pairs over long contexts: the keys split into chunks, so the partials go
    # through the scratch. The second call is smaller and must not see the first call's partials.
    first = problem(cuda, dtype, 4, 8, 64, 16, 512, 1500, 1, fused=True)
    second = problem(cuda, dtype, 2, 4, 64, 16, 128, 600, 2, fused=False)
    for p in (first, second):
        rows, heads = p["q"].shape[0], p["q"].shape[1]
        assert native.attention_workspace_bytes(rows, heads, 64, p["max_ctx"], dtype) > 0  # split-K is exercised
        want_out, want_k, want_v = run(p, cuda, noalloc=False)
        got_out, got_k, got_v = run(p, cuda, noalloc=True)
        assert torch.equal(got_out, want_out)
        assert torch.equal(got_k, want_k) and torch.equal(got_v, want_v)
        kp, vp = got_k.double().cpu().numpy(), got_v.double().cpu().numpy()
        ref = O.paged_attention(p["q"].double().cpu().numpy()[:, None], kp, vp, p["tables"].numpy(),
                                p["ctx"].tolist(), 1.0 / 8.0)[:, 0]
        half_ulp = 2.0 ** -11 if dtype == torch.float16 else 2.0 ** -8
        err = np.abs(got_out.double().cpu().numpy() - ref)
        assert (err <= 2e-3 + half_ulp * np.abs(ref)).all(), float(err.max())


def test_noalloc_encoder_attention_needs_no_scratch(cuda):
    """Encoder attention over a paged table (1500 queries x 8 heads) takes the 64-query kernel, which
    keeps each row's keys in one workgroup: no partials, so the call is accepted even with a chunk size
    whose split-K partials would exceed the scratch, and it equals the workspace entry point."""
    g = torch.Generator().manual_seed(9)
    dtype, heads, d, bs, t = torch.bfloat16, 8, 64, 16, 1500
    nblk = -(-t // bs)
    kp = torch.randn(nblk + 4, bs, heads, d, generator=g).to(cuda, dtype)
    vp = torch.randn(nblk + 4, bs, heads, d, generator=g).to(cuda, dtype)
    tables = torch.randperm(nblk + 4, generator=g)[:nblk].view(1, nblk).to(torch.int32).to(cuda)
    q = torch.randn(1, t, heads, d, generator=g).to(cuda, dtype)
    lens = torch.tensor([t], dtype=torch.int32, device=cuda)
    # chunk 64: 1500 query rows x 8 heads x 24 chunks of (64 + 4) floats = 78 MB of partials, were they used
    assert native.attention_workspace_bytes(t, heads, d, t, dtype, 64) > (4 << 20)
    got = native.paged_attention(q, kp, vp, tables, lens, t, 0.125, chunk_tokens=64, noalloc=True)
    want = native.paged_attention(q, kp, vp, tables, lens, t, 0.125)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_noalloc_refuses_partials_beyond_its_scratch(cuda):
    # 64 rows x 32 heads x 16 chunks of 64 keys x (64 + 4) floats = 8.9 MB of partials > 4 MiB.
    p = problem(cuda, torch.float16, 64, 32, 64, 16, 4096, 1024, 3, fused=False)
    with pytest.raises(RuntimeError, match="scratch"):
        native.paged_attention(p["q"], p["kp"], p["vp"], p["tables"].to(cuda), p["ctx"].to(torch.int32).to(cuda),
                               1024, 0.125, chunk_tokens=64, noalloc=True)
