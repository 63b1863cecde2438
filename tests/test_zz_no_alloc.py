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


def test_noalloc_refuses_partials_beyond_its_scratch(cuda):
    # 64 rows x 32 heads x 16 chunks of 64 keys x (64 + 4) floats = 8.9 MB of partials > 4 MiB.
    p = problem(cuda, torch.float16, 64, 32, 64, 16, 4096, 1024, 3, fused=False)
    with pytest.raises(RuntimeError, match="scratch"):
        native.paged_attention(p["q"], p["kp"], p["vp"], p["tables"].to(cuda), p["ctx"].to(torch.int32).to(cuda),
                               1024, 0.125, chunk_tokens=64, noalloc=True)
