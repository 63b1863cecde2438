"""The Whisper-large-v3 decode path at its full sizes, through the C ABI (bf16, 20 heads x 64, block size 16):

- paged self-attention with the fused append at batch 64 and 128 (ctx U[1, 452] in drawn order, tables from a
  permuted pool), against the float64 oracle, and the appended rows in the pool bit for bit;
- cross-attention over each request's 1500 encoder positions at batch 64, against the float64 oracle;
- the encoder K/V store (64 requests x 1500 positions appended through a permuted slot map) gathered back bit for
  bit: the append -> gather round trip at the size of one layer's encoder K/V.

Bar: max |out - oracle| <= 2e-3 + 2^-8 |oracle| (the bf16 output's relative half-ulp), as in the other tests.
The attention outputs are also held to the rounding step itself: each bf16 output is the float64 result
rounded to bf16 or one of that value's two bf16 neighbours (an fp32 result within 2^-16 of the float64 one,
rounded once, can land no further)."""
import numpy as np
import pytest
import torch

from oracle import paged_kv as O
from speech_serving import native

pytestmark = pytest.mark.gpu

H, D, BS = 20, 64, 16
REL_BF16 = 2.0 ** -8


def f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def check(got, want, what):
    err = np.abs(f64(got) - want)
    tol = 2e-3 + REL_BF16 * np.abs(want)
    assert (err <= tol).all(), f"{what}: max err {err.max():.3e}"
    return float(err.max())


def bf16_ulp(x):
    """Spacing of the bf16 values at |x| (8 significant bits; the subnormal spacing below 2^-126)."""
    a = np.maximum(np.abs(x), np.float64(2.0 ** -126))
    return np.exp2(np.floor(np.log2(a)) - 7)


def check_bf16_rounding(got, want, what):
    """got (bf16) is want rounded to bf16, or a neighbour of that value: |got - rne(want)| <= ulp + 2^-16.
    Returns the fraction of outputs equal to the rounded float64 result."""
    g = f64(got)
    r = torch.from_numpy(want).to(torch.bfloat16).double().numpy()  # round to nearest even
    gap = np.abs(g - r)
    bound = bf16_ulp(r) + 2.0 ** -16
    bad = gap > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} outputs beyond one bf16 step of the rounded float64 result, "
                           f"worst gap {gap.max():.3e}")
    return float((gap == 0).mean())


@pytest.mark.parametrize("bsz", [64, 128])
def test_large_v3_paged_attention_fused_append(cuda, bsz):
    gen = torch.Generator().manual_seed(900 + bsz)
    max_ctx, maxblk = 452, 29  # 29 blocks of 16 hold 452 keys
    nb = bsz * maxblk + 64
    ctx = torch.randint(1, max_ctx + 1, (bsz,), generator=gen)
    ctx[bsz // 2] = max_ctx
    tables = torch.randperm(nb, generator=gen)[: bsz * maxblk].view(bsz, maxblk).to(torch.int32)
    kp = torch.randn(nb, BS, H, D, generator=gen).to(cuda, torch.bfloat16)
    vp = torch.randn(nb, BS, H, D, generator=gen).to(cuda, torch.bfloat16)
    q, kn, vn = (torch.randn(bsz, H, D, generator=gen).to(cuda, torch.bfloat16) for _ in range(3))
    out = native.paged_attention(q, kp, vp, tables.to(cuda), ctx.to(torch.int32).to(cuda), max_ctx, 0.125,
                                 k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    # The new key of row b went to its position ctx[b] - 1 through the table.
    pos = ctx - 1
    blk = tables[torch.arange(bsz), pos // BS].long().to(cuda)
    off = (pos % BS).to(cuda)
    assert torch.equal(kp[blk, off], kn) and torch.equal(vp[blk, off], vn)
    want = O.paged_attention(f64(q)[:, None], f64(kp), f64(vp), tables.numpy(), ctx.tolist(), 0.125)[:, 0]
    err = check(out, want, f"large-v3 paged attention, batch {bsz}")
    exact = check_bf16_rounding(out, want, f"large-v3 paged attention, batch {bsz}")
    print(f"large-v3 paged attention with fused append, batch {bsz}: max err {err:.2e}, "
          f"{exact:.4f} of outputs equal the rounded float64 result, the rest one bf16 step from it")


def test_large_v3_cross_attention(cuda):
    gen = torch.Generator().manual_seed(910)
    b, t = 64, 1500
    kv = torch.randn(b, 2, H, t, D, generator=gen).to(cuda, torch.bfloat16)
    q = torch.randn(b, 1, H, D, generator=gen).to(cuda, torch.bfloat16)
    lens = [t] * (b - 4) + [1, 700, t - 1, 0]
    out = native.dense_attention(q, kv[:, 0], kv[:, 1], torch.tensor(lens, dtype=torch.int32, device=cuda), t,
                                 0.125)
    torch.cuda.synchronize()
    want = O.dense_attention(f64(q), f64(kv[:, 0]), f64(kv[:, 1]), lens, 0.125)
    err = check(out, want, "large-v3 cross-attention")
    exact = check_bf16_rounding(out, want, "large-v3 cross-attention")
    assert np.all(f64(out)[-1] == 0.0)  # an empty row gives zeros
    print(f"large-v3 cross-attention, batch 64 x 1500 positions: max err {err:.2e}, "
          f"{exact:.4f} of outputs equal the rounded float64 result, the rest one bf16 step from it")


def test_large_v3_encoder_store_round_trip(cuda):
    gen = torch.Generator().manual_seed(920)
    b, t = 64, 1500
    per = -(-t // BS)  # 94 blocks per request
    nb = b * per + 16
    tables = torch.randperm(nb, generator=gen)[: b * per].view(b, per).to(torch.int32)
    src_k = torch.randn(b * t, H, D, generator=gen).to(cuda, torch.bfloat16)
    src_v = torch.randn(b * t, H, D, generator=gen).to(cuda, torch.bfloat16)
    slots = np.concatenate([O.slot_mapping(tables[r].tolist(), range(t), BS) for r in range(b)])
    kp = torch.zeros(nb, BS, H, D, dtype=torch.bfloat16, device=cuda)
    vp = torch.zeros_like(kp)
    native.append(src_k, src_v, kp, vp, torch.from_numpy(slots).to(cuda))
    ko, vo = native.gather(kp, vp, tables.to(cuda), torch.full((b,), t, dtype=torch.int32, device=cuda), t)
    torch.cuda.synchronize()
    assert torch.equal(ko, src_k.view(b, t, H, D).permute(0, 2, 1, 3))
    assert torch.equal(vo, src_v.view(b, t, H, D).permute(0, 2, 1, 3))
