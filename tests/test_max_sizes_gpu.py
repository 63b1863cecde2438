"""The kernels at the sizes where their addressing changes form.

* A paged pool past 2 GiB per layer: the paged attention leaves its buffer-descriptor path (32-bit byte
  offsets) for 64-bit addressing, and the fused append writes rows beyond the 2 GiB mark.
* A gather whose output holds 2^31 or more 16-byte vectors (B x H x T x D past 32 GiB) and an append of
  that many vectors: both leave their 32-bit index kernels for 64-bit ones.

Bars as elsewhere: attention within 2e-3 (+ half an output ulp) of the float64 oracle, append and gather
bit-exact (compared as raw 16-bit words). Reference sites: append speech_serving/phase_aware_scheduler.py:
1004-1010, gather speech_serving/tts_engine.py:177-185, attention speech_serving/models.py:140-164.
"""
import math

import numpy as np
import pytest
import torch

from oracle import paged_kv as O
from speech_serving import native

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _release_memory():
    torch.cuda.empty_cache()
    yield
    torch.cuda.empty_cache()


def test_paged_attention_and_append_in_a_pool_past_2gib(cuda):
    dt, h, d, bs, nb = torch.bfloat16, 16, 64, 16, 70000  # 2.29 GB per pool
    assert nb * bs * h * d * 2 > 2 ** 31
    gen = torch.Generator().manual_seed(77)
    ctx = [1, 17, 300, 1000, 16, 999]
    b = len(ctx)
    maxblk = (max(ctx) + bs - 1) // bs
    # Block ids from the top of the pool: every row's K/V and appended rows lie past 2 GiB.
    used = (nb - 1 - torch.randperm(9000, generator=gen)[: b * maxblk]).to(torch.int32)
    tables = used.view(b, maxblk)
    kp = torch.empty(nb, bs, h, d, dtype=dt, device=cuda)
    vp = torch.empty(nb, bs, h, d, dtype=dt, device=cuda)
    ids = used.long().to(cuda)
    kp[ids] = torch.randn(len(used), bs, h, d, generator=gen).to(cuda, dt)
    vp[ids] = torch.randn(len(used), bs, h, d, generator=gen).to(cuda, dt)
    q = torch.randn(b, h, d, generator=gen).to(cuda, dt)
    kn = torch.randn(b, h, d, generator=gen).to(cuda, dt)
    vn = torch.randn(b, h, d, generator=gen).to(cuda, dt)
    scale = 1.0 / math.sqrt(d)
    lens = torch.tensor(ctx, dtype=torch.int32, device=cuda)
    # Expected: the new rows written at position ctx-1 of each row, then attention, on a compact copy.
    kc = kp[ids].double().cpu().numpy()
    vc = vp[ids].double().cpu().numpy()
    compact = np.arange(b * maxblk, dtype=np.int64).reshape(b, maxblk)
    slots = [int(compact[r, (c - 1) // bs]) * bs + (c - 1) % bs for r, c in enumerate(ctx)]
    O.append(kc, vc, kn.double().cpu().numpy(), vn.double().cpu().numpy(), slots)
    want = O.paged_attention(q.double().cpu().numpy()[:, None], kc, vc, compact, ctx, scale)[:, 0]
    out = native.paged_attention(q, kp, vp, tables.to(cuda), lens, max(ctx), scale, k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    err = np.abs(out.double().cpu().numpy() - want)
    assert (err <= 2e-3 + 2.0 ** -8 * np.abs(want)).all(), f"max err {err.max():.3e}"
    for r, c in enumerate(ctx):  # the appended rows, bit for bit, past 2 GiB
        blk = int(tables[r, (c - 1) // bs])
        assert torch.equal(kp[blk, (c - 1) % bs].view(torch.int16), kn[r].view(torch.int16))
        assert torch.equal(vp[blk, (c - 1) % bs].view(torch.int16), vn[r].view(torch.int16))


def test_gather_past_2_31_vectors(cuda):
    dt, b, h, d, bs, nb, t = torch.bfloat16, 129, 32, 64, 16, 4096, 65536
    assert b * h * t * d * 2 // 16 >= 2 ** 31  # the output's 16-byte vectors need 64-bit indices
    g = torch.Generator(device=cuda).manual_seed(5)
    kp = torch.randint(-2 ** 15, 2 ** 15, (nb, bs, h, d), generator=g, dtype=torch.int16, device=cuda).view(dt)
    tables = torch.argsort(torch.rand(b, nb, generator=g, device=cuda), dim=1).to(torch.int32)
    lens = torch.randint(0, t + 1, (b,), generator=g, device=cuda, dtype=torch.int32)
    lens[0], lens[1], lens[2], lens[-1] = t, 0, 1, t - 1
    out, _ = native.gather(kp, None, tables, lens, t)
    torch.cuda.synchronize()
    pos = torch.arange(t, device=cuda)
    for r in range(b):
        want = kp[tables[r].long()].reshape(t, h, d).transpose(0, 1).view(torch.int16)
        want = torch.where((pos < lens[r])[None, :, None], want, torch.zeros_like(want))
        assert torch.equal(out[r].view(torch.int16), want), f"row {r} (len {int(lens[r])})"
    del out, kp


def test_append_past_2_31_vectors(cuda):
    dt, h, d, bs = torch.bfloat16, 32, 64, 16
    n = (1 << 23) + 3  # n * h * d * 2 / 16 > 2^31 vectors
    nb = n // bs + 2
    g = torch.Generator(device=cuda).manual_seed(6)
    kn = torch.randint(-2 ** 15, 2 ** 15, (n, h, d), generator=g, dtype=torch.int16, device=cuda).view(dt)
    kp = torch.zeros(nb, bs, h, d, dtype=dt, device=cuda)
    slots = torch.randperm(nb * bs, generator=g, device=cuda)[:n]
    slots[:: 1_000_003] = -1  # skipped rows
    native.append(kn, None, kp, None, slots)
    torch.cuda.synchronize()
    rows = kp.view(nb * bs, h, d).view(torch.int16)
    src = kn.view(torch.int16)
    step = 1 << 20
    for i in range(0, n, step):
        s = slots[i:i + step]
        ok = s >= 0
        assert torch.equal(rows[s[ok]], src[i:i + step][ok]), f"tokens {i}..{i + step}"
    written = torch.zeros(nb * bs, dtype=torch.bool, device=cuda)
    written[slots[slots >= 0]] = True
    untouched = (~written).nonzero().squeeze(1)
    assert untouched.numel() > 0 and not rows[untouched].any()
    del kn, kp, rows
