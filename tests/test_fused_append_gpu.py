"""Fused append + paged attention (skv_paged_attention with k_new/v_new).

The pool after the call must equal the oracle's append at positions
ctx-Q .. ctx-1 through each row's block table (bit-exact), and the output
must match the oracle's attention over the appended pool (tolerance as in
test_kernels_gpu).
"""
import math

import numpy as np
import pytest
import torch

from oracle import paged_kv as O
from speech_serving import native

from test_kernels_gpu import assert_close, f64, make_pool, make_tables

pytestmark = pytest.mark.gpu


def run_case(cuda, dtype, bsz, qlen, h, hkv, d, bs, nb, ctx, causal, seed, chunk=0, table_rows=None):
    gen = torch.Generator().manual_seed(seed)
    kp, vp = make_pool(gen, nb, bs, hkv, d, dtype, cuda)
    maxblk = -(-max(ctx) // bs) + 1
    ntab = bsz if table_rows is None else max(table_rows) + 1
    tables = make_tables(gen, ntab, nb, maxblk)
    q = torch.randn(bsz, qlen, h, d, generator=gen).to(cuda, dtype)
    kn = torch.randn(bsz, qlen, hkv, d, generator=gen).to(cuda, dtype)
    vn = torch.randn(bsz, qlen, hkv, d, generator=gen).to(cuda, dtype)
    pool_k, pool_v = f64(kp), f64(vp)
    tr = None if table_rows is None else torch.tensor(table_rows, dtype=torch.int32, device=cuda)
    out = native.paged_attention(q, kp, vp, tables.to(cuda), torch.tensor(ctx, dtype=torch.int32, device=cuda),
                                 max(ctx), 1 / math.sqrt(d), causal=causal, table_rows=tr, k_new=kn, v_new=vn,
                                 chunk_tokens=chunk)
    torch.cuda.synchronize()
    # oracle: append the new rows through the table, then attend
    rows_tbl = tables.numpy() if table_rows is None else tables.numpy()[table_rows]
    pk, pv = pool_k.copy(), pool_v.copy()
    for b in range(bsz):
        pos = list(range(ctx[b] - qlen, ctx[b]))
        slots = O.slot_mapping(rows_tbl[b].tolist(), pos, bs)
        O.append(pk, pv, f64(kn[b]), f64(vn[b]), slots)
    assert np.array_equal(f64(kp), pk) and np.array_equal(f64(vp), pv), "pool after fused append"
    want = O.paged_attention(f64(q), pk, pv, rows_tbl, ctx, 1 / math.sqrt(d), causal=causal)
    return out, want, None


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bs", [16, 32, 64])
def test_fused_decode_append(cuda, dtype, bs):
    out, want, _ = run_case(cuda, dtype, 16, 1, 8, 8, 64, bs, 512, [1, 2, 15, 16, 17, 100, 255, 256, 257, 300,
                                                                   448, 64, 65, 31, 32, 33], False, 1)
    assert_close(out, want, dtype, f"fused decode bs={bs}")


@pytest.mark.parametrize("chunk", [0, 256, 512])
def test_fused_prompt_append_causal(cuda, chunk):
    out, want, _ = run_case(cuda, torch.float16, 3, 4, 4, 4, 64, 16, 128, [4, 37, 300], True, 2, chunk=chunk)
    assert_close(out, want, torch.float16, "fused prompt")


def test_fused_gqa_and_row_indirection(cuda):
    out, want, _ = run_case(cuda, torch.bfloat16, 4, 1, 8, 2, 64, 8, 256, [9, 1, 64, 200], False, 3,
                            table_rows=[2, 0, 5, 3])
    assert_close(out, want, torch.bfloat16, "fused gqa")


def test_fused_equals_separate_append_then_attend(cuda):
    """Same bytes in the pool as skv_append followed by skv_paged_attention, and the same output up to
    the summation order (the fused decode scores the new key before the pool keys)."""
    gen = torch.Generator().manual_seed(4)
    bsz, h, d, bs, nb = 32, 20, 64, 16, 2048
    ctx = torch.randint(1, 453, (bsz,), generator=gen)
    tables = make_tables(gen, bsz, nb, 29)
    kp, vp = make_pool(gen, nb, bs, h, d, torch.bfloat16, cuda)
    kp2, vp2 = kp.clone(), vp.clone()
    q = torch.randn(bsz, h, d, generator=gen).to(cuda, torch.bfloat16)
    kn = torch.randn(bsz, h, d, generator=gen).to(cuda, torch.bfloat16)
    vn = torch.randn(bsz, h, d, generator=gen).to(cuda, torch.bfloat16)
    ctx_d = ctx.to(torch.int32).to(cuda)
    tab_d = tables.to(cuda)
    fused = native.paged_attention(q, kp, vp, tab_d, ctx_d, 452, 0.125, k_new=kn, v_new=vn)
    pos = (ctx - 1).tolist()
    slots = torch.tensor([int(tables[i, p // bs]) * bs + p % bs for i, p in enumerate(pos)], dtype=torch.int64)
    native.append(kn, vn, kp2, vp2, slots.to(cuda))
    sep = native.paged_attention(q, kp2, vp2, tab_d, ctx_d, 452, 0.125)
    torch.cuda.synchronize()
    assert torch.equal(kp, kp2) and torch.equal(vp, vp2)
    assert_close(fused, f64(sep), torch.bfloat16, "fused vs separate")
    # Both against the oracle over the appended pool.
    want = O.paged_attention(f64(q)[:, None], f64(kp2), f64(vp2), tables.numpy(), ctx.tolist(), 0.125)[:, 0]
    assert_close(fused, want, torch.bfloat16, "fused")
    assert_close(sep, want, torch.bfloat16, "separate")
