"""GPU parity of the HIP kernels (through the C ABI) against the CPU oracle.

Bars:
  * append / gather: bit-exact (compared as raw bytes).
  * attention: max |out - oracle| <= 2e-3 + r*|oracle|, where r is the
    output dtype's relative half-ulp (fp32 0, fp16 2^-11, bf16 2^-8): the
    kernel returns the fp32 result rounded once to the tensor dtype, as the
    reference's own fp16/bf16 outputs are. The oracle computes in float64 from
    the same (already rounded) inputs.
"""
import math

import numpy as np
import pytest
import torch

from oracle import paged_kv as O
from speech_serving import native

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
REL = {torch.float32: 0.0, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}


def f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def raw(t):
    return t.detach().cpu().contiguous().view(torch.uint8).numpy() if t.dtype != torch.bfloat16 else \
        t.detach().cpu().contiguous().view(torch.int16).numpy()


def assert_close(got, want, dtype, what=""):
    g = f64(got)
    err = np.abs(g - want)
    tol = 2e-3 + REL[dtype] * np.abs(want)
    bad = err > tol
    assert not bad.any(), f"{what}: max err {err.max():.3e} at {np.argwhere(bad)[:3].tolist()} (dtype {dtype})"
    return float(err.max())


def make_pool(gen, nb, bs, h, d, dtype, device):
    k = torch.randn(nb, bs, h, d, generator=gen, dtype=torch.float32).to(device=device, dtype=dtype)
    v = torch.randn(nb, bs, h, d, generator=gen, dtype=torch.float32).to(device=device, dtype=dtype)
    return k, v


def make_tables(gen, nrows, nb, maxblk):
    perm = torch.randperm(nb, generator=gen)[: nrows * maxblk]
    return perm.view(nrows, maxblk).to(torch.int32)


# ------------------------------------------------------------------ append
@pytest.mark.parametrize("dtype", DTYPES)
def test_append_bit_exact(cuda, dtype):
    gen = torch.Generator().manual_seed(1)
    nb, bs, h, d = 24, 16, 4, 64
    kp, vp = make_pool(gen, nb, bs, h, d, dtype, cuda)
    kp0, vp0 = kp.clone(), vp.clone()
    n = 9
    k_new = torch.randn(n, h, d, generator=gen).to(cuda, dtype)
    v_new = torch.randn(n, h, d, generator=gen).to(cuda, dtype)
    slots = torch.randperm(nb * bs, generator=gen)[:n].to(torch.int64)
    slots[3] = -1
    native.append(k_new, v_new, kp, vp, slots.to(cuda))
    torch.cuda.synchronize()
    want_k, want_v = kp0.cpu().clone(), vp0.cpu().clone()
    for i, s in enumerate(slots.tolist()):  # the reference's index_put form
        if s >= 0:
            want_k[s // bs, s % bs] = k_new[i].cpu()
            want_v[s // bs, s % bs] = v_new[i].cpu()
    assert np.array_equal(raw(kp), raw(want_k)) and np.array_equal(raw(vp), raw(want_v))


def test_append_from_strided_cache_view(cuda):
    """new_k = keys[b, :, -1, :] of a [B, H, T, D] cache (phase_aware_scheduler.py:1007-1008)."""
    gen = torch.Generator().manual_seed(2)
    bsz, h, t, d, nb, bs = 5, 4, 7, 64, 16, 8
    keys = torch.randn(bsz, h, t, d, generator=gen).to(cuda, torch.float16)
    vals = torch.randn(bsz, h, t, d, generator=gen).to(cuda, torch.float16)
    kp = torch.zeros(nb, bs, h, d, dtype=torch.float16, device=cuda)
    vp = torch.zeros_like(kp)
    slots = torch.tensor([3, 17, 40, 63, 100], dtype=torch.int64)
    native.append(keys[:, :, -1, :], vals[:, :, -1, :], kp, vp, slots.to(cuda))
    pk = kp.cpu().numpy().copy() * 0
    pv = pk.copy()
    O.append(pk, pv, keys[:, :, -1, :].cpu().numpy(), vals[:, :, -1, :].cpu().numpy(), slots.tolist())
    assert np.array_equal(kp.cpu().numpy(), pk) and np.array_equal(vp.cpu().numpy(), pv)


# ------------------------------------------------------------------ gather
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("bs", [8, 16])
def test_gather_bit_exact(cuda, dtype, bs):
    gen = torch.Generator().manual_seed(3)
    nb, h, d, maxblk = 64, 3, 64, 6
    kp, vp = make_pool(gen, nb, bs, h, d, dtype, cuda)
    tables = make_tables(gen, 4, nb, maxblk)
    lens = [0, 1, bs * maxblk, 2 * bs + 3]
    tmax = bs * maxblk
    ko, vo = native.gather(kp, vp, tables.to(cuda), torch.tensor(lens, dtype=torch.int32, device=cuda), tmax)
    torch.cuda.synchronize()
    want_k = O.gather(kp.cpu().float().numpy(), tables.numpy(), lens, tmax)
    want_v = O.gather(vp.cpu().float().numpy(), tables.numpy(), lens, tmax)
    assert np.array_equal(ko.cpu().float().numpy(), want_k)
    assert np.array_equal(vo.cpu().float().numpy(), want_v)
    # bytes, not just values: compare against torch indexing of the same pool
    for b, n in enumerate(lens):
        if n:
            nblk = -(-n // bs)
            ref = kp[tables[b, :nblk].long().to(cuda)].view(-1, h, d)[:n].permute(1, 0, 2)
            assert np.array_equal(raw(ko[b, :, :n]), raw(ref))


@pytest.mark.parametrize("bs,tmax", [(5, 29), (16, 29), (16, 2), (3, 31)])
def test_gather_ragged_lengths_and_invalid_ids(cuda, bs, tmax):
    """Output lengths that are not a multiple of the kernel's 4-row groups, block sizes that are not
    a multiple of 4, lengths beyond the output (clamped) and beyond the table row, and block ids
    outside the pool (zeros), against the oracle."""
    gen = torch.Generator().manual_seed(bs * 100 + tmax)
    nb, h, d, maxblk = 64, 2, 32, 7
    kp, vp = make_pool(gen, nb, bs, h, d, torch.float16, cuda)
    tables = make_tables(gen, 6, nb, maxblk)
    tables[1, 1] = -1
    tables[2, 0] = nb + 3
    lens = [tmax, 1, min(tmax, 2 * bs + 1), tmax + 5, 0, bs * maxblk + 9]
    ko, vo = native.gather(kp, vp, tables.to(cuda), torch.tensor(lens, dtype=torch.int32, device=cuda), tmax)
    want_k = O.gather(kp.cpu().float().numpy(), tables.numpy(), lens, tmax)
    want_v = O.gather(vp.cpu().float().numpy(), tables.numpy(), lens, tmax)
    assert np.array_equal(ko.cpu().float().numpy(), want_k)
    assert np.array_equal(vo.cpu().float().numpy(), want_v)


@pytest.mark.parametrize("dtype,d,bs", [(torch.bfloat16, 128, 16), (torch.float16, 64, 64), (torch.float32, 32, 8),
                                         (torch.bfloat16, 16, 32), (torch.float16, 16, 16), (torch.bfloat16, 80, 16)])
def test_gather_row_widths_and_block_sizes(cuda, dtype, d, bs):
    """Row widths of 1-16 16-byte vectors and block sizes 8-64: the wave path (8 lanes per 128-byte row,
    a block id per load instruction) where the block holds one instruction's rows, the per-thread path
    otherwise (16-wide bf16 rows in 16-key blocks; 80-wide rows). Output lengths that are not a multiple
    of the wave's 32-row groups, lengths past the output, ids outside the pool: against the oracle."""
    gen = torch.Generator().manual_seed(d * 10 + bs)
    nb, h, maxblk, tmax = 48, 3, 5, 5 * bs - 3
    kp, vp = make_pool(gen, nb, bs, h, d, dtype, cuda)
    tables = make_tables(gen, 5, nb, maxblk)
    tables[3, 2] = nb
    lens = [tmax, 1, 0, 3 * bs + 1, tmax + 7]
    ko, vo = native.gather(kp, vp, tables.to(cuda), torch.tensor(lens, dtype=torch.int32, device=cuda), tmax)
    want_k = O.gather(kp.cpu().float().numpy(), tables.numpy(), lens, tmax)
    want_v = O.gather(vp.cpu().float().numpy(), tables.numpy(), lens, tmax)
    assert np.array_equal(ko.cpu().float().numpy(), want_k)
    assert np.array_equal(vo.cpu().float().numpy(), want_v)


def test_append_then_gather_round_trip(cuda):
    gen = torch.Generator().manual_seed(4)
    nb, bs, h, d, n = 128, 16, 8, 64, 300
    kp = torch.zeros(nb, bs, h, d, dtype=torch.bfloat16, device=cuda)
    vp = torch.zeros_like(kp)
    table = torch.randperm(nb, generator=gen)[: -(-n // bs)].to(torch.int32)
    src_k = torch.randn(n, h, d, generator=gen).to(cuda, torch.bfloat16)
    src_v = torch.randn(n, h, d, generator=gen).to(cuda, torch.bfloat16)
    slots = torch.from_numpy(O.slot_mapping(table.tolist(), range(n), bs)).to(cuda)
    native.append(src_k, src_v, kp, vp, slots)
    ko, vo = native.gather(kp, vp, table[None].to(cuda), torch.tensor([n], dtype=torch.int32, device=cuda), n)
    assert torch.equal(ko[0], src_k.permute(1, 0, 2)) and torch.equal(vo[0], src_v.permute(1, 0, 2))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bs", [16, 12])  # the fast path (block ids per trip), the general path (staged in LDS)
def test_paged_attention_few_rows_long_context_default_split(cuda, dtype, bs):
    """2 rows x 4 heads over 4000 / 1700 keys: too few (row, head) pairs for the GPU and too many keys for one
    workgroup each, so the default chunk splits the keys (partials in the workspace, combined by the merge
    launch); with the new key appended through the table."""
    gen = torch.Generator().manual_seed(300 + bs)
    h, d, lens = 4, 64, [4000, 1700]
    assert native.attention_workspace_bytes(len(lens), h, d, max(lens), dtype) > 0  # the keys are split
    maxblk = -(-max(lens) // bs)
    nb = 2 * maxblk + 4
    kp, vp = make_pool(gen, nb, bs, h, d, dtype, cuda)
    tables = make_tables(gen, len(lens), nb, maxblk)
    q = torch.randn(len(lens), h, d, generator=gen).to(cuda, dtype)
    kn = torch.randn(len(lens), h, d, generator=gen).to(cuda, dtype)
    vn = torch.randn(len(lens), h, d, generator=gen).to(cuda, dtype)
    out = native.paged_attention(q, kp, vp, tables.to(cuda), torch.tensor(lens, dtype=torch.int32, device=cuda),
                                 max(lens), 0.125, k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    want = O.paged_attention(f64(q)[:, None], f64(kp), f64(vp), tables.numpy(), lens, 0.125)[:, 0]
    err = assert_close(out, want, dtype, f"default split, block size {bs}")
    print(f"few rows, long context, {dtype}, block size {bs}: max err {err:.2e}")


# ------------------------------------------------------------------ paged attention
@pytest.mark.parametrize("bsz,h,bs,max_ctx", [(64, 16, 16, 4100), (64, 16, 8, 2100), (64, 16, 12, 4100),
                                               (8, 20, 6, 1500)])
def test_paged_attention_long_context_default_chunk(cuda, bsz, h, bs, max_ctx):
    """Rows whose default chunk would span more than the general path's 254 staged block ids. Power-of-two
    blocks (the fast path, block ids read per trip) take one chunk per row; block sizes of 12 and 6 (the
    general path) get the default chunk capped at 254 blocks (rows split, partials merged)."""
    gen = torch.Generator().manual_seed(bs + max_ctx)
    d, dtype = 64, torch.bfloat16
    lens = [max_ctx, (max_ctx * 3) // 4] + torch.randint(1, 41, (bsz - 2,), generator=gen).tolist()
    maxblk = -(-max_ctx // bs)
    need = [-(-n // bs) for n in lens]
    nb = sum(need) + 8
    chunk = native.paged_chunk_tokens(bsz, h, h, d, max_ctx, dtype, bs, nb)
    if bs & (bs - 1):
        assert chunk // bs + 2 <= 256 and chunk < max_ctx, chunk
    else:
        assert chunk == native.default_chunk_tokens(bsz, h, d, max_ctx, dtype), chunk
    kp, vp = make_pool(gen, nb, bs, h, d, dtype, cuda)
    perm = torch.randperm(nb, generator=gen).to(torch.int32)
    tables = torch.full((bsz, maxblk), -1, dtype=torch.int32)
    at = 0
    for i, n in enumerate(need):
        tables[i, :n] = perm[at:at + n]
        at += n
    q = torch.randn(bsz, h, d, generator=gen).to(cuda, dtype)
    out = native.paged_attention(q, kp, vp, tables.to(cuda), torch.tensor(lens, dtype=torch.int32, device=cuda),
                                 max_ctx, 0.125)
    torch.cuda.synchronize()
    want = O.paged_attention(f64(q)[:, None], f64(kp), f64(vp), tables.numpy(), lens, 0.125)[:, 0]
    err = assert_close(out, want, dtype, f"long context bs={bs} max_ctx={max_ctx}")
    print(f"long context, default chunk {chunk}, block size {bs}: max err {err:.2e}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("d", [16, 32, 64, 128])
@pytest.mark.parametrize("bs", [8, 16, 32, 64, 12])  # 32, 64: blocks longer than a wave's trip; 12: general path
def test_paged_attention_matches_oracle(cuda, dtype, d, bs):
    gen = torch.Generator().manual_seed(100 + d + bs)
    nb, h, maxblk = 256, 4, 12
    kp, vp = make_pool(gen, nb, bs, h, d, dtype, cuda)
    lens = [0, 1, bs, bs + 1, 5, maxblk * bs, maxblk * bs - 1, 77 % (maxblk * bs)]
    bsz = len(lens)
    tables = make_tables(gen, bsz, nb, maxblk)
    q = torch.randn(bsz, h, d, generator=gen).to(cuda, dtype)
    scale = 1.0 / math.sqrt(d)
    out = native.paged_attention(q, kp, vp, tables.to(cuda), torch.tensor(lens, dtype=torch.int32, device=cuda),
                                 max(lens), scale)
    torch.cuda.synchronize()
    want = O.paged_attention(f64(q)[:, None], f64(kp), f64(vp), tables.numpy(), lens, scale)[:, 0]
    assert_close(out, want, dtype, f"paged d={d} bs={bs}")
    assert not out[0].any()  # zero visible keys -> zeros
    if dtype == torch.float32:
        assert torch.equal(out[1], vp[tables[1, 0].item(), 0].to(out.dtype))  # one key -> that value


def test_paged_attention_config2_full_size(cuda):
    """Kernel microbench shape: fp16, 32 heads x 64, 1 layer, BS 16, batch 64,
    ctx U[1, 448], tables from a seeded permutation of a 4096-block pool, N(0,1)."""
    gen = torch.Generator().manual_seed(2024)
    bsz, h, d, bs, nb = 64, 32, 64, 16, 4096
    ctx = torch.randint(1, 449, (bsz,), generator=gen)
    maxblk = 28
    tables = make_tables(gen, bsz, nb, maxblk)
    kp, vp = make_pool(gen, nb, bs, h, d, torch.float16, cuda)
    q = torch.randn(bsz, h, d, generator=gen).to(cuda, torch.float16)
    out = native.paged_attention(q, kp, vp, tables.to(cuda), ctx.to(torch.int32).to(cuda), 448, 1 / 8.0)
    torch.cuda.synchronize()
    want = O.paged_attention(f64(q)[:, None], f64(kp), f64(vp), tables.numpy(), ctx.tolist(), 1 / 8.0)[:, 0]
    err = assert_close(out, want, torch.float16, "fp16 H32 B64 microbench")
    print(f"fp16 H32 B64 microbench paged attention max abs err {err:.3e}")


@pytest.mark.parametrize("bsz,h", [(20, 20), (13, 31), (64, 20), (3, 2), (100, 3)])
def test_paged_attention_every_row_head_once(cuda, bsz, h):
    """Grids of rows x heads workgroups that end in a full, a partial even and a partial odd round of
    workgroups per compute unit (the launch maps workgroups to (row, head) items in rounds, the odd ones
    reversed): every (row, head) output matches the oracle, rows sorted longest-first as the engine sends them."""
    gen = torch.Generator().manual_seed(1000 + bsz * h)
    d, bs, nb = 64, 16, bsz * 13
    ctx = torch.randint(1, 200, (bsz,), generator=gen).sort(descending=True).values.to(torch.int32)
    tables = make_tables(gen, bsz, nb, 13)
    kp, vp = make_pool(gen, nb, bs, h, d, torch.float16, cuda)
    q = torch.randn(bsz, h, d, generator=gen).to(cuda, torch.float16)
    out = native.paged_attention(q, kp, vp, tables.to(cuda), ctx.to(cuda), 200, 0.125)
    torch.cuda.synchronize()
    want = O.paged_attention(f64(q)[:, None], f64(kp), f64(vp), tables.numpy(), ctx.tolist(), 0.125)[:, 0]
    assert_close(out, want, torch.float16, f"{bsz}x{h}")


@pytest.mark.parametrize("chunk", [64, 128, 256, 512])
def test_paged_attention_split_sizes_agree_and_repeat(cuda, chunk):
    gen = torch.Generator().manual_seed(5)
    bsz, h, d, bs, nb = 16, 8, 64, 16, 1024
    ctx = torch.randint(1, 449, (bsz,), generator=gen).to(torch.int32)
    tables = make_tables(gen, bsz, nb, 28)
    kp, vp = make_pool(gen, nb, bs, h, d, torch.bfloat16, cuda)
    q = torch.randn(bsz, h, d, generator=gen).to(cuda, torch.bfloat16)
    args = (q, kp, vp, tables.to(cuda), ctx.to(cuda), 448, 0.125)
    a = native.paged_attention(*args, chunk_tokens=chunk)
    b = native.paged_attention(*args, chunk_tokens=chunk)  # deterministic merge order
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    want = O.paged_attention(f64(q)[:, None], f64(kp), f64(vp), tables.numpy(), ctx.tolist(), 0.125)[:, 0]
    assert_close(a, want, torch.bfloat16, f"chunk {chunk}")


def test_paged_attention_causal_multi_query(cuda):
    """Prompt attention: Q new tokens, each sees the cached prefix plus itself and earlier prompt tokens."""
    gen = torch.Generator().manual_seed(6)
    bsz, qlen, h, d, bs, nb = 3, 4, 4, 64, 16, 64
    kp, vp = make_pool(gen, nb, bs, h, d, torch.float16, cuda)
    tables = make_tables(gen, bsz, nb, 8)
    ctx = [4, 37, 128]
    q = torch.randn(bsz, qlen, h, d, generator=gen).to(cuda, torch.float16)
    out = native.paged_attention(q, kp, vp, tables.to(cuda), torch.tensor(ctx, dtype=torch.int32, device=cuda),
                                 128, 0.125, causal=True)
    want = O.paged_attention(f64(q), f64(kp), f64(vp), tables.numpy(), ctx, 0.125, causal=True)
    assert_close(out, want, torch.float16, "causal")


def test_paged_attention_table_row_indirection_and_gqa(cuda):
    gen = torch.Generator().manual_seed(7)
    bsz, h, hkv, d, bs, nb = 5, 8, 2, 64, 16, 128
    kp, vp = make_pool(gen, nb, bs, hkv, d, torch.float32, cuda)
    tables = make_tables(gen, 9, nb, 10)
    rows = [8, 0, 3, 3, 5]
    ctx = [160, 1, 20, 99, 50]
    q = torch.randn(bsz, h, d, generator=gen).to(cuda)
    out = native.paged_attention(q, kp, vp, tables.to(cuda), torch.tensor(ctx, dtype=torch.int32, device=cuda),
                                 160, 0.125, table_rows=torch.tensor(rows, dtype=torch.int32, device=cuda))
    want = O.paged_attention(f64(q)[:, None], f64(kp), f64(vp), tables.numpy(), ctx, 0.125, table_rows=rows)[:, 0]
    assert_close(out, want, torch.float32, "indirection+gqa")


def test_paged_attention_ignores_invalid_block_ids(cuda):
    """Block ids outside [0, num_blocks) inside the context are excluded, never read."""
    gen = torch.Generator().manual_seed(8)
    h, d, bs, nb = 2, 64, 16, 8
    kp, vp = make_pool(gen, nb, bs, h, d, torch.float32, cuda)
    tables = torch.tensor([[1, -1, 3, 1 << 20]], dtype=torch.int32)
    q = torch.randn(1, h, d, generator=gen).to(cuda)
    out = native.paged_attention(q, kp, vp, tables.to(cuda), torch.tensor([64], dtype=torch.int32, device=cuda),
                                 64, 0.125)
    # only blocks 1 and 3 hold keys the kernel may use
    kk = np.concatenate([f64(kp)[1], f64(kp)[3]])[None].transpose(0, 2, 1, 3)
    vv = np.concatenate([f64(vp)[1], f64(vp)[3]])[None].transpose(0, 2, 1, 3)
    want = O.attention(f64(q)[:, None], kk, vv, [32], 0.125)[:, 0]
    assert_close(out, want, torch.float32, "invalid ids")


# ------------------------------------------------------------------ dense / cross attention
@pytest.mark.parametrize("dtype", DTYPES)
def test_cross_attention_over_slot_major_buffer(cuda, dtype):
    """g_cross_kv [S, L, 2, H, T, D]: row b attends slot slot_ids[b], layer l, first lens[b] positions."""
    gen = torch.Generator().manual_seed(9)
    s, nl, h, t, d = 6, 2, 4, 1500, 64
    g = torch.randn(s, nl, 2, h, t, d, generator=gen).to(cuda, dtype)
    slots = [5, 0, 2, 2]
    lens = [1500, 500, 1, 731]
    q = torch.randn(len(slots), h, d, generator=gen).to(cuda, dtype)
    layer = 1
    out = native.dense_attention(q, g[:, layer, 0], g[:, layer, 1], torch.tensor(lens, dtype=torch.int32, device=cuda),
                                 t, 0.125, slot_ids=torch.tensor(slots, dtype=torch.int32, device=cuda))
    want = O.dense_attention(f64(q)[:, None], f64(g[:, layer, 0]), f64(g[:, layer, 1]), lens, 0.125,
                             slot_ids=slots)[:, 0]
    assert_close(out, want, dtype, "cross")


def test_dense_causal_prompt_attention(cuda):
    gen = torch.Generator().manual_seed(10)
    bsz, qlen, h, t, d = 2, 4, 4, 4, 64
    k = torch.randn(bsz, h, t, d, generator=gen).to(cuda, torch.float32)
    v = torch.randn(bsz, h, t, d, generator=gen).to(cuda, torch.float32)
    q = torch.randn(bsz, qlen, h, d, generator=gen).to(cuda, torch.float32)
    out = native.dense_attention(q, k, v, torch.tensor([4, 4], dtype=torch.int32, device=cuda), t, 0.125,
                                 causal=True)
    want = O.attention(f64(q), f64(k), f64(v), [4, 4], 0.125, causal=True)
    assert_close(out, want, torch.float32, "causal dense")


# ------------------------------------------------------------------ HIP graph replay
def test_graph_replay_matches_eager(cuda):
    """append + paged attention + cross attention captured once, replayed with new inputs."""
    gen = torch.Generator().manual_seed(11)
    bsz, h, d, bs, nb, t = 8, 4, 64, 16, 256, 300
    kp, vp = make_pool(gen, nb, bs, h, d, torch.float16, cuda)
    tables = make_tables(gen, bsz, nb, 28).to(cuda)
    cross = torch.randn(bsz, 2, h, t, d, generator=gen).to(cuda, torch.float16)
    q = torch.zeros(bsz, h, d, dtype=torch.float16, device=cuda)
    knew = torch.zeros_like(q)
    vnew = torch.zeros_like(q)
    slots = torch.zeros(bsz, dtype=torch.int64, device=cuda)
    ctx = torch.zeros(bsz, dtype=torch.int32, device=cuda)
    elen = torch.zeros(bsz, dtype=torch.int32, device=cuda)
    out_s = torch.empty_like(q)
    out_c = torch.empty_like(q)

    def step():
        native.append(knew, vnew, kp, vp, slots)
        native.paged_attention(q, kp, vp, tables, ctx, 448, 0.125, out=out_s)
        native.dense_attention(q, cross[:, 0], cross[:, 1], elen, t, 0.125, out=out_c)

    native.reserve_attention(bsz, h, d, 448, torch.float16, cuda)
    native.reserve_attention(bsz, h, d, t, torch.float16, cuda)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()

    for it in range(4):
        g2 = torch.Generator().manual_seed(50 + it)
        pos = torch.randint(0, 447, (bsz,), generator=g2)
        q.copy_(torch.randn(bsz, h, d, generator=g2).to(cuda, torch.float16))
        knew.copy_(torch.randn(bsz, h, d, generator=g2).to(cuda, torch.float16))
        vnew.copy_(torch.randn(bsz, h, d, generator=g2).to(cuda, torch.float16))
        tb = tables.cpu()
        slots.copy_(torch.tensor([tb[b, p // bs].item() * bs + p % bs for b, p in enumerate(pos.tolist())]))
        ctx.copy_((pos + 1).to(torch.int32))
        elen.copy_(torch.randint(1, t + 1, (bsz,), generator=g2).to(torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        gs, gc = out_s.clone(), out_c.clone()
        kp_after = kp.clone()
        step()  # eager on the same inputs (append is idempotent)
        torch.cuda.synchronize()
        assert torch.equal(kp, kp_after)
        assert torch.equal(gs, out_s) and torch.equal(gc, out_c), f"replay {it} differs from eager"
        want = O.paged_attention(f64(q)[:, None], f64(kp), f64(vp), tb.numpy(), (pos + 1).tolist(), 0.125)[:, 0]
        assert_close(gs, want, torch.float16, f"graph replay {it}")


# ------------------------------------------------------------------ row order
@pytest.mark.parametrize("bsz,ties,trows", [(64, False, False), (64, True, False), (63, False, True), (65, False, False),
                                            (20, True, True), (1, False, False), (128, False, False),
                                            (100, True, True), (129, False, False)])
def test_paged_attention_rows_in_any_order(cuda, bsz, ties, trows):
    """A launch of up to 128 decode rows takes its (row, head) items in length-class order whatever order the
    rows come in (rows 0-63 from one lane each, rows 64-127 from a second load; more rows, or rows flagged
    longest-first, keep the given order): the same rows in any order, flagged or not, give row for row the
    same bits (outputs and appended pool rows), within the oracle bar. Ties: lengths from a few values."""
    gen = torch.Generator().manual_seed(700 + bsz + 2 * ties + trows)
    h, d, bs, dtype, max_ctx = 20, 64, 16, torch.bfloat16, 452
    maxblk = -(-max_ctx // bs)
    nb = bsz * maxblk + 16
    if ties:
        ctx = torch.tensor([1, 7, 200, 452])[torch.randint(0, 4, (bsz,), generator=gen)]
    else:
        ctx = torch.randint(1, max_ctx + 1, (bsz,), generator=gen)
    tables = torch.randperm(nb, generator=gen)[: bsz * maxblk].view(bsz, maxblk).to(torch.int32)
    kp, vp = make_pool(gen, nb, bs, h, d, dtype, cuda)
    q, kn, vn = (torch.randn(bsz, h, d, generator=gen).to(cuda, dtype) for _ in range(3))

    def run(order, longest_first=False):
        kpool, vpool = kp.clone(), vp.clone()
        o = torch.as_tensor(order)
        if trows:  # rows read table row perm[b] of a shuffled table
            shuffle = torch.randperm(bsz, generator=torch.Generator().manual_seed(1))
            tab = torch.empty_like(tables)
            tab[shuffle] = tables
            rows = shuffle[o].to(torch.int32).to(cuda)
            out = native.paged_attention(q[o.to(cuda)], kpool, vpool, tab.to(cuda), ctx[o].to(torch.int32).to(cuda),
                                         max_ctx, 0.125, table_rows=rows, k_new=kn[o.to(cuda)], v_new=vn[o.to(cuda)],
                                         rows_longest_first=longest_first)
        else:
            out = native.paged_attention(q[o.to(cuda)], kpool, vpool, tables[o].to(cuda),
                                         ctx[o].to(torch.int32).to(cuda), max_ctx, 0.125, k_new=kn[o.to(cuda)],
                                         v_new=vn[o.to(cuda)], rows_longest_first=longest_first)
        torch.cuda.synchronize()
        back = torch.empty_like(out)
        back[o.to(cuda)] = out
        return back, kpool, vpool

    longest_first = sorted(range(bsz), key=lambda i: (-int(ctx[i]), i))
    drawn = torch.randperm(bsz, generator=gen).tolist()
    shortest_first = longest_first[::-1]
    ref_out, ref_k, ref_v = run(longest_first)
    # with the longest-first flag (rows in that order, and, wrongly, in drawn order: only the work's
    # placement may change) and without it
    for order, flag in ((longest_first, True), (drawn, True), (list(range(bsz)), False), (drawn, False),
                        (shortest_first, False)):
        out, k2, v2 = run(order, flag)
        assert torch.equal(out, ref_out)
        assert torch.equal(k2, ref_k) and torch.equal(v2, ref_v)
    want = O.paged_attention(f64(q)[:, None], f64(ref_k), f64(ref_v), tables.numpy(), ctx.tolist(), 0.125)[:, 0]
    err = assert_close(ref_out, want, dtype, f"rows in any order, batch {bsz}")
    print(f"rows in any order, batch {bsz}, ties {ties}, table rows {trows}: bit-equal in 6 runs, max err {err:.2e}")
