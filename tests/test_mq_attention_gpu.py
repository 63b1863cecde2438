"""Multi-query cross-attention (several prompt tokens per row against one read of the row's encoder
K/V, both products on the matrix cores) through skv_dense_attention, against the float64 oracle.

The reference's prompt prefill runs its cross-attention with seq_len = prompt length
(speech_serving/models.py:184-202, called from phase_aware_scheduler.py:664-670). Bar: the
attention bar of the other kernel tests, max |out - oracle| <= 2e-3 + r |oracle| (r the output
dtype's relative half-ulp). Covered: 2 to 40 queries (one to three 16-query tiles), lengths 0, 1,
one and two MFMA steps and the full 1500, slot indirection into the slot-major buffer, rows split
into key chunks (combined by the merge launch), graph replays against the eager result, and the
same kernel over paged K/V (block tables with row indirection, invalid block ids, grouped KV heads).

With 64 or more queries per row and enough (row, head, 64-query) workgroups to fill the GPU, the launch
takes the 64-query kernel instead (K/V staged in LDS once per 64 queries, each wave over all keys):
the last tests cover it at 64 to 257 queries, contiguous and paged, and at the encoder-attention
shape (1500 queries x 20 heads over 94 blocks).
"""
import numpy as np
import pytest
import torch

from oracle import paged_kv as O
from speech_serving import native

pytestmark = pytest.mark.gpu

REL = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}


def f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def check(got, want, dtype, what):
    err = np.abs(f64(got) - want)
    tol = 2e-3 + REL[dtype] * np.abs(want)
    assert (err <= tol).all(), f"{what}: max err {err.max():.3e} (dtype {dtype})"
    return float(err.max())


def cross_case(cuda, dtype, qlen, seed, lens, slots, h=4, t=1500, layers=2, layer=1):
    gen = torch.Generator().manual_seed(seed)
    s = max(slots) + 1
    g = torch.randn(s, layers, 2, h, t, 64, generator=gen).to(cuda, dtype)
    q = torch.randn(len(slots), qlen, h, 64, generator=gen).to(cuda, dtype)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=cuda)
    slots_t = torch.tensor(slots, dtype=torch.int32, device=cuda)
    return g, q, lens_t, slots_t, layer


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("qlen", [2, 4, 16, 17, 40])
def test_multi_query_cross_attention_matches_oracle(cuda, dtype, qlen):
    lens = [1500, 0, 1, 31, 33, 500, 64, 1499]
    slots = [3, 0, 5, 1, 1, 2, 4, 0]
    g, q, lens_t, slots_t, layer = cross_case(cuda, dtype, qlen, 40 + qlen, lens, slots)
    out = native.dense_attention(q, g[:, layer, 0], g[:, layer, 1], lens_t, 1500, 0.125, slot_ids=slots_t)
    want = O.dense_attention(f64(q), f64(g[:, layer, 0]), f64(g[:, layer, 1]), lens, 0.125, slot_ids=slots)
    err = check(out, want, dtype, f"q_len {qlen}")
    assert np.all(f64(out)[1] == 0.0)  # an empty row gives zeros
    print(f"q_len {qlen} {dtype}: max err {err:.2e}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_split_rows_merge(cuda, dtype):
    # One row x 2 heads: too few (row, head) pairs to fill the GPU, so the keys split into chunks
    # whose per-query partials the merge launch combines.
    g, q, lens_t, slots_t, layer = cross_case(cuda, dtype, 4, 7, [1437], [0], h=2)
    rows = q.shape[0] * q.shape[1]
    assert native.attention_workspace_bytes(rows, 2, 64, 1500, dtype) > 0
    out = native.dense_attention(q, g[:, layer, 0], g[:, layer, 1], lens_t, 1500, 0.125, slot_ids=slots_t)
    want = O.dense_attention(f64(q), f64(g[:, layer, 0]), f64(g[:, layer, 1]), [1437], 0.125, slot_ids=[0])
    check(out, want, dtype, "split rows")


def test_graph_replays_equal_eager(cuda):
    dtype = torch.bfloat16
    lens = [1500, 700, 3]
    slots = [2, 0, 1]
    g, q, lens_t, slots_t, layer = cross_case(cuda, dtype, 4, 11, lens, slots)
    out = torch.empty_like(q)
    native.reserve_attention(q.shape[0] * q.shape[1], 4, 64, 1500, dtype, cuda)

    def call():
        native.dense_attention(q, g[:, layer, 0], g[:, layer, 1], lens_t, 1500, 0.125, slot_ids=slots_t, out=out)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    gen = torch.Generator().manual_seed(12)
    for _ in range(4):
        q.copy_(torch.randn(q.shape, generator=gen).to(cuda, dtype))
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        call()
        torch.cuda.synchronize()
        assert torch.equal(replayed, out)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("qlen,kv_heads", [(3, 4), (16, 4), (33, 2), (200, 4)])  # 200: too few 64-query tiles
def test_multi_query_over_paged_blocks(cuda, dtype, qlen, kv_heads):
    """Non-causal multi-query attention through block tables (the encoder attention path, the
    reference's EncoderAttentionBackend, encoder_attention.py:22-71): row indirection, invalid
    block ids excluded, grouped KV heads, lengths up to the table's capacity."""
    gen = torch.Generator().manual_seed(60 + qlen)
    h, bs, nb, maxblk = 4, 16, 300, 94
    kp = torch.randn(nb, bs, kv_heads, 64, generator=gen).to(cuda, dtype)
    vp = torch.randn(nb, bs, kv_heads, 64, generator=gen).to(cuda, dtype)
    tables = torch.randperm(nb, generator=gen)[: 3 * maxblk].view(3, maxblk).to(torch.int32)
    tables[1, 5] = -1          # an invalid id: its keys drop out of the softmax
    tables[2, 7] = nb + 3
    rows = [2, 0, 1, 0]
    lens = [1504, 1, 700, 33]
    q = torch.randn(len(rows), qlen, h, 64, generator=gen).to(cuda, dtype)
    out = native.paged_attention(q, kp, vp, tables.to(cuda), torch.tensor(lens, dtype=torch.int32, device=cuda),
                                 maxblk * bs, 0.125, table_rows=torch.tensor(rows, dtype=torch.int32, device=cuda))
    # Expected: attention over the keys of valid blocks only (an invalid block's keys are left out).
    kp64, vp64, tb = f64(kp), f64(vp), tables.numpy()
    want = np.zeros(q.shape)
    for i, (r, n) in enumerate(zip(rows, lens)):
        blocks = [int(tb[r, j // bs]) for j in range(n)]
        keep = [j for j in range(n) if 0 <= blocks[j] < nb]
        kk = np.stack([kp64[blocks[j], j % bs] for j in keep]).transpose(1, 0, 2)[None]
        vv = np.stack([vp64[blocks[j], j % bs] for j in keep]).transpose(1, 0, 2)[None]
        want[i] = O.attention(f64(q)[i:i + 1], kk, vv, [len(keep)], 0.125)[0]
    check(out, want, dtype, f"paged q_len {qlen} kv_heads {kv_heads}")


def mqt_selected(rows, heads, qlen):
    # The library picks the 64-query kernel when rows * heads * ceil(qlen / 64) reaches three
    # quarters of the CU count.
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    return qlen >= 64 and 4 * rows * heads * ((qlen + 63) // 64) >= 3 * cus


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("qlen,rows", [(64, 16), (100, 8), (257, 4)])
def test_many_queries_contiguous(cuda, dtype, qlen, rows):
    """64-query tiles over contiguous K/V: lengths 0, 1, partial steps, the full 1500; slot indirection."""
    h = 20
    assert mqt_selected(rows, h, qlen)
    lens = ([1500, 0, 1, 33, 700, 1499, 64, 95] * 2)[:rows]
    slots = ([3, 0, 5, 1, 1, 2, 4, 0] * 2)[:rows]
    g, q, lens_t, slots_t, layer = cross_case(cuda, dtype, qlen, 90 + qlen, lens, slots, h=h)
    out = native.dense_attention(q, g[:, layer, 0], g[:, layer, 1], lens_t, 1500, 0.125, slot_ids=slots_t)
    want = O.dense_attention(f64(q), f64(g[:, layer, 0]), f64(g[:, layer, 1]), lens, 0.125, slot_ids=slots)
    err = check(out, want, dtype, f"64-query tiles, q_len {qlen}")
    assert np.all(f64(out)[1] == 0.0)
    print(f"q_len {qlen} {dtype}: max err {err:.2e}")


@pytest.mark.parametrize("scale", [-0.125, 0.0])
def test_many_queries_non_positive_scale(cuda, scale):
    """A scale of 0 or below at a 64-query-tile shape: the scores' maximum then is not the scaled maximum
    of the raw scores, and the result still matches the oracle."""
    dtype, h, qlen, rows = torch.bfloat16, 20, 64, 16
    assert mqt_selected(rows, h, qlen)
    lens = ([1500, 0, 1, 33, 700, 1499, 64, 95] * 2)[:rows]
    slots = ([3, 0, 5, 1, 1, 2, 4, 0] * 2)[:rows]
    g, q, lens_t, slots_t, layer = cross_case(cuda, dtype, qlen, 123, lens, slots, h=h)
    out = native.dense_attention(q, g[:, layer, 0], g[:, layer, 1], lens_t, 1500, scale, slot_ids=slots_t)
    want = O.dense_attention(f64(q), f64(g[:, layer, 0]), f64(g[:, layer, 1]), lens, scale, slot_ids=slots)
    check(out, want, dtype, f"64-query tiles, scale {scale}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("qlen,rows", [(16, 4), (64, 16)])  # the 16-query kernel, the 64-query kernel
def test_rising_scores_rescale_mid_row(cuda, dtype, qlen, rows):
    """Scores that keep rising along the keys (a ramp up to ~58 in log2 units, steeper for later
    queries) and a spike at key 1400: both kernels move their reference maximum only when a step's
    maximum exceeds it by more than 8 (log2 units), so these rows rescale their accumulators several
    times mid-row and once near the end, with weights up to 2^8 in between."""
    h = 20 if qlen == 64 else 4
    assert mqt_selected(rows, h, qlen) == (qlen == 64)
    lens = ([1500, 1401, 1399, 800] * 4)[:rows]
    slots = list(range(rows))
    g, q, lens_t, slots_t, layer = cross_case(cuda, torch.float32, qlen, 140 + qlen, lens, slots, h=h)
    g[:, layer, 0, :, :, 0] = torch.linspace(0.0, 40.0, 1500, device=cuda)
    g[:, layer, 0, :, 1400, 0] = 60.0
    q[..., 0] = torch.linspace(0.5, 8.0, qlen, device=cuda)[None, :, None]
    g, q = g.to(dtype), q.to(dtype)
    out = native.dense_attention(q, g[:, layer, 0], g[:, layer, 1], lens_t, 1500, 0.125, slot_ids=slots_t)
    want = O.dense_attention(f64(q), f64(g[:, layer, 0]), f64(g[:, layer, 1]), lens, 0.125, slot_ids=slots)
    err = check(out, want, dtype, f"rising scores, q_len {qlen}")
    print(f"rising scores q_len {qlen} {dtype}: max err {err:.2e}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("kv_heads", [20, 4])
def test_encoder_attention_shape_paged(cuda, dtype, kv_heads):
    """The encoder-attention shape on the 64-query kernel: 1500 queries x 20 heads over one table of 94
    blocks (row indirection to a shared table row), a second row with an invalid block id and a shorter
    length, grouped KV heads."""
    h, bs, nb, maxblk, qlen = 20, 16, 200, 94, 1500
    gen = torch.Generator().manual_seed(70 + kv_heads)
    kp = torch.randn(nb, bs, kv_heads, 64, generator=gen).to(cuda, dtype)
    vp = torch.randn(nb, bs, kv_heads, 64, generator=gen).to(cuda, dtype)
    tables = torch.randperm(nb, generator=gen)[: 2 * maxblk].view(2, maxblk).to(torch.int32)
    tables[1, 9] = -1          # keys 144..159: in the first half of the row's 32 steps
    tables[1, 50] = nb + 7     # keys 800..815: in the second half
    rows, lens = [0, 1], [1500, 1001]
    assert mqt_selected(len(rows), h, qlen)
    q = torch.randn(len(rows), qlen, h, 64, generator=gen).to(cuda, dtype)
    out = native.paged_attention(q, kp, vp, tables.to(cuda), torch.tensor(lens, dtype=torch.int32, device=cuda),
                                 maxblk * bs, 0.125, table_rows=torch.tensor(rows, dtype=torch.int32, device=cuda))
    kp64, vp64, tb = f64(kp), f64(vp), tables.numpy()
    want = np.zeros(q.shape)
    for i, (r, n) in enumerate(zip(rows, lens)):
        blocks = [int(tb[r, j // bs]) for j in range(n)]
        keep = [j for j in range(n) if 0 <= blocks[j] < nb]
        kk = np.stack([kp64[blocks[j], j % bs] for j in keep]).transpose(1, 0, 2)[None]
        vv = np.stack([vp64[blocks[j], j % bs] for j in keep]).transpose(1, 0, 2)[None]
        want[i] = O.attention(f64(q)[i:i + 1], kk, vv, [len(keep)], 0.125)[0]
    err = check(out, want, dtype, f"encoder shape kv_heads {kv_heads}")
    print(f"encoder shape {dtype} kv_heads {kv_heads}: max err {err:.2e}")
