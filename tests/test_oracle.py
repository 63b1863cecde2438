"""Pins for the CPU oracle (oracle/paged_kv.py), CPU only.

Each oracle function is checked against something that does not retype its
own formula: closed forms, invariants, brute force with Python scalars, an
independent library formulation (torch advanced indexing / torch.softmax),
and the reference's padded-and-masked formulation. The last tests plant
mistakes in copies of the oracle and show that the pins catch them.
"""
import math

import numpy as np
import pytest
import torch

from oracle import paged_kv as O


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- slot mapping
def test_slot_mapping_closed_form():
    # table [7, 2, 9], BS 4: position 0 -> 7*4+0, 5 -> 2*4+1, 11 -> 9*4+3
    assert O.slot_mapping([7, 2, 9], [0, 5, 11], 4).tolist() == [28, 9, 39]


# ---------------------------------------------------------------- append
def test_append_writes_rows_and_leaves_other_slots_untouched():
    r = rng(0)
    pool_k = r.standard_normal((6, 4, 2, 8)).astype(np.float32)
    pool_v = r.standard_normal((6, 4, 2, 8)).astype(np.float32)
    before_k, before_v = pool_k.copy(), pool_v.copy()
    new_k = r.standard_normal((3, 2, 8)).astype(np.float32)
    new_v = r.standard_normal((3, 2, 8)).astype(np.float32)
    slots = [5, -1, 23]
    O.append(pool_k, pool_v, new_k, new_v, slots)
    assert np.array_equal(pool_k[1, 1], new_k[0]) and np.array_equal(pool_v[5, 3], new_v[2])
    mask = np.ones((6, 4), bool)
    mask[1, 1] = mask[5, 3] = False
    assert np.array_equal(pool_k[mask], before_k[mask]) and np.array_equal(pool_v[mask], before_v[mask])


def test_append_skips_out_of_range_slots():
    pool = np.zeros((2, 4, 1, 8), np.float32)
    O.append(pool, None, np.ones((2, 1, 8), np.float32), None, [8, 100])
    assert not pool.any()


# ---------------------------------------------------------------- gather
def test_gather_matches_torch_indexing_of_the_reference_form():
    """pool[table].view(-1, H, D)[:T].permute(1, 0, 2) via torch indexing (tts_engine.py:177-185)."""
    r = rng(1)
    nb, bs, h, d = 16, 4, 3, 8
    pool = r.standard_normal((nb, bs, h, d)).astype(np.float32)
    tables = np.stack([r.permutation(nb)[:5] for _ in range(3)]).astype(np.int32)
    lens = [17, 1, 20]
    got = O.gather(pool, tables, lens, 20)
    tp = torch.from_numpy(pool)
    for b, n in enumerate(lens):
        nblk = -(-n // bs)
        ref = tp[torch.from_numpy(tables[b, :nblk]).long()].view(-1, h, d)[:n].permute(1, 0, 2).numpy()
        assert np.array_equal(got[b, :, :n], ref)
        assert not got[b, :, n:].any()


def test_gather_brute_force_elementwise():
    r = rng(2)
    nb, bs, h, d = 8, 2, 2, 4
    pool = r.standard_normal((nb, bs, h, d))
    tables = np.array([[3, 0, 7, 5], [1, 2, 6, 4]], np.int32)
    lens = [7, 3]
    got = O.gather(pool, tables, lens, 8)
    for b in range(2):
        for hh in range(h):
            for t in range(8):
                for dd in range(d):
                    want = pool[tables[b, t // bs], t % bs, hh, dd] if t < lens[b] else 0.0
                    assert got[b, hh, t, dd] == want


def test_append_then_gather_round_trip():
    r = rng(3)
    nb, bs, h, d, n = 32, 16, 4, 8, 45
    pool_k = np.zeros((nb, bs, h, d), np.float16)
    pool_v = np.zeros((nb, bs, h, d), np.float16)
    table = r.permutation(nb)[: -(-n // bs)]
    src_k = r.standard_normal((n, h, d)).astype(np.float16)
    src_v = r.standard_normal((n, h, d)).astype(np.float16)
    O.append(pool_k, pool_v, src_k, src_v, O.slot_mapping(table, range(n), bs))
    got = O.gather(pool_k, table[None].astype(np.int32), [n], n)
    assert np.array_equal(got[0], src_k.transpose(1, 0, 2))
    got_v = O.gather(pool_v, table[None].astype(np.int32), [n], n)
    assert np.array_equal(got_v[0], src_v.transpose(1, 0, 2))


# ---------------------------------------------------------------- attention
def test_single_key_returns_that_value_exactly():
    r = rng(4)
    q = r.standard_normal((1, 1, 2, 8))
    k = r.standard_normal((1, 2, 5, 8))
    v = r.standard_normal((1, 2, 5, 8))
    out = O.attention(q, k, v, [1], 0.3)
    assert np.array_equal(out[0, 0], v[0, :, 0])


def test_identical_keys_give_mean_of_values():
    r = rng(5)
    k = np.repeat(r.standard_normal((1, 1, 1, 8)), 6, axis=2)
    v = r.standard_normal((1, 1, 6, 8))
    out = O.attention(r.standard_normal((1, 1, 1, 8)), k, v, [6], 0.125)
    np.testing.assert_allclose(out[0, 0, 0], v[0, 0].mean(axis=0), rtol=1e-12, atol=1e-12)


def test_zero_length_gives_zeros():
    out = O.attention(np.ones((1, 1, 1, 4)), np.ones((1, 1, 3, 4)), np.ones((1, 1, 3, 4)), [0], 1.0)
    assert not out.any()


def test_masked_tail_has_no_influence():
    r = rng(6)
    q = r.standard_normal((2, 1, 3, 8))
    k = r.standard_normal((2, 3, 10, 8))
    v = r.standard_normal((2, 3, 10, 8))
    lens = [4, 7]
    a = O.attention(q, k, v, lens, 0.25)
    k2, v2 = k.copy(), v.copy()
    k2[0, :, 4:] = 1e6
    v2[1, :, 7:] = np.nan
    b = O.attention(q, k2, v2, lens, 0.25)
    assert np.array_equal(a, b)


def test_brute_force_python_scalars():
    r = rng(7)
    q = r.standard_normal((1, 1, 1, 3))
    k = r.standard_normal((1, 1, 4, 3))
    v = r.standard_normal((1, 1, 4, 3))
    scale = 0.7
    s = [sum(q[0, 0, 0, i] * k[0, 0, t, i] for i in range(3)) * scale for t in range(4)]
    mx = max(s)
    w = [math.exp(x - mx) for x in s]
    z = sum(w)
    want = [sum(w[t] / z * v[0, 0, t, i] for t in range(4)) for i in range(3)]
    got = O.attention(q, k, v, [4], scale)[0, 0, 0]
    np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-13)


def test_matches_torch_softmax_library_routine():
    r = rng(8)
    q = r.standard_normal((3, 1, 4, 16))
    k = r.standard_normal((3, 4, 9, 16))
    v = r.standard_normal((3, 4, 9, 16))
    lens = [9, 5, 2]
    got = O.attention(q, k, v, lens, 0.25)
    for b, n in enumerate(lens):
        tq = torch.from_numpy(q[b, 0])  # [H, D]
        tk = torch.from_numpy(k[b, :, :n])
        tv = torch.from_numpy(v[b, :, :n])
        p = torch.softmax(torch.einsum("hd,htd->ht", tq, tk) * 0.25, dim=-1)
        want = torch.einsum("ht,htd->hd", p, tv).numpy()
        np.testing.assert_allclose(got[b, 0], want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("form", ["finfo_min_fill", "additive_minus_10000"])
def test_padded_masked_reference_form_equals_length_form(form):
    """The reference attends over [prefix | masked pad | new] (eager) or a whole
    masked bucket (graph); masked weights underflow to exactly 0, so it equals
    attention over the valid keys."""
    r = rng(9)
    bsz, h, t, d = 3, 2, 12, 8
    q = r.standard_normal((bsz, 1, h, d)).astype(np.float32)
    k = r.standard_normal((bsz, h, t, d)).astype(np.float32)
    v = r.standard_normal((bsz, h, t, d)).astype(np.float32)
    lens = [12, 5, 1]
    keep = np.zeros((bsz, 1, t), bool)
    for b, n in enumerate(lens):
        keep[b, 0, :n] = True
    if form == "finfo_min_fill":
        masked = O.attention_masked(q, k, v, keep, 1 / math.sqrt(d), fill=float(np.finfo(np.float32).min))
    else:
        add = np.where(keep, 0.0, -10000.0)
        masked = O.attention_masked(q, k, v, keep, 1 / math.sqrt(d), additive=add)
    want = O.attention(q, k, v, lens, 1 / math.sqrt(d))
    np.testing.assert_allclose(masked, want, rtol=1e-12, atol=1e-12)


def test_causal_equals_prefix_attention_per_query():
    r = rng(10)
    q = r.standard_normal((1, 4, 2, 8))
    k = r.standard_normal((1, 2, 10, 8))
    v = r.standard_normal((1, 2, 10, 8))
    got = O.attention(q, k, v, [10], 0.3, causal=True)
    for qi in range(4):
        want = O.attention(q[:, qi:qi + 1], k, v, [10 - 3 + qi], 0.3)
        np.testing.assert_array_equal(got[:, qi], want[:, 0])


def test_causal_triu_form_of_the_reference():
    """models.py:159-161: a triu(-inf, diagonal=1) mask over [past | prompt] keys."""
    r = rng(11)
    past, qlen, h, d = 3, 4, 2, 8
    q = r.standard_normal((1, qlen, h, d))
    k = r.standard_normal((1, h, past + qlen, d))
    v = r.standard_normal((1, h, past + qlen, d))
    s = np.einsum("bqhd,bhtd->bhqt", q, k) * 0.5
    tri = np.triu(np.full((qlen, past + qlen), -np.inf), k=1 + past)
    s = s + tri
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    want = np.einsum("bhqt,bhtd->bqhd", p, v)
    got = O.attention(q, k, v, [past + qlen], 0.5, causal=True)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_grouped_kv_heads_repeat():
    r = rng(12)
    q = r.standard_normal((1, 1, 4, 8))
    k = r.standard_normal((1, 2, 6, 8))
    v = r.standard_normal((1, 2, 6, 8))
    got = O.attention(q, k, v, [6], 0.3)
    full = O.attention(q, np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1), [6], 0.3)
    np.testing.assert_array_equal(got, full)


def test_paged_attention_equals_contiguous_attention():
    r = rng(13)
    nb, bs, h, d = 40, 16, 2, 8
    pool_k = r.standard_normal((nb, bs, h, d))
    pool_v = r.standard_normal((nb, bs, h, d))
    tables = np.stack([r.permutation(nb)[:6] for _ in range(3)]).astype(np.int32)
    lens = [1, 50, 96]
    q = r.standard_normal((3, 1, h, d))
    got = O.paged_attention(q, pool_k, pool_v, tables, lens, 0.2)
    for b, n in enumerate(lens):
        k = np.concatenate([pool_k[tables[b, i]] for i in range(6)])[:n].transpose(1, 0, 2)[None]
        v = np.concatenate([pool_v[tables[b, i]] for i in range(6)])[:n].transpose(1, 0, 2)[None]
        np.testing.assert_allclose(got[b:b + 1], O.attention(q[b:b + 1], k, v, [n], 0.2), rtol=0, atol=0)


# ---------------------------------------------------------------- planted mistakes
# Each pin below is a predicate over an attention implementation; the correct
# oracle passes all of them and every planted mistake fails at least one.
def _pin_brute_force(attn):
    r = rng(20)
    q, k, v = r.standard_normal((1, 1, 1, 3)), r.standard_normal((1, 1, 4, 3)), r.standard_normal((1, 1, 4, 3))
    s = [sum(q[0, 0, 0, i] * k[0, 0, t, i] for i in range(3)) * 0.7 for t in range(4)]
    w = [math.exp(x - max(s)) for x in s]
    want = [sum(w[t] / sum(w) * v[0, 0, t, i] for t in range(4)) for i in range(3)]
    return np.allclose(attn(q, k, v, [4], 0.7)[0, 0, 0], want, rtol=1e-12, atol=1e-12)


def _pin_torch(attn):
    r = rng(21)
    q, k, v = r.standard_normal((2, 1, 2, 8)), r.standard_normal((2, 2, 6, 8)), r.standard_normal((2, 2, 6, 8))
    got = attn(q, k, v, [6, 3], 0.25)
    for b, n in enumerate([6, 3]):
        p = torch.softmax(torch.einsum("hd,htd->ht", torch.from_numpy(q[b, 0]), torch.from_numpy(k[b, :, :n])) * 0.25, -1)
        if not np.allclose(got[b, 0], torch.einsum("ht,htd->hd", p, torch.from_numpy(v[b, :, :n])).numpy(), atol=1e-12):
            return False
    return True


def _pin_masked_tail(attn):
    r = rng(22)
    q, k, v = r.standard_normal((1, 1, 2, 8)), r.standard_normal((1, 2, 8, 8)), r.standard_normal((1, 2, 8, 8))
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 5:] += 3.0
    v2[:, :, 5:] -= 3.0
    return np.array_equal(attn(q, k, v, [5], 0.3), attn(q, k2, v2, [5], 0.3))


def _pin_single_key(attn):
    r = rng(23)
    q, k, v = r.standard_normal((1, 1, 2, 8)), r.standard_normal((1, 2, 4, 8)), r.standard_normal((1, 2, 4, 8))
    return np.array_equal(attn(q, k, v, [1], 0.3)[0, 0], v[0, :, 0])


PINS = [_pin_brute_force, _pin_torch, _pin_masked_tail, _pin_single_key]


def _mutant(kind):
    def f(q, k, v, lens, scale, causal=False):
        if kind == "no_scale":
            return O.attention(q, k, v, lens, 1.0, causal)
        if kind == "off_by_one_len":
            return O.attention(q, k, v, [n + 1 for n in lens], scale, causal)
        if kind == "k_v_swapped":
            return O.attention(q, v, k, lens, scale, causal)
        if kind == "no_max_subtraction_and_wrong_sign":
            return O.attention(-q, k, v, lens, scale, causal)
        raise ValueError(kind)
    return f


def test_oracle_passes_every_pin():
    assert all(pin(O.attention) for pin in PINS)


@pytest.mark.parametrize("kind", ["no_scale", "off_by_one_len", "k_v_swapped", "no_max_subtraction_and_wrong_sign"])
def test_pins_catch_planted_attention_mistakes(kind):
    assert not all(pin(_mutant(kind)) for pin in PINS)


def test_pins_catch_planted_gather_index_swap():
    """A gather that reverses the block table fails the torch-indexing pin."""
    r = rng(15)
    pool = r.standard_normal((8, 4, 2, 4))
    tables = np.array([[3, 1, 6]], np.int32)
    bad = O.gather(pool, tables[:, ::-1].copy(), [10], 10)
    ref = torch.from_numpy(pool)[torch.tensor([3, 1, 6])].view(-1, 2, 4)[:10].permute(1, 0, 2).numpy()
    assert not np.array_equal(bad[0], ref)
