"""skv_argmax: greedy sampling with first-max tie-breaking and slot feedback.

Integer results: must equal numpy's argmax (first occurrence) bit for bit.
"""
import numpy as np
import pytest
import torch

from speech_serving import native

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
# 16-byte vectors per thread: 1, 100: one; 12345: two (16-bit logits) or four (fp32); 30000: four
# (16-bit) or two passes of seven (fp32); 51865, 51866: one pass of seven (16-bit) or two (fp32);
# 100003: two passes of seven (16-bit) or four (fp32).
@pytest.mark.parametrize("vocab", [1, 100, 12345, 30000, 51865, 51866, 100003])
def test_argmax_matches_numpy_first_max(cuda, dtype, vocab):
    gen = torch.Generator().manual_seed(vocab)
    rows = 7
    x = torch.randn(rows, vocab, generator=gen).to(dtype)
    if vocab > 10:
        x[1, 5] = x[1, vocab - 3] = 1e4  # tie: the first index wins
        x[2, :] = -float("inf")           # all -inf: index 0
        x[3, vocab // 2] = float("nan")    # NaN counts as the maximum
        x[4, 7] = float("nan")
        x[4, 3] = float("nan")             # first NaN wins
    got = native.argmax(x.to(cuda)).cpu().numpy()
    xf = x.float().numpy()
    want = []
    for r in range(rows):
        nan = np.flatnonzero(np.isnan(xf[r]))
        want.append(int(nan[0]) if nan.size else int(np.argmax(xf[r])))
    assert got.tolist() == want
    if vocab > 10:
        assert got[1] == 5 and got[2] == 0 and got[3] == vocab // 2 and got[4] == 3


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_argmax_row_edges(cuda, dtype):
    """Rows that start 2 bytes into a word (a lone first element), an odd element count (a lone last
    element), NaNs in those lone elements and in two threads' ranges, and rows whose maximum is -inf."""
    gen = torch.Generator().manual_seed(11)
    vocab = 40001
    full = torch.randn(8, vocab + 1, generator=gen).to(dtype)
    x = full[:, 1:]                       # 16-bit rows start 2 bytes into a word
    x[0, :] = -float("inf")               # maximum -inf: index 0
    x[1, 0] = float("nan")                # NaN in the lone first element
    x[2, vocab - 1] = float("nan")        # NaN in the lone last element
    x[3, 30000] = float("nan")            # NaNs in two threads' ranges: the first wins
    x[3, 9000] = float("nan")
    x[4, :] = -float("inf")
    x[4, vocab - 1] = 0.0                 # the maximum in the lone last element
    x[5, :] = 2.0                         # all equal: index 0
    got = native.argmax(x.to(cuda)).cpu().tolist()
    xf = x.float().numpy()
    want = []
    for r in range(x.shape[0]):
        nan = np.flatnonzero(np.isnan(xf[r]))
        want.append(int(nan[0]) if nan.size else int(np.argmax(xf[r])))
    assert got == want
    assert got[:6] == [0, 0, vocab - 1, 9000, vocab - 1, 0]


def test_argmax_strided_rows_and_slot_feedback(cuda):
    gen = torch.Generator().manual_seed(0)
    full = torch.randn(5, 1, 300, generator=gen).to(cuda, torch.bfloat16)
    logits = full[:, -1, :256]  # row stride 300, vocab 256
    slots = torch.tensor([3, -1, 0, 7, 2], dtype=torch.int32, device=cuda)
    slot_tokens = torch.full((9,), -5, dtype=torch.int64, device=cuda)
    out = native.argmax(logits, row_slots=slots, slot_tokens=slot_tokens)
    want = logits.float().cpu().numpy().argmax(axis=1)
    assert out.cpu().tolist() == want.tolist()
    st = slot_tokens.cpu().tolist()
    assert st[3] == want[0] and st[0] == want[2] and st[7] == want[3] and st[2] == want[4]
    assert st[1] == st[4] == st[5] == st[6] == st[8] == -5


def test_argmax_eos_flags_and_count(cuda):
    """A token equal to its slot's EOS id sets the slot's finished flag once and counts it; rows whose slot has no
    EOS id (< 0) or lies outside [0, num_slots) change nothing."""
    vocab, n_slots = 64, 8
    logits = torch.full((6, vocab), -1.0, dtype=torch.float16, device=cuda)
    winners = [5, 9, 5, 33, 7, 12]
    for r, w in enumerate(winners):
        logits[r, w] = 1.0
    slots = torch.tensor([0, 1, 2, 3, 7, 9], dtype=torch.int32, device=cuda)  # slot 9 is out of range
    eos = torch.tensor([5, 9, -1, 4, 7, 5, 5, 7], dtype=torch.int64, device=cuda)
    finished = torch.tensor([0, 1, 0, 0, 0, 0, 0, 0], dtype=torch.int32, device=cuda)  # slot 1 already finished
    count = torch.tensor([10], dtype=torch.int64, device=cuda)
    tokens = torch.zeros(n_slots, dtype=torch.int64, device=cuda)
    out = native.argmax(logits, row_slots=slots, slot_tokens=tokens, slot_eos=eos, slot_finished=finished,
                        finished_count=count)
    torch.cuda.synchronize()
    assert out.cpu().tolist() == winners
    # (slot, token): (0, 5) finishes; (1, 9) was already finished; (2, 5) has no EOS; (3, 33) is not 4;
    # (7, 7) finishes; (9, 12) is outside the slots.
    assert finished.cpu().tolist() == [1, 1, 0, 0, 0, 0, 0, 1]
    assert count.item() == 12
    assert tokens.cpu().tolist() == [5, 9, 5, 33, 0, 0, 0, 7]
    # Same step again: finished slots are not counted twice.
    native.argmax(logits, row_slots=slots, slot_tokens=tokens, slot_eos=eos, slot_finished=finished,
                  finished_count=count)
    torch.cuda.synchronize()
    assert count.item() == 12


def test_argmax_in_graph_replays(cuda):
    x = torch.zeros(4, 51866, dtype=torch.float16, device=cuda)
    out = torch.zeros(4, dtype=torch.int64, device=cuda)
    native.argmax(x, out=out)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        native.argmax(x, out=out)
    for it in range(3):
        gen = torch.Generator().manual_seed(it)
        x.copy_(torch.randn(4, 51866, generator=gen).to(cuda, torch.float16))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert out.cpu().tolist() == x.float().cpu().numpy().argmax(axis=1).tolist()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("vocab", [2, 3, 4097, 12345, 30001, 51865])
def test_argmax_rows_starting_mid_word(cuda, dtype, vocab):
    # A view one element into each row: every row starts 2 bytes past a 4-byte
    # boundary, so the first element is read alone; odd lengths leave a last one.
    gen = torch.Generator().manual_seed(vocab + 1)
    full = torch.randn(6, vocab + 1, generator=gen).to(dtype)
    full[0, 1] = 100.0          # the maximum is the first element of the view
    full[1, vocab] = 100.0      # ... or its last element
    full[2, 1 + vocab // 2] = 100.0
    x = full.to(cuda)[:, 1:]
    assert x.data_ptr() % 4 == 2
    got = native.argmax(x).cpu().numpy()
    want = x.float().cpu().numpy().argmax(axis=1)
    assert got.tolist() == want.tolist()
    assert got[0] == 0 and got[1] == vocab - 1
