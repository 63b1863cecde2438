"""EncoderAttentionBackend: non-causal attention over paged encoder K/V (reference
speech_serving/encoder_attention.py:22-71), through the paged attention kernel.

Checked against the oracle (float64, gather then dense attention) and against the reference's own
torch math restated in float32 (gather, view, permute, matmul, softmax, matmul), to the attention bar."""
import math

import numpy as np
import pytest
import torch

from oracle import paged_kv as O
from speech_serving import EncoderAttentionBackend

from test_kernels_gpu import assert_close, f64

pytestmark = pytest.mark.gpu


def torch_reference(query, table, kp, vp, seq):
    b, h, q, d = query.shape
    k = kp[table].view(-1, h, d)[:seq].permute(1, 0, 2).unsqueeze(0).expand(b, -1, -1, -1).float()
    v = vp[table].view(-1, h, d)[:seq].permute(1, 0, 2).unsqueeze(0).expand(b, -1, -1, -1).float()
    s = torch.matmul(query.float(), k.transpose(-2, -1).contiguous()) / math.sqrt(d)
    return torch.matmul(torch.softmax(s, dim=-1), v.contiguous())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("b,q,seq,table", [(2, 7, 37, [5, 2, 9]), (1, 1, 16, [3]), (3, 20, 100, [8, 1, 4, 6, 0, 7, 11]),
                                           (2, 5, 200, [1, 2])])
def test_matches_oracle_and_reference_math(cuda, dtype, b, q, seq, table):
    gen = torch.Generator().manual_seed(seq + q)
    h, d, bs, nb = 4, 64, 16, 12
    kp = torch.randn(nb, bs, h, d, generator=gen).to(cuda, dtype)
    vp = torch.randn(nb, bs, h, d, generator=gen).to(cuda, dtype)
    query = torch.randn(b, h, q, d, generator=gen).to(cuda, dtype)
    out = EncoderAttentionBackend.forward(query, table, kp, vp, seq, bs)
    assert out.shape == query.shape and out.dtype == dtype
    eff = min(seq, len(table) * bs)  # the reference's [:seq] slice of the gathered blocks
    tbl = np.array([table], dtype=np.int32)
    want = O.paged_attention(f64(query).transpose(0, 2, 1, 3), f64(kp), f64(vp), np.repeat(tbl, b, 0), [eff] * b,
                             1 / math.sqrt(d))
    assert_close(out.transpose(1, 2), want, dtype, "oracle")
    ref = torch_reference(query, torch.tensor(table, device=cuda), kp, vp, eff)
    assert_close(out, f64(ref), dtype, "reference math")


def test_empty_table_or_length_gives_zeros(cuda):
    kp = torch.randn(4, 16, 2, 64, device=cuda)
    query = torch.randn(1, 2, 3, 64, device=cuda)
    assert not EncoderAttentionBackend.forward(query, [], kp, kp, 10).any()
    assert not EncoderAttentionBackend.forward(query, [1, 2], kp, kp, 0).any()
