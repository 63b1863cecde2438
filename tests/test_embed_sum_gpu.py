"""skv_codebook_embed_sum against the reference's embedding loop (speech_serving/models.py:39-52):
embeds = emb_0(codes[..., 0]); embeds = embeds + emb_k(codes[..., k]) for k = 1..K-1, in the tables' dtype.
The bar is bit-exact: the kernel rounds every partial sum to the dtype, as torch's elementwise add does."""
import pytest
import torch

from speech_serving import native

pytestmark = pytest.mark.gpu


def reference_loop(codes, tables):
    x = torch.nn.functional.embedding(codes[..., 0], tables[0])
    for k in range(1, len(tables)):
        x = x + torch.nn.functional.embedding(codes[..., k], tables[k])
    return x


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("books,vocab,dim,shape", [(1, 50, 64, (3, 5)), (4, 1024, 256, (64, 1)),
                                                   (4, 1024, 256, (2, 33)), (7, 300, 40, (9, 4)),
                                                   (16, 17, 8, (5, 2))])
def test_matches_reference_loop_bitwise(cuda, dtype, books, vocab, dim, shape):
    g = torch.Generator(device=cuda).manual_seed(books * 1000 + dim)
    tables = [(torch.randn(vocab, dim, generator=g, device=cuda) * 3).to(dtype) for _ in range(books)]
    codes = torch.randint(0, vocab, shape + (books,), generator=g, device=cuda)
    got = native.codebook_embed_sum(codes, tables)
    want = reference_loop(codes, tables)
    assert got.shape == want.shape and got.dtype == dtype
    assert torch.equal(got.view(torch.int8 if dtype != torch.float32 else torch.int32),
                       want.view(torch.int8 if dtype != torch.float32 else torch.int32))


def test_rounding_order_is_left_to_right(cuda):
    """(a + b) + c differs from a + (b + c) in bf16 for these rows; the kernel must give the former."""
    t = [torch.tensor([[1.0] * 8], dtype=torch.bfloat16, device=cuda),
         torch.tensor([[2.0 ** -8] * 8], dtype=torch.bfloat16, device=cuda),
         torch.tensor([[2.0 ** -8] * 8], dtype=torch.bfloat16, device=cuda)]
    codes = torch.zeros(1, 1, 3, dtype=torch.int64, device=cuda)
    got = native.codebook_embed_sum(codes, t)
    assert torch.equal(got, reference_loop(codes, t))
    assert got[0, 0, 0].item() == 1.0  # 1 + 2^-8 rounds to 1 (ties to even), twice; a + (b + c) would give 1 + 2^-7


def test_out_of_range_codes_add_zero_rows(cuda):
    tables = [torch.randn(10, 16, device=cuda) for _ in range(3)]
    codes = torch.tensor([[[3, -1, 10], [2, 4, 9]]], device=cuda)
    got = native.codebook_embed_sum(codes, tables)
    assert torch.equal(got[0, 0], tables[0][3])
    assert torch.equal(got[0, 1], reference_loop(codes[:, 1:], tables)[0, 0])


def test_strided_codes_and_empty_batch(cuda):
    tables = [torch.randn(20, 32, device=cuda, dtype=torch.float16) for _ in range(2)]
    wide = torch.randint(0, 20, (6, 5), device=cuda)
    codes = wide[:, 1:3]  # row stride 5
    assert torch.equal(native.codebook_embed_sum(codes, tables), reference_loop(codes.contiguous(), tables))
    assert native.codebook_embed_sum(torch.zeros(0, 2, dtype=torch.int64, device=cuda), tables).shape == (0, 32)


def test_bad_arguments_raise(cuda):
    tables = [torch.randn(20, 32, device=cuda) for _ in range(2)]
    with pytest.raises(RuntimeError):
        native.codebook_embed_sum(torch.zeros(3, 3, dtype=torch.int64, device=cuda), tables)  # 3 codes, 2 tables
    with pytest.raises(RuntimeError):
        native.codebook_embed_sum(torch.zeros(3, 2, dtype=torch.int64, device=cuda),
                                  [tables[0], torch.randn(20, 30, device=cuda)])
