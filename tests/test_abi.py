"""The C-ABI library loads, exports every symbol the header declares, and
rejects bad arguments before launching anything (no GPU needed)."""
import ctypes
import os
import re

import pytest

from speech_serving import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "speech_kv.h")


def declared_symbols():
    text = open(HEADER).read()
    return set(re.findall(r"SKV_API\s+[\w\s\*]+?\b(skv_\w+)\s*\(", text))


def test_header_declares_the_bound_entry_points():
    decl = declared_symbols()
    assert decl == set(native.SIGNATURES), (decl, set(native.SIGNATURES))
    assert {"skv_append", "skv_gather", "skv_paged_attention", "skv_dense_attention"} <= decl


def test_library_loads_and_exports_every_declared_symbol():
    lib = native.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert "gfx950" in native.version()


def test_no_undeclared_exports():
    # The .so exports exactly the header's entry points (hidden visibility elsewhere).
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", native.library_path()], capture_output=True, text=True)
    assert out.returncode == 0, out.stderr
    exported = {ln.split()[-1] for ln in out.stdout.splitlines() if " T " in ln}
    assert exported == declared_symbols(), exported ^ declared_symbols()


def test_workspace_bytes_formula():
    lib = native.lib()
    # 64 rows x 32 heads, keys up to 448 in chunks of 64 -> 7 chunks of (64 + 4) floats each.
    got = lib.skv_attention_workspace_bytes(64, 32, 64, 448, 64, native.SKV_F16)
    assert got == 64 * 32 * 7 * (64 + 4) * 4
    # one chunk covers every key: no workspace
    assert lib.skv_attention_workspace_bytes(64, 32, 64, 448, 512, native.SKV_F16) == 0
    assert lib.skv_attention_workspace_bytes(0, 32, 64, 448, 64, native.SKV_F16) == 0


def test_default_chunk():
    lib = native.lib()
    # Enough (row, head) pairs to fill the GPU: one chunk covering every key,
    # rounded up to whole 4-wave passes (fp16 D=64: 4 waves x 64 keys = 256).
    assert lib.skv_default_chunk_tokens(64, 32, 64, 448, native.SKV_F16) == 512
    assert lib.skv_default_chunk_tokens(64, 20, 64, 1500, native.SKV_BF16) == 1536
    # Few pairs over long keys: split the keys so that ~1024 workgroups run.
    c = lib.skv_default_chunk_tokens(1, 20, 64, 1500, native.SKV_BF16)
    assert c == 256 and 20 * -(-1500 // c) <= 1024
    assert lib.skv_default_chunk_tokens(8, 20, 64, 4096, native.SKV_BF16) == 768
    # A (row, head) of at most 128 KB of K and V (512 keys at bf16 D=64) is never split ...
    assert lib.skv_default_chunk_tokens(1, 20, 64, 512, native.SKV_BF16) == 512
    assert lib.skv_default_chunk_tokens(1, 20, 64, 513, native.SKV_BF16) == 256
    # ... nor is one of at most 512 KB when there are 128 or more pairs.
    assert lib.skv_default_chunk_tokens(8, 20, 64, 1500, native.SKV_BF16) == 1536
    assert lib.skv_default_chunk_tokens(6, 20, 64, 1500, native.SKV_BF16) == 256
    assert lib.skv_default_chunk_tokens(8, 20, 64, 2049, native.SKV_BF16) == 512
    # fp32 D=64: 4 rows x 8 = 32 keys per wave -> 128-key passes
    assert lib.skv_default_chunk_tokens(1, 1, 64, 10, native.SKV_F32) == 128


def test_paged_default_chunk_fits_staged_block_ids():
    """Pools read through staged block ids (block sizes that are not powers of two, blocks shorter
    than one load instruction's keys, pools past 2 GiB) keep the default chunk within 254 blocks
    and a whole number of 64-key sub-chunks; the fast path keeps the dense default."""
    lib = native.lib()
    bf16 = native.SKV_BF16
    # 8 rows x 20 heads over 1500 keys: one 1536-key chunk by default; block size 6 caps it.
    assert lib.skv_paged_chunk_tokens(8, 20, 20, 64, 1500, bf16, 16, 4096) == 1536
    c = lib.skv_paged_chunk_tokens(8, 20, 20, 64, 1500, bf16, 6, 4096)
    assert c == (254 * 6 // 64) * 64 == 1472
    assert c // 6 + 2 <= 256
    # 64 rows x 16 heads over 4100 keys: block size 12 -> at most 254 * 12 = 3048 keys.
    assert lib.skv_paged_chunk_tokens(64, 16, 16, 64, 4100, bf16, 16, 20000) == 4352
    assert lib.skv_paged_chunk_tokens(64, 16, 16, 64, 4100, bf16, 12, 20000) == (254 * 12 // 64) * 64
    # 4-token blocks are below one bf16 D=64 load instruction's 8 keys: general path.
    assert lib.skv_paged_chunk_tokens(64, 16, 16, 64, 4100, bf16, 4, 80000) == (254 * 4 // 64) * 64
    # A 16-token-block pool past 2 GiB per layer (70000 blocks x 16 x 16 heads x 128 B) is general too.
    assert lib.skv_paged_chunk_tokens(64, 16, 16, 64, 4100, bf16, 16, 70000) == (254 * 16 // 64) * 64
    # Short rows are unaffected by the cap.
    assert lib.skv_paged_chunk_tokens(64, 20, 20, 64, 448, bf16, 6, 4096) == \
        lib.skv_default_chunk_tokens(64, 20, 64, 448, bf16)


FAKE = 1 << 20  # aligned, never dereferenced: validation fails before any launch


def test_append_rejects_bad_dtype():
    lib = native.lib()
    rc = lib.skv_append(FAKE, FAKE, 64, 64, FAKE, FAKE, FAKE, 4, 1, 64, 16, 7, None)
    assert rc == -2 and b"dtype" in lib.skv_last_error()


def test_append_rejects_misaligned_stride():
    lib = native.lib()
    rc = lib.skv_append(FAKE, FAKE, 63, 64, FAKE, FAKE, FAKE, 4, 1, 64, 16, native.SKV_F16, None)
    assert rc == -3


def test_attention_rejects_unsupported_head_dim():
    lib = native.lib()
    rc = lib.skv_paged_attention(FAKE, 48, 48, 48, FAKE, FAKE, FAKE, 4, None, FAKE, None, None, 0, 0, 0,
                                 FAKE, 48, 48, 48,
                                 1, 1, 1, 1, 48, 16, 8, 64, 1.0, 0, native.SKV_F16, 0, None, 0, None)
    assert rc == -1 and b"head_dim" in lib.skv_last_error()


def test_attention_requires_workspace_for_split_keys():
    lib = native.lib()
    rc = lib.skv_dense_attention(FAKE, 64, 64, 64, FAKE, FAKE, 64 * 1500, 64 * 1500, 64, None, FAKE, FAKE,
                                 64, 64, 64, 4, 1, 1, 1, 64, 1500, 0.125, 0, native.SKV_F16, 64, None, 0, None)
    assert rc == -4 and b"workspace" in lib.skv_last_error()
    # too small
    rc = lib.skv_dense_attention(FAKE, 64, 64, 64, FAKE, FAKE, 64 * 1500, 64 * 1500, 64, None, FAKE, FAKE,
                                 64, 64, 64, 4, 1, 1, 1, 64, 1500, 0.125, 0, native.SKV_F16, 64, FAKE, 64, None)
    assert rc == -4


def test_attention_rejects_bad_group():
    lib = native.lib()
    rc = lib.skv_dense_attention(FAKE, 64, 64, 64, FAKE, FAKE, 64, 64, 64, None, FAKE, FAKE, 64, 64, 64,
                                 1, 1, 3, 2, 64, 10, 0.125, 0, native.SKV_F16, 0, None, 0, None)
    assert rc == -1


def test_argmax_rejects_bad_arguments():
    lib = native.lib()

    def call(stride=100, rows=4, dtype=native.SKV_F16, slots=None, num_slots=0, tokens=None, eos=None,
             finished=None, count=None):
        return lib.skv_argmax(FAKE, stride, rows, 100, dtype, FAKE, slots, num_slots, tokens, eos, finished, count,
                              None)

    assert call(dtype=9) == -2
    assert call(stride=50) == -1                                    # stride < vocab
    assert call(slots=FAKE) == -1                                   # row_slots with no per-slot output
    assert call(tokens=FAKE, num_slots=8) == -1                     # slot output without row_slots
    assert call(slots=FAKE, num_slots=8, eos=FAKE, finished=FAKE) == -1   # EOS group incomplete
    assert call(slots=FAKE, num_slots=-1, tokens=FAKE) == -1
    assert call(rows=0) == 0                                        # nothing to do


def test_add_layernorm_rejects_bad_arguments():
    lib = native.lib()

    def call(dtype=native.SKV_BF16, hidden=1280, ldx=1280, rows=4, eps=1e-5):
        return lib.skv_add_layernorm(FAKE, ldx, None, hidden, FAKE, FAKE, eps, None, hidden, FAKE, hidden, rows,
                                     hidden, dtype, None)

    assert call(dtype=7) == -2
    assert call(hidden=1284, ldx=1288) == -1      # not a multiple of 8 bf16 elements
    assert call(hidden=8192, ldx=8192) == -1      # more than 512 vectors per row
    assert call(ldx=1284) == -3                   # row stride breaks 16-byte alignment
    assert call(eps=-1.0) == -1
    assert call(rows=0) == 0


def test_copy_cross_kv_rejects_bad_arguments():
    import ctypes as C
    lib = native.lib()

    def call(layers=2, heads=20, n=1500, d=64, dtype=native.SKV_BF16, srcs=True, stride_t=64):
        arr = (C.c_void_p * max(layers, 1))(*([FAKE] * max(layers, 1)))
        p = C.cast(arr, C.c_void_p) if srcs else None
        return lib.skv_copy_cross_kv(p, p, layers, 1500 * 64, stride_t, FAKE, 2 * 20 * 1500 * 64, 20 * 1500 * 64,
                                     1500 * 64, 64, heads, n, d, dtype, None)

    assert call(dtype=9) == -2
    assert call(layers=0) == -1 and call(layers=65) == -1
    assert call(heads=0) == -1 and call(n=-1) == -1
    assert call(d=48) == -3            # 96 bytes: not a power-of-two multiple of 16
    assert call(stride_t=60) == -3     # breaks 16-byte row alignment
    assert call(srcs=False) == -1
    assert call(n=0) == 0              # nothing to copy, no launch


def test_python_wrapper_refuses_cpu_tensors():
    import torch

    q = torch.zeros(1, 1, 64, dtype=torch.float16)
    pool = torch.zeros(4, 16, 1, 64, dtype=torch.float16)
    tbl = torch.zeros(1, 1, dtype=torch.int32)
    lens = torch.ones(1, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        native.paged_attention(q, pool, pool, tbl, lens, 1, 0.125)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        native.append(q, q, pool, pool, torch.zeros(1, dtype=torch.int64))


def test_library_was_built_from_this_tree():
    # skv_version() carries the digest of the sources and flags the library was compiled from;
    # the binding refuses a library whose digest is not this tree's.
    got = native.library_digest(native.lib())
    assert len(got) == 16 and got in native.expected_digests()
    assert f"src:{got}" in native.version()
