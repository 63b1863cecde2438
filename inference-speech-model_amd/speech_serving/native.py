"""ctypes binding of libspeechkv.so — the gfx950 decoder KV-cache kernels.

Every function here launches a hand-written HIP kernel on the caller's current
stream. There is no fallback: a missing library or a tensor that is not on a
GPU raises RuntimeError.

Functions:
    append(k_new, v_new, k_pool, v_pool, slot_mapping)
    gather(k_pool, v_pool, block_tables, lens, max_len)
    paged_attention(q, k_pool, v_pool, block_tables, ctx_lens, max_ctx, scale, ...)
    dense_attention(q, k, v, lens, max_len, scale, ...)
    argmax(logits, ...), copy_cross_kv(...), add_layernorm(...), codebook_embed_sum(...)
    linear(x, weight, bias)   (hipBLASLt with a plan cached per shape)
"""
from __future__ import annotations

import ctypes
import functools
import os
import threading
from typing import Dict, Optional, Sequence, Tuple

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libspeechkv.so")
_lib: Optional[ctypes.CDLL] = None
_lib_lock = threading.Lock()

SKV_F32, SKV_F16, SKV_BF16 = 0, 1, 2
SKV_ATTN_CAUSAL, SKV_ATTN_ROWS_LONGEST_FIRST = 1, 2  # bits of the attention calls' `causal`
_DTYPE_CODE = {torch.float32: SKV_F32, torch.float16: SKV_F16, torch.bfloat16: SKV_BF16}

# Exported entry points and their ctypes signatures (must match include/speech_kv.h).
_c_int, _c_i32, _c_i64, _c_p, _c_f = ctypes.c_int, ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float
SIGNATURES = {
    "skv_version": (ctypes.c_char_p, []),
    "skv_last_error": (ctypes.c_char_p, []),
    "skv_append": (_c_int, [_c_p, _c_p, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32, _c_p]),
    "skv_gather": (_c_int, [_c_p, _c_p, _c_p, _c_i32, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                            _c_i32, _c_i32, _c_p]),
    "skv_argmax": (_c_int, [_c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_p, _c_i32, _c_p, _c_p, _c_p, _c_p, _c_p]),
    "skv_copy_cross_kv": (_c_int, [_c_p, _c_p, _c_i32, _c_i64, _c_i64, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32,
                                   _c_i32, _c_i32, _c_i32, _c_p]),
    "skv_attention_workspace_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "skv_default_chunk_tokens": (_c_i32, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "skv_paged_chunk_tokens": (_c_i32, [_c_i32] * 8),
    "skv_paged_attention": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i32, _c_p, _c_p,
                                     _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p,
                                     _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                     _c_i32, _c_i32, _c_f, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_p]),
    "skv_paged_attention_noalloc": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_i32, _c_p, _c_p,
                                             _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p,
                                             _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                             _c_i32, _c_i32, _c_f, _c_i32, _c_i32, _c_i32, _c_p]),
    "skv_dense_attention": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p,
                                     _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
                                     _c_f, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_p]),
    "skv_add_layernorm": (_c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_f, _c_p, _c_i64, _c_p, _c_i64,
                                   _c_i32, _c_i32, _c_i32, _c_p]),
    "skv_codebook_embed_sum": (_c_int, [_c_p, _c_i64, _c_i32, _c_p, _c_i32, _c_i32, _c_i32, _c_p, _c_i64, _c_i32,
                                        _c_p]),
    "skv_linear": (_c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_p]),
}
SKV_EUNSUPPORTED = -5  # skv_linear: no workspace-free hipBLASLt algorithm for the shape
MAX_CODEBOOKS = 16  # kMaxCodebooks of the library


def library_path() -> str:
    return _LIB_PATH


_BUILD_SCRIPT = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "build.py")


def expected_digests() -> Optional[Tuple[str, ...]]:
    """Source digests a library built from this tree carries (release and debug flags), or None when
    the tree holds no build script and sources to compare with."""
    if not os.path.exists(_BUILD_SCRIPT):
        return None
    import importlib.util

    spec = importlib.util.spec_from_file_location("_speechkv_build", _BUILD_SCRIPT)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    if not mod.hashed_files():
        return None
    return mod.source_digest(False), mod.source_digest(True)


def library_digest(handle: ctypes.CDLL) -> str:
    """The src:<digest> field of a loaded library's skv_version()."""
    v = handle.skv_version().decode()
    return v.split("src:", 1)[1].split()[0] if "src:" in v else ""


def check_library(handle: ctypes.CDLL) -> None:
    """Raise RuntimeError unless the library was built from the sources in this tree."""
    want = expected_digests()
    if want is None:
        return
    got = library_digest(handle)
    if got not in want:
        raise RuntimeError(
            f"{_LIB_PATH} was built from other sources (library src:{got or 'none'}, this tree src:{want[0]}); "
            "rebuild it with `python inference-speech-model_amd/build.py`")


def lib() -> ctypes.CDLL:
    """Load libspeechkv.so (after torch, so it binds to torch's HIP runtime).

    The library must carry the source digest of this tree (see check_library): a
    binary left over from an earlier version of the kernels is refused."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise RuntimeError(
                    f"libspeechkv.so not found at {_LIB_PATH}; build it with "
                    "`python inference-speech-model_amd/build.py`")
            handle = ctypes.CDLL(_LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            check_library(handle)
            _lib = handle
    return _lib


def version() -> str:
    return lib().skv_version().decode()


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().skv_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def _code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


def _gpu(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (got device {t.device}); the HIP kernels have no CPU path")


# The current stream's raw handle without building a torch.cuda.Stream object (the per-call host
# cost of every entry point below).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    if _raw_stream is not None:
        return _raw_stream(torch.cuda.current_device() if device.index is None else device.index)
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _i32(t: torch.Tensor, name: str) -> torch.Tensor:
    _gpu(t, name)
    if t.dtype != torch.int32:
        raise RuntimeError(f"{name} must be int32 (got {t.dtype})")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    return t


# ---------------------------------------------------------------------------
# Split-K workspace: one buffer per device (fp32 partials; any content on
# entry), grown only outside graph capture.
# ---------------------------------------------------------------------------
_workspaces: Dict[int, torch.Tensor] = {}


def _dev_index(device) -> int:
    idx = (device if isinstance(device, torch.device) else torch.device(device)).index
    return torch.cuda.current_device() if idx is None else idx


def reserve_workspace(nbytes: int, device) -> torch.Tensor:
    """Return the device's workspace, grown to at least `nbytes`."""
    idx = _dev_index(device)
    ws = _workspaces.get(idx)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"attention workspace of {nbytes} bytes must be reserved before graph capture")
        size = max(int(nbytes), 1 << 20, 0 if ws is None else 2 * ws.numel())
        ws = torch.empty(size, dtype=torch.uint8, device=torch.device("cuda", idx))
        _workspaces[idx] = ws
    return ws


def reserve_attention(rows: int, heads: int, head_dim: int, max_len: int, dtype: torch.dtype, device,
                      chunk_tokens: int = 0) -> None:
    """Pre-size the workspace for an attention call shape (call before graph capture)."""
    need = attention_workspace_bytes(rows, heads, head_dim, max(max_len, 1), dtype, chunk_tokens)
    if need > 0:
        reserve_workspace(need, device)


def _scratch(need: int, device):
    if need <= 0:
        return None, 0
    ws = reserve_workspace(need, device)
    return ws.data_ptr(), ws.numel()


# The sizing queries are pure functions of their arguments: memoised, so a decode step's calls
# cost a dictionary lookup rather than a foreign call each.
@functools.lru_cache(maxsize=4096)
def _workspace_bytes(rows: int, heads: int, head_dim: int, max_len: int, chunk_tokens: int, code: int) -> int:
    return int(lib().skv_attention_workspace_bytes(rows, heads, head_dim, max_len, chunk_tokens, code))


@functools.lru_cache(maxsize=4096)
def _default_chunk(rows: int, heads: int, head_dim: int, max_len: int, code: int) -> int:
    return int(lib().skv_default_chunk_tokens(rows, heads, head_dim, max_len, code))


@functools.lru_cache(maxsize=4096)
def _paged_chunk(rows: int, heads: int, kv_heads: int, head_dim: int, max_ctx: int, code: int, block_size: int,
                 num_blocks: int) -> int:
    return int(lib().skv_paged_chunk_tokens(rows, heads, kv_heads, head_dim, max_ctx, code, block_size, num_blocks))


def attention_workspace_bytes(rows: int, heads: int, head_dim: int, max_len: int, dtype: torch.dtype,
                              chunk_tokens: int = 0) -> int:
    return _workspace_bytes(int(rows), int(heads), int(head_dim), int(max_len), int(chunk_tokens), _code(dtype))


def default_chunk_tokens(rows: int, heads: int, head_dim: int, max_len: int, dtype: torch.dtype) -> int:
    return _default_chunk(int(rows), int(heads), int(head_dim), int(max_len), _code(dtype))


def paged_chunk_tokens(rows: int, heads: int, kv_heads: int, head_dim: int, max_ctx: int, dtype: torch.dtype,
                       block_size: int, num_blocks: int) -> int:
    """The chunk skv_paged_attention takes by default for pools of num_blocks x block_size tokens."""
    return _paged_chunk(int(rows), int(heads), int(kv_heads), int(head_dim), int(max_ctx), _code(dtype),
                        int(block_size), int(num_blocks))


# ---------------------------------------------------------------------------
# Entry points.
# ---------------------------------------------------------------------------
def append(k_new: torch.Tensor, v_new: Optional[torch.Tensor], k_pool: torch.Tensor,
           v_pool: Optional[torch.Tensor], slot_mapping: torch.Tensor) -> None:
    """pool[slot // BS, slot % BS] = new row, for each of the N rows of k_new/v_new.

    k_new, v_new: [N, H, D] (any row/head strides, D contiguous).
    k_pool, v_pool: [num_blocks, block_size, H, D] contiguous.
    slot_mapping: int64 [N]; a negative slot skips the row.
    Same bytes as `key_pool[l][blk, off] = new_k` in the reference
    (speech_serving/phase_aware_scheduler.py:1004-1010).
    """
    for t, n in ((k_new, "k_new"), (k_pool, "k_pool"), (slot_mapping, "slot_mapping")):
        _gpu(t, n)
    if (v_new is None) != (v_pool is None):
        raise RuntimeError("append: v_new and v_pool must both be given or both be None")
    if k_new.dim() != 3:
        raise RuntimeError(f"append: k_new must be [N, H, D], got {tuple(k_new.shape)}")
    n, h, d = k_new.shape
    if k_pool.dim() != 4 or k_pool.shape[2] != h or k_pool.shape[3] != d or not k_pool.is_contiguous():
        raise RuntimeError(f"append: pool {tuple(k_pool.shape)} does not match rows [*, *, {h}, {d}] / not contiguous")
    if k_new.dtype != k_pool.dtype:
        k_new = k_new.to(k_pool.dtype)
    if k_new.stride(2) != 1:
        k_new = k_new.contiguous()
    if v_new is not None:
        _gpu(v_new, "v_new")
        _gpu(v_pool, "v_pool")
        if v_pool.shape != k_pool.shape or v_pool.dtype != k_pool.dtype or not v_pool.is_contiguous():
            raise RuntimeError("append: v_pool must match k_pool")
        if v_new.dtype != v_pool.dtype:
            v_new = v_new.to(v_pool.dtype)
        if v_new.shape != k_new.shape:
            raise RuntimeError("append: v_new must match k_new's shape")
        if v_new.stride() != k_new.stride():
            k_new, v_new = k_new.contiguous(), v_new.contiguous()
    if slot_mapping.dtype != torch.int64 or slot_mapping.numel() != n:
        raise RuntimeError(f"append: slot_mapping must be int64 [{n}]")
    slot_mapping = slot_mapping.contiguous()
    num_slots = k_pool.shape[0] * k_pool.shape[1]
    rc = lib().skv_append(k_new.data_ptr(), _ptr(v_new), k_new.stride(0), k_new.stride(1), k_pool.data_ptr(),
                          _ptr(v_pool), slot_mapping.data_ptr(), n, h, d, num_slots, _code(k_pool.dtype),
                          _stream(k_pool.device))
    _check(rc, "skv_append")


MAX_CROSS_LAYERS = 64  # layers per skv_copy_cross_kv launch


def copy_cross_kv(k_srcs: Sequence[torch.Tensor], v_srcs: Sequence[torch.Tensor], dst: torch.Tensor,
                  n_tokens: int) -> None:
    """dst[l, 0, :, :n] = k_srcs[l][:, :n] and dst[l, 1, :, :n] = v_srcs[l][:, :n] for every layer l, in one
    launch per 64 layers.

    k_srcs, v_srcs: per-layer [H, T, D] tensors (D contiguous; cast to dst's dtype when they differ).
    dst: the slot's [L, 2, H, T_max, D] region of the slot-major cross-attention buffer (D contiguous).
    Same bytes as GraphDecodeBuffers.assign_slot's per-layer copy_ loop in the reference
    (speech_serving/graph_decode_buffers.py:317-327).
    """
    if len(k_srcs) != len(v_srcs) or not k_srcs:
        raise RuntimeError("copy_cross_kv: k_srcs and v_srcs must be non-empty lists of equal length")
    _gpu(dst, "dst")
    if dst.dim() != 5 or dst.shape[1] != 2 or dst.stride(4) != 1 or dst.shape[0] < len(k_srcs):
        raise RuntimeError(f"copy_cross_kv: dst must be [L>={len(k_srcs)}, 2, H, T, D] with D contiguous, "
                           f"got {tuple(dst.shape)}")
    _, _, h, t_max, d = dst.shape
    if not 0 <= n_tokens <= t_max:
        raise RuntimeError(f"copy_cross_kv: n_tokens {n_tokens} outside [0, {t_max}]")
    srcs = []
    for k, v in zip(k_srcs, v_srcs):
        pair = []
        for x, name in ((k, "k_srcs"), (v, "v_srcs")):
            _gpu(x, name)
            if x.dim() != 3 or x.shape[0] != h or x.shape[2] != d or x.shape[1] < n_tokens:
                raise RuntimeError(f"copy_cross_kv: {name} entries must be [{h}, >={n_tokens}, {d}], "
                                   f"got {tuple(x.shape)}")
            if x.dtype != dst.dtype or x.stride(2) != 1:
                x = x[:, :n_tokens].to(dst.dtype).contiguous()
            pair.append(x)
        srcs.append(tuple(pair))
    if n_tokens == 0:
        return
    if len({(x.stride(0), x.stride(1)) for pr in srcs for x in pr}) != 1:  # one stride pair per launch
        srcs = [tuple(x[:, :n_tokens].contiguous() for x in pr) for pr in srcs]
    sh, st = srcs[0][0].stride(0), srcs[0][0].stride(1)
    for l0 in range(0, len(srcs), MAX_CROSS_LAYERS):
        part = srcs[l0:l0 + MAX_CROSS_LAYERS]
        kp = (ctypes.c_void_p * len(part))(*[k.data_ptr() for k, _ in part])
        vp = (ctypes.c_void_p * len(part))(*[v.data_ptr() for _, v in part])
        base = dst[l0]
        rc = lib().skv_copy_cross_kv(ctypes.cast(kp, ctypes.c_void_p), ctypes.cast(vp, ctypes.c_void_p), len(part),
                                     sh, st, base.data_ptr(), dst.stride(0), dst.stride(1),
                                     dst.stride(2), dst.stride(3), h, n_tokens, d, _code(dst.dtype),
                                     _stream(dst.device))
        _check(rc, "skv_copy_cross_kv")


def gather(k_pool: torch.Tensor, v_pool: Optional[torch.Tensor], block_tables: torch.Tensor,
           lens: torch.Tensor, max_len: int, k_out: Optional[torch.Tensor] = None,
           v_out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Contiguous [B, H, max_len, D] copies of the paged K/V, zero beyond lens[b].

    Row b's token t comes from pool[block_tables[b, t // BS], t % BS]; this is
    `pool[table].view(-1, H, D)[:T].permute(1, 0, 2)` of the reference
    (speech_serving/tts_engine.py:177-185) batched with zero padding
    (speech_serving/phase_aware_scheduler.py:818-830).
    """
    _gpu(k_pool, "k_pool")
    block_tables = _i32(block_tables, "block_tables")
    lens = _i32(lens, "lens")
    if block_tables.dim() != 2:
        raise RuntimeError("gather: block_tables must be [B, max_blocks]")
    b = block_tables.shape[0]
    nb, bs, h, d = k_pool.shape
    if not k_pool.is_contiguous():
        raise RuntimeError("gather: pool must be contiguous")
    if lens.numel() < b:
        raise RuntimeError(f"gather: lens has {lens.numel()} entries for {b} rows")
    if k_out is None:
        k_out = torch.empty((b, h, max_len, d), dtype=k_pool.dtype, device=k_pool.device)
    if v_pool is not None and v_out is None:
        v_out = torch.empty((b, h, max_len, d), dtype=v_pool.dtype, device=v_pool.device)
    for t in (k_out, v_out):
        if t is not None and (tuple(t.shape) != (b, h, max_len, d) or not t.is_contiguous()):
            raise RuntimeError(f"gather: output must be contiguous [{b}, {h}, {max_len}, {d}]")
    if v_pool is not None and (v_pool.shape != k_pool.shape or not v_pool.is_contiguous()):
        raise RuntimeError("gather: v_pool must match k_pool")
    rc = lib().skv_gather(k_pool.data_ptr(), _ptr(v_pool), block_tables.data_ptr(), block_tables.shape[1],
                          lens.data_ptr(), k_out.data_ptr(), _ptr(v_out), b, h, d, bs, nb, max_len,
                          _code(k_pool.dtype), _stream(k_pool.device))
    _check(rc, "skv_gather")
    return k_out, v_out


def argmax(logits: torch.Tensor, out: Optional[torch.Tensor] = None, row_slots: Optional[torch.Tensor] = None,
           slot_tokens: Optional[torch.Tensor] = None, slot_eos: Optional[torch.Tensor] = None,
           slot_finished: Optional[torch.Tensor] = None, finished_count: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Greedy tokens: first index of each row's maximum, int64 [rows].

    logits: [rows, vocab] (row stride may exceed vocab). torch.argmax(dim=-1)
    semantics (speech_serving/models.py:486-487). Per-slot outputs for rows whose
    slot row_slots[r] (int32 [rows]) is in [0, num_slots):
      slot_tokens (int64 [num_slots]): slot_tokens[slot] = token;
      slot_eos (int64 [num_slots], < 0 = none), slot_finished (int32 [num_slots]),
      finished_count (int64 [>= 1]): a token equal to its slot's EOS id sets the
      slot's finished flag once and adds 1 to finished_count[0].
    """
    _gpu(logits, "logits")
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise RuntimeError("argmax: logits must be [rows, vocab] with a contiguous last dim")
    rows, vocab = logits.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    if out.dtype != torch.int64 or out.numel() < rows or not out.is_contiguous():
        raise RuntimeError("argmax: out must be contiguous int64 covering the rows")
    eos_args = (slot_eos, slot_finished, finished_count)
    if any(a is not None for a in eos_args) and not all(a is not None for a in eos_args):
        raise RuntimeError("argmax: slot_eos, slot_finished and finished_count go together")
    want_slots = slot_tokens is not None or slot_eos is not None
    if want_slots != (row_slots is not None):
        raise RuntimeError("argmax: row_slots is required by, and only used with, slot_tokens / slot_eos")
    num_slots = 0
    if row_slots is not None:
        row_slots = _i32(row_slots, "row_slots")
        if row_slots.numel() < rows:
            raise RuntimeError("argmax: row_slots must cover the rows")
        sizes = []
        if slot_tokens is not None:
            _gpu(slot_tokens, "slot_tokens")
            if slot_tokens.dtype != torch.int64 or not slot_tokens.is_contiguous():
                raise RuntimeError("argmax: slot_tokens must be contiguous int64")
            sizes.append(slot_tokens.numel())
        if slot_eos is not None:
            for t, n, dt in ((slot_eos, "slot_eos", torch.int64), (slot_finished, "slot_finished", torch.int32),
                             (finished_count, "finished_count", torch.int64)):
                _gpu(t, n)
                if t.dtype != dt or not t.is_contiguous():
                    raise RuntimeError(f"argmax: {n} must be contiguous {dt}")
            if slot_finished.numel() != slot_eos.numel() or finished_count.numel() < 1:
                raise RuntimeError("argmax: slot_finished must match slot_eos; finished_count needs one element")
            sizes.append(slot_eos.numel())
        if len(set(sizes)) != 1:
            raise RuntimeError("argmax: slot_tokens and slot_eos must have one entry per slot")
        num_slots = sizes[0]
    rc = lib().skv_argmax(logits.data_ptr(), logits.stride(0), rows, vocab, _code(logits.dtype), out.data_ptr(),
                          _ptr(row_slots), num_slots, _ptr(slot_tokens), _ptr(slot_eos), _ptr(slot_finished),
                          _ptr(finished_count), _stream(logits.device))
    _check(rc, "skv_argmax")
    return out


def _q4(q: torch.Tensor, name: str) -> torch.Tensor:
    """View q/out as [B, Q, H, D]; a 3-D input is [B, H, D] with Q = 1."""
    if q.dim() == 3:
        return q.unsqueeze(1)
    if q.dim() == 4:
        return q
    raise RuntimeError(f"{name} must be [B, H, D] or [B, Q, H, D], got {tuple(q.shape)}")


def paged_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor, block_tables: torch.Tensor,
                    ctx_lens: torch.Tensor, max_ctx: int, scale: float, causal: bool = False,
                    table_rows: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                    chunk_tokens: int = 0, k_new: Optional[torch.Tensor] = None,
                    v_new: Optional[torch.Tensor] = None, noalloc: bool = False,
                    rows_longest_first: bool = False) -> torch.Tensor:
    """softmax(q K^T * scale) V over each row's paged K/V.

    q: [B, H, D] or [B, Q, H, D]; pools [num_blocks, BS, Hkv, D]; block_tables
    int32 [*, max_blocks]; ctx_lens int32 [B] = keys visible to the last query
    (new token included); causal: query qi sees ctx_lens[b] - (Q - 1 - qi) keys.
    With k_new/v_new ([B, Q, Hkv, D] or [B, Hkv, D]) the Q newest keys
    (positions ctx_lens[b]-Q .. ctx_lens[b]-1) are appended into the pools
    through the block table in the same launch.
    With noalloc the call goes through skv_paged_attention_noalloc: split-K partials in the library's
    fixed per-device scratch (at most 4 MiB), no workspace; pass `out` to allocate nothing at all.
    rows_longest_first: the rows come in non-increasing ctx_lens order (the launch then skips ranking
    them by length; results are the same either way).
    Reference math: speech_serving/models.py:126-165 and :444-466; append:
    speech_serving/phase_aware_scheduler.py:1004-1010.
    """
    for t, n in ((q, "q"), (k_pool, "k_pool"), (v_pool, "v_pool")):
        _gpu(t, n)
    block_tables = _i32(block_tables, "block_tables")
    ctx_lens = _i32(ctx_lens, "ctx_lens")
    if table_rows is not None:
        table_rows = _i32(table_rows, "table_rows")
    q4 = _q4(q, "q")
    bsz, qlen, heads, d = q4.shape
    nb, bs, hkv, dk = k_pool.shape
    if dk != d or v_pool.shape != k_pool.shape or not (k_pool.is_contiguous() and v_pool.is_contiguous()):
        raise RuntimeError("paged_attention: pools must be contiguous [num_blocks, BS, Hkv, D] matching q")
    if q4.dtype != k_pool.dtype or v_pool.dtype != k_pool.dtype:
        raise RuntimeError(f"paged_attention: dtype mismatch q={q4.dtype} pool={k_pool.dtype}")
    if block_tables.dim() != 2 or ctx_lens.numel() < bsz:
        raise RuntimeError("paged_attention: block_tables must be 2-D and ctx_lens must cover the batch")
    if table_rows is None and block_tables.shape[0] < bsz:
        raise RuntimeError(f"paged_attention: {block_tables.shape[0]} table rows for batch {bsz}")
    if table_rows is not None and table_rows.numel() < bsz:
        raise RuntimeError("paged_attention: table_rows must cover the batch")
    if q4.stride(3) != 1:
        q4 = q4.contiguous()
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    o4 = _q4(out, "out")
    if tuple(o4.shape) != tuple(q4.shape) or o4.stride(3) != 1:
        raise RuntimeError("paged_attention: out must match q's shape with contiguous head_dim")
    code = _code(q4.dtype)
    max_ctx = max(0, min(int(max_ctx), block_tables.shape[1] * bs))
    if chunk_tokens <= 0:
        chunk_tokens = _paged_chunk(bsz * qlen, heads, hkv, d, max(max_ctx, 1), code, bs, nb)
    kn4 = vn4 = None
    nstr = (0, 0, 0)
    if (k_new is None) != (v_new is None):
        raise RuntimeError("paged_attention: k_new and v_new must both be given or both be None")
    if k_new is not None:
        _gpu(k_new, "k_new")
        _gpu(v_new, "v_new")
        kn4, vn4 = _q4(k_new, "k_new"), _q4(v_new, "v_new")
        if tuple(kn4.shape) != (bsz, qlen, hkv, d) or tuple(vn4.shape) != (bsz, qlen, hkv, d):
            raise RuntimeError(f"paged_attention: k_new/v_new must be [{bsz}, {qlen}, {hkv}, {d}]")
        if kn4.dtype != k_pool.dtype or vn4.dtype != k_pool.dtype:
            raise RuntimeError("paged_attention: k_new/v_new dtype must match the pool")
        if kn4.stride(3) != 1 or vn4.stride(3) != 1 or kn4.stride() != vn4.stride():
            kn4, vn4 = kn4.contiguous(), vn4.contiguous()
        nstr = (kn4.stride(0), kn4.stride(1), kn4.stride(2))
    args = (q4.data_ptr(), q4.stride(0), q4.stride(1), q4.stride(2), k_pool.data_ptr(), v_pool.data_ptr(),
            block_tables.data_ptr(), block_tables.stride(0), _ptr(table_rows), ctx_lens.data_ptr(),
            _ptr(kn4), _ptr(vn4), nstr[0], nstr[1], nstr[2],
            o4.data_ptr(), o4.stride(0), o4.stride(1), o4.stride(2), bsz, qlen, heads, hkv, d, bs, nb, max_ctx,
            float(scale), (SKV_ATTN_CAUSAL if causal else 0) | (SKV_ATTN_ROWS_LONGEST_FIRST if rows_longest_first else 0),
            code, chunk_tokens)
    if noalloc:
        _check(lib().skv_paged_attention_noalloc(*args, _stream(q.device)), "skv_paged_attention_noalloc")
        return out
    need = _workspace_bytes(bsz * qlen, heads, d, max_ctx, chunk_tokens, code)
    wp, wn = _scratch(need, q.device)
    _check(lib().skv_paged_attention(*args, wp, wn, _stream(q.device)), "skv_paged_attention")
    return out


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, lens: torch.Tensor, max_len: int,
                    scale: float, causal: bool = False, slot_ids: Optional[torch.Tensor] = None,
                    out: Optional[torch.Tensor] = None, chunk_tokens: int = 0) -> torch.Tensor:
    """Attention over contiguous K/V laid out [S, Hkv, T, D] (any strides, D contiguous).

    Row b attends slot slot_ids[b] (or b) over its first lens[b] positions.
    Cross-attention reference: speech_serving/models.py:167-203 and :468-479.
    """
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _gpu(t, n)
    lens = _i32(lens, "lens")
    if slot_ids is not None:
        slot_ids = _i32(slot_ids, "slot_ids")
    if k.dim() != 4 or v.shape != k.shape or k.stride() != v.stride() or k.stride(3) != 1:
        raise RuntimeError("dense_attention: k/v must be [S, Hkv, T, D] with equal strides, D contiguous")
    q4 = _q4(q, "q")
    bsz, qlen, heads, d = q4.shape
    _, hkv, tmax, dk = k.shape
    if dk != d:
        raise RuntimeError("dense_attention: head_dim mismatch")
    if lens.numel() < bsz:
        raise RuntimeError("dense_attention: lens must cover the batch")
    if slot_ids is None and k.shape[0] < bsz:
        raise RuntimeError(f"dense_attention: {k.shape[0]} K/V slots for batch {bsz}")
    if slot_ids is not None and slot_ids.numel() < bsz:
        raise RuntimeError("dense_attention: slot_ids must cover the batch")
    if q4.dtype != k.dtype or v.dtype != k.dtype:
        raise RuntimeError(f"dense_attention: dtype mismatch q={q4.dtype} k={k.dtype}")
    if q4.stride(3) != 1:
        q4 = q4.contiguous()
    if out is None:
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    o4 = _q4(out, "out")
    if tuple(o4.shape) != tuple(q4.shape) or o4.stride(3) != 1:
        raise RuntimeError("dense_attention: out must match q's shape with contiguous head_dim")
    max_len = max(0, min(int(max_len), tmax))
    code = _code(q4.dtype)
    if chunk_tokens <= 0:
        chunk_tokens = _default_chunk(bsz * qlen, heads, d, max(max_len, 1), code)
    need = _workspace_bytes(bsz * qlen, heads, d, max_len, chunk_tokens, code)
    wp, wn = _scratch(need, q.device)
    rc = lib().skv_dense_attention(
        q4.data_ptr(), q4.stride(0), q4.stride(1), q4.stride(2), k.data_ptr(), v.data_ptr(),
        k.stride(0), k.stride(1), k.stride(2), _ptr(slot_ids), lens.data_ptr(), o4.data_ptr(),
        o4.stride(0), o4.stride(1), o4.stride(2), bsz, qlen, heads, hkv, d, max_len, float(scale),
        1 if causal else 0, code, chunk_tokens, wp, wn, _stream(q.device))
    _check(rc, "skv_dense_attention")
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """x @ weight.T (+ bias): x [..., k], weight [n, k] with contiguous rows, bias [n], one dtype, on the GPU.

    One skv_linear call: a hipBLASLt plan cached per shape, where torch's linear rebuilds its descriptors
    and reruns the algorithm heuristic on every call. At the decode shapes the algorithm (and so every
    bit of the result) is the one torch's linear runs. Where hipBLASLt has no workspace-free algorithm for
    the shape, torch's linear runs instead. Reference: the nn.Linear projections of
    speech_serving/models.py:127-207 and the LM head (:416, :486).
    """
    k = x.shape[-1]
    if not x.is_cuda or not weight.is_cuda:
        raise RuntimeError("linear: x and weight must be GPU tensors; the HIP path has no CPU variant")
    code = _DTYPE_CODE.get(x.dtype)
    if code is None or weight.dtype != x.dtype or weight.dim() != 2 or weight.shape[1] != k or weight.stride(1) != 1:
        raise RuntimeError(f"linear: weight {tuple(weight.shape)} {weight.dtype} does not fit x [..., {k}] {x.dtype}")
    n = weight.shape[0]
    if bias is not None and (bias.dtype != x.dtype or bias.dim() != 1 or bias.shape[0] != n or bias.stride(0) != 1
                             or not bias.is_cuda):
        raise RuntimeError(f"linear: bias must be a contiguous GPU [{n}] {x.dtype} vector")
    x2 = x.reshape(-1, k)
    m = x2.shape[0]
    if x2.stride(1) != 1 or (m > 1 and x2.stride(0) < k):  # e.g. rows broadcast from one (stride 0)
        x2 = x2.contiguous()
    y = torch.empty(x.shape[:-1] + (n,), dtype=x.dtype, device=x.device)
    rc = lib().skv_linear(x2.data_ptr(), x2.stride(0) if m > 1 else k, weight.data_ptr(),
                          weight.stride(0) if n > 1 else k, None if bias is None else bias.data_ptr(),
                          y.data_ptr(), n, m, n, k, code, _stream(x.device))
    if rc == SKV_EUNSUPPORTED:
        return torch.nn.functional.linear(x, weight, bias)
    _check(rc, "skv_linear")
    return y


def add_layernorm_supported(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether skv_add_layernorm takes this LayerNorm: a GPU tensor of a supported dtype whose
    hidden size is a multiple of the 16-byte vector (and at most 512 vectors), with 16-byte rows."""
    return _layernorm_rows(x, weight) is not None


def _layernorm_rows(x: torch.Tensor, weight: torch.Tensor):
    """(x as [rows, hidden], hidden, 16-byte vectors per element count) when skv_add_layernorm takes x
    with this weight, else None."""
    if not x.is_cuda or weight.dtype != x.dtype or x.dtype not in _DTYPE_CODE or x.stride(-1) != 1:
        return None
    h = x.shape[-1]
    epl = 16 // x.element_size()
    if h == 0 or h % epl or h > 512 * epl:
        return None
    x2 = x.reshape(-1, h)
    if x2.shape[0] and (x2.stride(0) % epl or x2.data_ptr() % 16):
        return None
    return x2, h, epl


def add_layernorm(x: torch.Tensor, y: Optional[torch.Tensor], weight: torch.Tensor, bias: torch.Tensor,
                  eps: float, sum_out: Optional[torch.Tensor] = None,
                  fallback: bool = False) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
    """(s, LayerNorm(s)) with s = x + y rounded to x's dtype (s = x when y is None).

    x, y [..., hidden]; weight, bias [hidden]. sum_out may be x (in-place residual). An x the kernel
    does not take (a CPU tensor, another dtype, a hidden size that is not a multiple of the 16-byte
    vector or above 512 of them, rows that are not 16-byte aligned, a weight or bias of another size)
    raises RuntimeError, or with fallback=True returns None (the caller then runs torch's ops).
    """
    got = _layernorm_rows(x, weight)
    if got is not None and (not weight.is_contiguous() or weight.numel() != got[1] or bias.dtype != x.dtype or
                            not bias.is_contiguous() or bias.numel() != got[1]):
        got = None
    if got is None:
        if fallback:
            return None
        _gpu(x, "x")
        raise RuntimeError("add_layernorm: unsupported dtype, hidden size, layout or weight/bias shape")
    x2, h, epl = got
    rows = x2.shape[0]
    y2 = None
    if y is not None:
        _gpu(y, "y")
        y2 = y.reshape(rows, h)
        if y2.dtype != x.dtype or y2.stride(-1) != 1 or y2.data_ptr() % 16:
            raise RuntimeError("add_layernorm: y must match x's dtype with 16-byte rows")
        if sum_out is None:
            sum_out = torch.empty_like(x)
    s2 = sum_out.reshape(rows, h) if sum_out is not None else None
    norm = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    many = rows > 1
    rc = lib().skv_add_layernorm(x2.data_ptr(), x2.stride(0) if many else h, _ptr(y2),
                                 y2.stride(0) if many and y2 is not None else h,
                                 weight.data_ptr(), bias.data_ptr(), float(eps),
                                 _ptr(s2), s2.stride(0) if many and s2 is not None else h, norm.data_ptr(), h, rows,
                                 h, _DTYPE_CODE[x.dtype], _stream(x.device))
    _check(rc, "skv_add_layernorm")
    return (sum_out if y is not None else x), norm


def codebook_embed_sum(codes: torch.Tensor, tables: Sequence[torch.Tensor]) -> torch.Tensor:
    """sum_k tables[k][codes[..., k]] added left to right, each partial sum rounded to the tables'
    dtype: the bits of the reference's `embeds = embeds + emb_k(codes[..., k])` loop
    (speech_serving/models.py:39-52), in one launch. codes [..., K] int64; tables K x [vocab, dim].
    A code outside [0, vocab) adds a zero row (nn.Embedding would raise)."""
    _gpu(codes, "codes")
    k = codes.shape[-1]
    if not 1 <= k <= MAX_CODEBOOKS or len(tables) != k:
        raise RuntimeError(f"codebook_embed_sum: {len(tables)} tables for {k} codebooks (1..{MAX_CODEBOOKS})")
    vocab, dim = tables[0].shape
    dt = tables[0].dtype
    for i, t in enumerate(tables):
        _gpu(t, f"tables[{i}]")
        if t.shape != (vocab, dim) or t.dtype != dt or not t.is_contiguous() or t.data_ptr() % 16:
            raise RuntimeError("codebook_embed_sum: tables must be contiguous [vocab, dim] of one dtype, "
                               "16-byte aligned")
    if dt not in _DTYPE_CODE:
        raise RuntimeError(f"codebook_embed_sum: unsupported dtype {dt}")
    c2 = codes.reshape(-1, k)
    if c2.dtype != torch.int64 or c2.stride(-1) != 1:
        c2 = c2.to(torch.int64).contiguous()
    rows = c2.shape[0]
    out = torch.empty(codes.shape[:-1] + (dim,), dtype=dt, device=codes.device)
    ptrs = (ctypes.c_void_p * k)(*[t.data_ptr() for t in tables])
    rc = lib().skv_codebook_embed_sum(c2.data_ptr(), c2.stride(0) if rows > 1 else k, rows, ptrs, k, vocab, dim,
                                      out.data_ptr(), dim, _code(dt), _stream(codes.device))
    _check(rc, "skv_codebook_embed_sum")
    return out
