"""numpy oracle: paged KV append, block-table gather and softmax attention.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Arithmetic is float64.

Reference sites restated here (paths relative to the reference repository):
    slot_mapping        speech_serving/phase_aware_scheduler.py:1004-1005
    append              speech_serving/phase_aware_scheduler.py:1009-1010 (decode),
                        :681-690 (prefill write)
    gather              speech_serving/tts_engine.py:177-185,
                        speech_serving/phase_aware_scheduler.py:617-623 (one row),
                        :818-830 (zero-padded batch)
    attention           speech_serving/models.py:140-164 (self), :184-202 (cross)
    attention_masked    speech_serving/models.py:140-163 with the eager padding mask
                        of phase_aware_scheduler.py:837-846 / bool cross mask
                        :884-887, and the graph additive masks of
                        graph_decode_buffers.py:527-529
    paged_attention     scripts/evaluate_paging_variants.py:56-133 (same math as
                        the reference's Triton kernel: gather + attention)
"""
from __future__ import annotations

from typing import Optional, Sequence

import numpy as np


def slot_mapping(block_table: Sequence[int], positions: Sequence[int], block_size: int) -> np.ndarray:
    """slot = block_table[pos // BS] * BS + pos % BS (phase_aware_scheduler.py:1004-1005)."""
    return np.array([int(block_table[p // block_size]) * block_size + p % block_size for p in positions],
                    dtype=np.int64)


def append(k_pool: np.ndarray, v_pool: Optional[np.ndarray], k_new: np.ndarray, v_new: Optional[np.ndarray],
           slots: Sequence[int]) -> None:
    """In place: pool[slot // BS, slot % BS] = new[n] (phase_aware_scheduler.py:1009-1010).

    Rows with a negative or out-of-range slot are skipped.
    """
    nb, bs = k_pool.shape[:2]
    for n, s in enumerate(slots):
        s = int(s)
        if s < 0 or s >= nb * bs:
            continue
        k_pool[s // bs, s % bs] = k_new[n]
        if v_pool is not None:
            v_pool[s // bs, s % bs] = v_new[n]


def gather(pool: np.ndarray, block_tables: np.ndarray, lens: Sequence[int], max_len: int) -> np.ndarray:
    """[B, H, max_len, D]: pool[table].view(-1, H, D)[:T].permute(1, 0, 2), zero beyond T.

    Follows tts_engine.py:177-185 per row and the zero-padded batching of
    phase_aware_scheduler.py:818-830. Block ids outside the pool give zeros.
    """
    nb, bs, h, d = pool.shape
    out = np.zeros((len(lens), h, max_len, d), dtype=pool.dtype)
    for b, n in enumerate(lens):
        n = min(int(n), max_len, block_tables.shape[1] * bs)
        if n <= 0:
            continue
        nblk = (n + bs - 1) // bs
        rows = np.zeros((nblk, bs, h, d), dtype=pool.dtype)
        for i in range(nblk):
            blk = int(block_tables[b, i])
            if 0 <= blk < nb:
                rows[i] = pool[blk]
        flat = rows.reshape(-1, h, d)[:n]
        out[b, :, :n] = flat.transpose(1, 0, 2)
    return out


def visible(lens: Sequence[int], q_len: int, qi: int, b: int, causal: bool) -> int:
    n = int(lens[b]) - ((q_len - 1 - qi) if causal else 0)
    return max(0, n)


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, lens: Sequence[int], scale: float,
              causal: bool = False) -> np.ndarray:
    """softmax(q k^T * scale) v over each row's first `n` keys, in float64.

    q: [B, Q, H, D]; k, v: [B, Hkv, T, D]; lens[b] = keys visible to the last
    query; with causal, query qi sees lens[b] - (Q - 1 - qi) keys (the causal
    triu mask of models.py:159-161 applied after a cached prefix). A row that
    sees no key gives zeros. Math of models.py:140-164.
    """
    bsz, qlen, heads, d = q.shape
    hkv = k.shape[1]
    group = heads // hkv
    out = np.zeros((bsz, qlen, heads, d), dtype=np.float64)
    for b in range(bsz):
        for qi in range(qlen):
            n = min(visible(lens, qlen, qi, b, causal), k.shape[2])
            if n == 0:
                continue
            kk = np.repeat(k[b, :, :n].astype(np.float64), group, axis=0)  # [H, n, D]
            vv = np.repeat(v[b, :, :n].astype(np.float64), group, axis=0)
            qq = q[b, qi].astype(np.float64)  # [H, D]
            s = np.einsum("hd,htd->ht", qq, kk) * scale
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[b, qi] = np.einsum("ht,htd->hd", p, vv)
    return out


def attention_masked(q: np.ndarray, k: np.ndarray, v: np.ndarray, keep: np.ndarray, scale: float,
                     fill: Optional[float] = None, additive: Optional[np.ndarray] = None) -> np.ndarray:
    """The reference's padded form: scores over ALL T keys, then a mask.

    keep: bool [B, Q, T] (True = attend). With `fill`, masked scores are set to
    `fill` (models.py:150-155 uses finfo(dtype).min); with `additive`, the
    array is added to the scores (models.py:156-157 and graph_decode_buffers.py
    :527-529 use -10000 beyond the length). q: [B, Q, H, D]; k, v [B, H, T, D].
    """
    qq = q.astype(np.float64)
    kk = k.astype(np.float64)
    vv = v.astype(np.float64)
    s = np.einsum("bqhd,bhtd->bhqt", qq, kk) * scale
    if additive is not None:
        s = s + additive[:, None, :, :]
    if fill is not None:
        s = np.where(keep[:, None, :, :], s, fill)
    s -= s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    o = np.einsum("bhqt,bhtd->bqhd", p, vv)
    return o


def paged_attention(q: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray, block_tables: np.ndarray,
                    ctx_lens: Sequence[int], scale: float, causal: bool = False,
                    table_rows: Optional[Sequence[int]] = None) -> np.ndarray:
    """Gather each row's K/V through its block table, then `attention`.

    Same computation as the reference's Triton paged kernel
    (scripts/evaluate_paging_variants.py:56-133) and its eager check
    (scripts/generate_ablation_notebook.py:464-475).
    """
    if table_rows is not None:
        block_tables = block_tables[np.asarray(table_rows, dtype=np.int64)]
    bs = k_pool.shape[1]
    t = int(max(ctx_lens)) if len(ctx_lens) else 0
    t = min(t, block_tables.shape[1] * bs)
    k = gather(k_pool, block_tables, ctx_lens, max(t, 1))
    v = gather(v_pool, block_tables, ctx_lens, max(t, 1))
    return attention(q, k, v, ctx_lens, scale, causal)


def dense_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, lens: Sequence[int], scale: float,
                    causal: bool = False, slot_ids: Optional[Sequence[int]] = None) -> np.ndarray:
    """Attention over contiguous [S, Hkv, T, D] K/V; row b reads slot slot_ids[b] (or b).

    Cross-attention of models.py:184-202 (eager) and :468-479 (graph) with
    the tail beyond lens[b] masked.
    """
    if slot_ids is not None:
        idx = np.asarray(slot_ids, dtype=np.int64)
        k, v = k[idx], v[idx]
    else:
        k, v = k[: q.shape[0]], v[: q.shape[0]]
    return attention(q, k, v, lens, scale, causal)
