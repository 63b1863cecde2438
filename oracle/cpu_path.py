"""fp32 torch restatement of the reference's eager CPU path: the CPU baseline bench.py times.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): bench.py's cpu_baseline leg times it on the
host cores, tests/test_cpu_path.py pins it. The product path never imports it.

The reference runs its engine eagerly in torch; on a CPU that is float32 torch ops on the host's
threads. Restated here from the reference's source text (paths relative to the reference repository):
    Decoder.layer        DecoderLayer.forward, speech_serving/models.py:110-208: pre-LN
                         self-attention over the concatenated past (triu mask for a
                         multi-token input, a 0/1 padding mask otherwise), cross-attention
                         over the encoder K/V (bool mask for padded lengths), MLP on norm3
                         when cross-attention ran, else norm2; exact GELU
    Decoder.decode_step  WhisperClassSpeechEncoderDecoderModel.decode_step, models.py:369-423
    EagerDecode          the scheduler's eager decode loop, phase_aware_scheduler.py:771-1044:
                         per step the batch's working K/V (each request's contiguous past,
                         concatenated when the lengths agree, zero-padded with a mask when
                         they do not), one batched decoder pass, the new K/V written into
                         the paged pool (:1001-1010) and appended to each request's working
                         copy (:1012-1018), a batched greedy argmax
    paged_attention_step append + block-table gather into a zero-padded batch + masked softmax
                         attention: the same step for one layer (:795-846, :1001-1010 with
                         models.py:126-165)
    TTSModel / tts_step  StreamingMultiCodebookTTSModel.forward, models.py:23-77, 251-295, and
                         StreamingTTSEngine.step, tts_engine.py:154-239: per request, gather the
                         past from the pool, one frame forward, scatter the new K/V, argmax per
                         codebook
"""
from __future__ import annotations

import math
import time
from typing import Dict, List, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

NEG = torch.finfo(torch.float32).min


def _ln(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return F.layer_norm(x, (x.shape[-1],), w, b, 1e-5)


class Decoder:
    """Decoder layers of a reference state dict (parameter names of models.py), float32 on the CPU."""

    def __init__(self, state: Dict[str, torch.Tensor], num_heads: int, head_dim: int, prefix: str = "decoder_layers",
                 norm: str = "decoder_norm"):
        self.p = {k: v.detach().to("cpu", torch.float32).contiguous() for k, v in state.items()}
        self.h, self.d = num_heads, head_dim
        self.prefix, self.norm = prefix, norm
        self.n = len({k.split(".")[1] for k in state if k.startswith(prefix + ".")})

    def _heads(self, x: torch.Tensor) -> torch.Tensor:
        b, s, _ = x.shape
        return x.view(b, s, self.h, self.d).transpose(1, 2)

    def layer(self, i: int, x: torch.Tensor, past: Optional[Tuple[torch.Tensor, torch.Tensor]],
              cross: Optional[Tuple[torch.Tensor, torch.Tensor]], self_mask: Optional[torch.Tensor] = None,
              cross_mask: Optional[torch.Tensor] = None):
        P = lambda n: self.p[f"{self.prefix}.{i}.{n}"]  # noqa: E731
        b, s, _ = x.shape
        scale = 1.0 / math.sqrt(self.d)
        h1 = _ln(x, P("norm1.weight"), P("norm1.bias"))
        q = self._heads(F.linear(h1, P("self_attn_q.weight")))
        k = self._heads(F.linear(h1, P("self_attn_k.weight")))
        v = self._heads(F.linear(h1, P("self_attn_v.weight")))
        if past is not None:
            k = torch.cat([past[0], k], dim=2)
            v = torch.cat([past[1], v], dim=2)
        w = torch.matmul(q, k.transpose(-2, -1)) * scale
        if s > 1:
            w = w + torch.triu(torch.full((s, k.shape[2]), NEG), diagonal=1)
        if self_mask is not None:  # [B, T] 1 = attend
            w = w.masked_fill(self_mask[:, None, None, :] == 0, NEG)
        o = torch.matmul(torch.softmax(w, dim=-1), v).transpose(1, 2).reshape(b, s, -1)
        x = x + F.linear(o, P("self_attn_out.weight"))
        if cross is not None:
            h2 = _ln(x, P("norm2.weight"), P("norm2.bias"))
            cq = self._heads(F.linear(h2, P("cross_attn_q.weight")))
            cw = torch.matmul(cq, cross[0].transpose(-2, -1)) * scale
            if cross_mask is not None:  # [B, 1, 1, T_enc] True = attend
                cw = cw.masked_fill(~cross_mask, NEG)
            co = torch.matmul(torch.softmax(cw, dim=-1), cross[1]).transpose(1, 2).reshape(b, s, -1)
            x = x + F.linear(co, P("cross_attn_out.weight"))
        n = "norm3" if cross is not None else "norm2"
        hm = _ln(x, P(f"{n}.weight"), P(f"{n}.bias"))
        m = F.linear(F.gelu(F.linear(hm, P("mlp.0.weight"), P("mlp.0.bias"))), P("mlp.2.weight"), P("mlp.2.bias"))
        return x + m, (k, v)

    def decode_step(self, ids: torch.Tensor, past: Optional[Sequence[Tuple[torch.Tensor, torch.Tensor]]],
                    cross: Optional[Sequence[Tuple[torch.Tensor, torch.Tensor]]], self_mask=None, cross_mask=None):
        """ids [B, S] -> logits [B, S, V] and the per-layer (K, V) past + new."""
        x = self.p["decoder_embed.weight"][ids]
        new = []
        for i in range(self.n):
            x, kv = self.layer(i, x, past[i] if past is not None else None,
                               cross[i] if cross is not None and i < len(cross) else None, self_mask, cross_mask)
            new.append(kv)
        x = _ln(x, self.p[f"{self.norm}.weight"], self.p[f"{self.norm}.bias"])
        return F.linear(x, self.p["lm_head.weight"]), new


class EagerDecode:
    """The reference scheduler's eager decode loop for a batch of requests (all admitted at once, EOS
    disabled), with the decoder pool it writes every step. cross: per request, per layer (K, V)
    [1, H, T_r, D] float32; or, with batched=True, per layer (K, V) [B, H, T, D] of equal lengths."""

    def __init__(self, dec: Decoder, cross, block_size: int = 16, batched: bool = False):
        self.dec, self.bs = dec, block_size
        self.cross_mask = None
        if batched:
            self.cross = list(cross)
            self.lens = [cross[0][0].shape[2]] * cross[0][0].shape[0]
            return
        b = len(cross)
        t = [c[0][0].shape[2] for c in cross]
        self.lens = t
        layers = len(cross[0])
        if min(t) == max(t):
            self.cross = [(torch.cat([c[l][0] for c in cross]), torch.cat([c[l][1] for c in cross]))
                          for l in range(layers)]
        else:
            self.cross = []
            for l in range(layers):
                k = torch.zeros(b, dec.h, max(t), dec.d)
                v = torch.zeros_like(k)
                for i, c in enumerate(cross):
                    k[i, :, :t[i]] = c[l][0][0]
                    v[i, :, :t[i]] = c[l][1][0]
                self.cross.append((k, v))
            self.cross_mask = (torch.arange(max(t))[None] < torch.tensor(t)[:, None])[:, None, None, :]

    def run(self, prompt: Sequence[int], new_tokens: int, budget_s: Optional[float] = None):
        """Prefill, then up to new_tokens - 1 decode steps (fewer once budget_s seconds of decode steps
        have run). Returns (tokens per request, decode steps, seconds spent in decode steps)."""
        b, dec, bs = len(self.lens), self.dec, self.bs
        p = len(prompt)
        per = -(-(p + new_tokens) // bs)
        pools = [(torch.zeros(b * per, bs, dec.h, dec.d), torch.zeros(b * per, bs, dec.h, dec.d))
                 for _ in range(dec.n)]
        tables = torch.arange(b * per).view(b, per)
        logits, past = dec.decode_step(torch.tensor([list(prompt)] * b), None, self.cross, cross_mask=self.cross_mask)
        for l, (k, v) in enumerate(past):  # prefill write, phase_aware_scheduler.py:678-690
            for pos in range(p):
                pools[l][0][tables[:, pos // bs], pos % bs] = k[:, :, pos]
                pools[l][1][tables[:, pos // bs], pos % bs] = v[:, :, pos]
        toks = [[t] for t in logits[:, -1].argmax(-1).tolist()]
        steps, busy = 0, 0.0
        for step in range(1, new_tokens):
            if budget_s is not None and busy >= budget_s:
                break
            t0 = time.perf_counter()
            pos = p + step - 1
            ids = torch.tensor([[r[-1]] for r in toks])
            logits, past = dec.decode_step(ids, past, self.cross, cross_mask=self.cross_mask)
            for l, (k, v) in enumerate(past):  # the pool write of the new token, :1001-1010
                pools[l][0][tables[:, pos // bs], pos % bs] = k[:, :, pos]
                pools[l][1][tables[:, pos // bs], pos % bs] = v[:, :, pos]
            for r, t in zip(toks, logits[:, -1].argmax(-1).tolist()):
                r.append(t)
            steps += 1
            busy += time.perf_counter() - t0
        return toks, steps, busy


def paged_attention_step(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor, tables: torch.Tensor,
                         ctx: Sequence[int], k_new: torch.Tensor, v_new: torch.Tensor, scale: float) -> torch.Tensor:
    """One layer of the eager decode step: append the B new rows at position ctx_b - 1 through the block
    table, gather each request's ctx_b keys into a zero-padded [B, H, T, D] batch with a padding mask,
    softmax attention. q, k_new, v_new [B, H, D]; pools [NB, BS, H, D]; tables [B, max_blocks]."""
    b, h, d = q.shape
    bs = k_pool.shape[1]
    c = torch.as_tensor(list(ctx))
    pos = c - 1
    rows = tables[torch.arange(b), pos // bs]
    k_pool[rows, pos % bs] = k_new
    v_pool[rows, pos % bs] = v_new
    t = int(c.max())
    nblk = -(-t // bs)
    kk = k_pool[tables[:, :nblk]].reshape(b, nblk * bs, h, d)[:, :t].transpose(1, 2)
    vv = v_pool[tables[:, :nblk]].reshape(b, nblk * bs, h, d)[:, :t].transpose(1, 2)
    keep = torch.arange(t)[None] < c[:, None]
    w = torch.matmul(q[:, :, None], kk.transpose(-2, -1)) * scale
    w = w.masked_fill(~keep[:, None, None, :], NEG)
    return torch.matmul(torch.softmax(w, dim=-1), vv)[:, :, 0]


class TTSModel:
    """StreamingMultiCodebookTTSModel of a reference state dict, float32 on the CPU."""

    def __init__(self, state: Dict[str, torch.Tensor], num_heads: int, head_dim: int):
        self.core = Decoder(state, num_heads, head_dim, prefix="layers", norm="norm")
        self.p = self.core.p
        self.k = len({k.split(".")[2] for k in state if k.startswith("embeddings.embeddings.")})

    def forward(self, codes: torch.Tensor, past=None):
        """codes [B, S, K] -> logits [B, S, K, V], per-layer (K, V)."""
        x = self.p["embeddings.embeddings.0.weight"][codes[..., 0]]
        for i in range(1, self.k):
            x = x + self.p[f"embeddings.embeddings.{i}.weight"][codes[..., i]]
        new = []
        for i in range(self.core.n):
            x, kv = self.core.layer(i, x, past[i] if past is not None else None, None)
            new.append(kv)
        x = _ln(x, self.p["norm.weight"], self.p["norm.bias"])
        return torch.stack([F.linear(x, self.p[f"heads.heads.{i}.weight"]) for i in range(self.k)], dim=2), new


def tts_step(model: TTSModel, pools: Sequence[Tuple[torch.Tensor, torch.Tensor]], table: Sequence[int], seq_len: int,
             frame: torch.Tensor) -> torch.Tensor:
    """One request's decode step of the reference TTS engine: gather its seq_len past positions from the
    pools through its block table, forward one frame [1, 1, K], write the new K/V at position seq_len,
    return the next frame [K] (argmax per codebook)."""
    bs = pools[0][0].shape[1]
    h, d = pools[0][0].shape[2], pools[0][0].shape[3]
    past = []
    for kp, vp in pools:
        k = kp[list(table)].view(-1, h, d)[:seq_len].permute(1, 0, 2).contiguous().unsqueeze(0)
        v = vp[list(table)].view(-1, h, d)[:seq_len].permute(1, 0, 2).contiguous().unsqueeze(0)
        past.append((k, v))
    logits, new = model.forward(frame, past)
    blk, off = table[seq_len // bs], seq_len % bs
    for (kp, vp), (k, v) in zip(pools, new):
        kp[blk, off] = k[0, :, -1]
        vp[blk, off] = v[0, :, -1]
    return logits[0, -1].argmax(-1)
