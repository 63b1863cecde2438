"""Whisper-class encoder-decoder model whose attention runs on the gfx950 kernels.

Same module structure and parameter names as the reference's
WhisperClassSpeechEncoderDecoderModel / DecoderLayer
(speech_serving/models.py:79-208, 298-487), so a reference state_dict loads
unchanged:
    DecoderLayer: self_attn_{q,k,v,out}, cross_attn_{q,k,v,out} (bias-free),
                  norm1/norm2/norm3 (LayerNorm), mlp = Linear-GELU-Linear.
    Model:        conv1, conv2, encoder_layers, encoder_norm, decoder_embed,
                  decoder_layers, decoder_norm, lm_head.
Semantics kept from the reference: pre-LN residual blocks; self-attention
scale head_dim^-1/2; causal mask for multi-token decoder inputs; cross-
attention only for layers that receive encoder K/V or hidden states, and
then the MLP normalises with norm3 (else norm2); no positional embedding.

Entry points:
    encode(mel) -> (hidden, [(K, V)] per encoder layer)        models.py:349-367
    decode_step(...)  the reference signature                   models.py:369-423
        With a PagedKVCache as past_key_values it runs the paged hot path (the
        scheduler's eager prefill and decode call it so); any other cache (a
        DynamicCache-like object with .layers, a list of (K, V), None) is
        contiguous past K/V, as in the reference.
    decode_step_graph_fixed(...) bucketed static KV signature   models.py:425-487
    decode_step_paged(ids, PagedKV, CrossKV)  the paged step itself: per layer
        one fused launch appends the new K/V through the block table and
        attends, and one launch attends the rows' contiguous encoder K/V (the
        captured graph decode step calls it directly).
    project_cross_kv(hidden) -> [(K, V)] per decoder layer via cross_attn_k/v.
Every attention, append and greedy step is a HIP kernel (speech_serving.native);
tensors must live on the GPU.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, List, Optional, Sequence, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import native


# ---------------------------------------------------------------------------
# KV containers.
# ---------------------------------------------------------------------------
class LayerKV:
    """One layer's contiguous self-attention K/V ([B, H, T, D]), shaped like the
    cache layers the reference returns (`.keys`, `.values`)."""

    def __init__(self, keys: torch.Tensor, values: torch.Tensor):
        self.keys = keys
        self.values = values
        self.is_initialized = True


class KVCache:
    """List of LayerKV, exposed as `.layers` like the reference's DynamicCache."""

    def __init__(self, layers: Optional[List[LayerKV]] = None):
        self.layers: List[LayerKV] = layers or []

    def __len__(self) -> int:
        return len(self.layers)

    def to_legacy_cache(self):
        return tuple((l.keys, l.values) for l in self.layers)


class ModelOutput:
    def __init__(self, logits: torch.Tensor, past_key_values: Optional[KVCache]):
        self.logits = logits
        self.past_key_values = past_key_values


@dataclass
class PagedKV:
    """Self-attention K/V that lives in a BlockManager pool.

    block_tables: int32 [R, max_blocks]; row b uses table row table_rows[b]
    (or b). ctx_lens: int32 [B] = keys of row b including its new tokens.
    max_ctx bounds ctx_lens (launch grid size).
    """
    k_pools: Sequence[torch.Tensor]
    v_pools: Sequence[torch.Tensor]
    block_tables: torch.Tensor
    ctx_lens: torch.Tensor
    max_ctx: int
    table_rows: Optional[torch.Tensor] = None
    rows_longest_first: bool = False  # rows in non-increasing ctx_lens order (the launch need not rank them)


class _GatheredLayer:
    """One layer of a PagedKVCache as contiguous [B, H, max_ctx, D] K/V (zero past each row's length)."""

    def __init__(self, cache: "PagedKVCache", layer: int):
        self._cache, self._layer = cache, layer
        self._kv: Optional[Tuple[torch.Tensor, torch.Tensor]] = None
        self.is_initialized = True

    def _get(self) -> Tuple[torch.Tensor, torch.Tensor]:
        if self._kv is None:
            c = self._cache
            tables = c.block_tables if c.table_rows is None else c.block_tables.index_select(0, c.table_rows.long())
            self._kv = native.gather(c.k_pools[self._layer], c.v_pools[self._layer], tables,
                                     c.ctx_lens[: c.batch], c.max_ctx)
        return self._kv

    @property
    def keys(self) -> torch.Tensor:
        return self._get()[0]

    @property
    def values(self) -> torch.Tensor:
        return self._get()[1]


class PagedKVCache:
    """Self-attention K/V of a decode batch held in a BlockManager pool, passed to
    decode_step as `past_key_values` (where the reference passes a DynamicCache of
    contiguous K/V, phase_aware_scheduler.py:793-846 and :982-991).

    It describes the cache as it stands once the call's tokens are in: row b's block
    table (table row table_rows[b], or b) covers ctx_lens[b] keys, the last Q of which
    are the Q tokens of input_ids (positions ctx_lens[b]-Q .. ctx_lens[b]-1). decode_step
    appends their K/V through the tables inside the attention launch and returns this
    object as its output's past_key_values. `.layers[l].keys / .values` gather layer l
    into a zero-padded [B, H, max_ctx, D] batch (skv_gather) for code that reads a cache
    the way the reference reads its DynamicCache.

    cross_lens / cross_mask: the batch's encoder lengths (int32 [B] on the device) and the
    encoder_attention_mask built from them. decode_step takes the lengths as they are when
    it receives that same mask object, and derives them from any other mask.
    rows_longest_first: the caller knows ctx_lens to be non-increasing (the attention launch
    then skips ranking the rows by length; results are the same either way)."""

    def __init__(self, k_pools: Sequence[torch.Tensor], v_pools: Sequence[torch.Tensor], block_tables: torch.Tensor,
                 ctx_lens: torch.Tensor, max_ctx: int, table_rows: Optional[torch.Tensor] = None,
                 cross_lens: Optional[torch.Tensor] = None, cross_mask: Optional[torch.Tensor] = None,
                 rows_longest_first: bool = False):
        self.k_pools, self.v_pools = k_pools, v_pools
        self.rows_longest_first = bool(rows_longest_first)
        self.block_tables, self.ctx_lens, self.max_ctx = block_tables, ctx_lens, int(max_ctx)
        self.table_rows = table_rows
        self.cross_lens, self.cross_mask = cross_lens, cross_mask
        self.batch = int(ctx_lens.shape[0])
        self.layers = [_GatheredLayer(self, l) for l in range(len(k_pools))]

    def __len__(self) -> int:
        return len(self.layers)

    def paged(self) -> "PagedKV":
        return PagedKV(self.k_pools, self.v_pools, self.block_tables, self.ctx_lens, self.max_ctx, self.table_rows,
                       self.rows_longest_first)


@dataclass
class CrossKV:
    """Encoder K/V per decoder layer as [S, H, T, D] views (slot-major buffer);
    row b reads slot slot_ids[b] (or b) over its first lens[b] positions.
    Layers at or beyond len(k) get no cross-attention (models.py:398-406)."""
    k: Sequence[torch.Tensor]
    v: Sequence[torch.Tensor]
    lens: torch.Tensor
    max_len: int
    slot_ids: Optional[torch.Tensor] = None

    def has(self, layer: int) -> bool:
        return layer < len(self.k)


# ---------------------------------------------------------------------------
# Mask handling for the reference's contiguous API.
# ---------------------------------------------------------------------------
def _keep_mask(mask: torch.Tensor, batch: int, t: int) -> torch.Tensor:
    """Reference masks (models.py:142-157, 186-199) as a bool keep-mask [B, T].

    bool: True = attend. Binary 0/1 integers: 1 = attend. Additive floats:
    0 = attend, <= -1000 = masked (the reference uses -10000 and finfo.min);
    other additive values are a bias these kernels do not apply.
    """
    m = mask
    while m.dim() > 2:
        if m.shape[1] != 1:
            if not bool((m == m[:, :1]).all()):
                raise NotImplementedError("per-head / per-query attention masks are not supported")
            m = m[:, :1]
        m = m[:, 0]
    m = m.expand(batch, t) if m.shape[0] == 1 else m
    if m.dtype == torch.bool:
        return m
    if not m.is_floating_point() or bool(torch.isin(m, torch.tensor([0, 1], device=m.device)).all()):
        return m != 0
    keep = m == 0
    if not bool((keep | (m <= -1000)).all()):
        raise NotImplementedError("additive attention bias other than 0 / large-negative masking")
    return keep


def _compact(k: torch.Tensor, v: torch.Tensor, keep: torch.Tensor):
    """Move each row's kept positions to the front (order preserved); returns K, V, lens."""
    lens = keep.sum(dim=-1).to(torch.int32)
    if bool((keep == (torch.arange(keep.shape[1], device=keep.device)[None] < lens[:, None])).all()):
        return k, v, lens  # already a prefix mask
    order = torch.argsort((~keep).to(torch.int8), dim=-1, stable=True)
    idx = order[:, None, :, None].expand(k.shape[0], k.shape[1], k.shape[2], k.shape[3])
    return torch.gather(k, 2, idx).contiguous(), torch.gather(v, 2, idx).contiguous(), lens


def _bucket_mask_lens(mask: torch.Tensor, rows: int, width: int, what: str) -> torch.Tensor:
    """Per-row lengths of the additive masks of the bucketed graph step (graph_decode_buffers.py:520-537):
    0 over each row's first positions, -10000 beyond. A row masked everywhere is an idle slot; its
    uniform -10000 cancels in the reference's softmax, which then weighs every position, so its length
    is the full width. Outside graph capture the masks are checked: values 0 or <= -1000 only, and the
    kept positions of each row a prefix. Inside a capture nothing can be read back; the masks are the
    buffers' own, prefix masks by construction."""
    m = mask.reshape(rows, -1)
    if m.shape[1] != width:
        raise ValueError(f"{what}: mask covers {m.shape[1]} positions per slot, expected {width}")
    keep = m > -1000
    n = keep.sum(-1)
    if not torch.cuda.is_current_stream_capturing():
        if not bool(((m == 0) | (m <= -1000)).all()):
            raise NotImplementedError(f"{what}: additive bias other than 0 / large-negative masking")
        if bool((keep.to(torch.int32).cumprod(-1).sum(-1) != n).any()):
            raise ValueError(f"{what}: the kept positions of each slot must form a prefix")
    return torch.where(n == 0, torch.full_like(n, width), n).to(torch.int32)


def _hooked(mod: nn.Module) -> bool:
    """Whether calling the module would run forward hooks (its own or global ones)."""
    return bool(mod._forward_hooks or mod._forward_pre_hooks or nn.modules.module._global_forward_hooks or
                nn.modules.module._global_forward_pre_hooks)


def proj(mod: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """mod(x). A plain nn.Linear without hooks on a GPU tensor runs as one skv_linear call (a hipBLASLt plan
    cached per shape: the algorithm and bits of torch's linear without its per-call descriptor set-up and
    heuristic); any other module, or one with hooks, is called as usual."""
    if x.is_cuda and type(mod) is nn.Linear and not _hooked(mod):
        return native.linear(x, mod.weight, mod.bias)
    return mod(x)


def mlp(seq: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """seq(x) for the layers' Linear-GELU-Linear MLP, its projections through proj() (other modules and
    hooked ones are called as usual)."""
    if x.is_cuda and type(seq) is nn.Sequential and not _hooked(seq):
        parts = tuple(seq._modules.values())
        if len(parts) == 3 and type(parts[1]) is nn.GELU and not _hooked(parts[1]):
            return proj(parts[2], F.gelu(proj(parts[0], x), approximate=parts[1].approximate))
    return seq(x)


def add_norm(x: torch.Tensor, y: Optional[torch.Tensor], norm: nn.LayerNorm) -> Tuple[torch.Tensor, torch.Tensor]:
    """(s, norm(s)) for s = x + y (s = x when y is None): one skv_add_layernorm launch
    on the GPU, the same two torch ops elsewhere."""
    if x.is_cuda and norm.elementwise_affine and not _hooked(norm):
        bias = norm.bias
        if bias is not None:
            got = native.add_layernorm(x, y, norm.weight, bias, norm.eps, fallback=True)
            if got is not None:
                return got
    s = x if y is None else x + y
    return s, norm(s)


@torch.no_grad()
def _init_normal(model: nn.Module, std: float, seed: int, draw_device: Optional[str]):
    dev = torch.device(draw_device or "cpu")
    g = torch.Generator(device=dev).manual_seed(seed)
    for m in model.modules():
        if isinstance(m, (nn.Linear, nn.Conv1d, nn.Embedding)):
            w = torch.empty(m.weight.shape, dtype=torch.float32, device=dev).normal_(0.0, std, generator=g)
            m.weight.copy_(w.to(m.weight.dtype))
            if getattr(m, "bias", None) is not None:
                m.bias.zero_()
        elif isinstance(m, nn.LayerNorm):
            m.weight.fill_(1.0)
            m.bias.zero_()
    return model


# ---------------------------------------------------------------------------
# Layers.
# ---------------------------------------------------------------------------
class DecoderLayer(nn.Module):
    """Pre-LN transformer layer with self-attention, optional cross-attention and a GELU MLP."""

    def __init__(self, hidden_dim: int, num_heads: int, head_dim: int, is_decoder: bool = True):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.is_decoder = is_decoder
        hd = num_heads * head_dim
        self.self_attn_q = nn.Linear(hidden_dim, hd, bias=False)
        self.self_attn_k = nn.Linear(hidden_dim, hd, bias=False)
        self.self_attn_v = nn.Linear(hidden_dim, hd, bias=False)
        self.self_attn_out = nn.Linear(hd, hidden_dim, bias=False)
        self.cross_attn_q = nn.Linear(hidden_dim, hd, bias=False)
        self.cross_attn_k = nn.Linear(hidden_dim, hd, bias=False)
        self.cross_attn_v = nn.Linear(hidden_dim, hd, bias=False)
        self.cross_attn_out = nn.Linear(hd, hidden_dim, bias=False)
        self.norm1 = nn.LayerNorm(hidden_dim)
        self.norm2 = nn.LayerNorm(hidden_dim)
        self.norm3 = nn.LayerNorm(hidden_dim)
        self.mlp = nn.Sequential(nn.Linear(hidden_dim, hidden_dim * 4), nn.GELU(),
                                 nn.Linear(hidden_dim * 4, hidden_dim))
        self._qkv_key = None
        self._qkv_w: Optional[torch.Tensor] = None

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.head_dim)

    def qkv_weight(self) -> torch.Tensor:
        """[3*H*D, hidden] concatenation of the q/k/v weights, rebuilt when any of them changes."""
        ws = (self.self_attn_q.weight, self.self_attn_k.weight, self.self_attn_v.weight)
        key = tuple((w.data_ptr(), w._version, w.dtype) for w in ws)
        if key != self._qkv_key:
            if ws[0].is_cuda and torch.cuda.is_current_stream_capturing():
                raise RuntimeError("fused q/k/v weight must be built before graph capture (run one eager step)")
            self._qkv_w = torch.cat([w.detach() for w in ws], dim=0).contiguous()
            self._qkv_key = key
        return self._qkv_w

    def _qkv(self, x: torch.Tensor):
        return self._qkv_normed(self.norm1(x))

    def _qkv_normed(self, h: torch.Tensor):
        """q, k, v [B, S, H, D] from the already normalised input h."""
        b, s, _ = h.shape
        hd = self.num_heads * self.head_dim
        qkv = native.linear(h, self.qkv_weight()) if h.is_cuda else F.linear(h, self.qkv_weight())
        shape = (b, s, self.num_heads, self.head_dim)
        return qkv[..., :hd].view(shape), qkv[..., hd:2 * hd].view(shape), qkv[..., 2 * hd:].view(shape)

    def _finish(self, x: torch.Tensor, cross_used: bool) -> torch.Tensor:
        norm = self.norm3 if cross_used else self.norm2
        return x + mlp(self.mlp, norm(x))

    def _cross_q(self, x: torch.Tensor) -> torch.Tensor:
        b, s, _ = x.shape
        return proj(self.cross_attn_q, self.norm2(x)).view(b, s, self.num_heads, self.head_dim)

    # -- paged hot path ---------------------------------------------------------
    def forward_paged(self, x: torch.Tensor, layer: int, kv: PagedKV, cross: Optional[CrossKV],
                      pending: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        """One decoder layer over the paged cache. The residual stream is x + pending
        (pending: the previous layer's MLP output, not yet added). Returns (x, mlp
        output) with the MLP output left for the next layer (or the final norm) to
        add, so every residual add shares a launch with the LayerNorm that follows it."""
        b, s, _ = x.shape
        hd = self.num_heads * self.head_dim
        x, h = add_norm(x, pending, self.norm1)
        q, k, v = self._qkv_normed(h)
        attn = native.paged_attention(q, kv.k_pools[layer], kv.v_pools[layer], kv.block_tables, kv.ctx_lens,
                                      kv.max_ctx, self.scale, causal=s > 1, table_rows=kv.table_rows,
                                      k_new=k, v_new=v, rows_longest_first=kv.rows_longest_first)
        a = proj(self.self_attn_out, attn.view(b, s, hd))
        used = cross is not None and cross.has(layer)
        if used:
            x, h = add_norm(x, a, self.norm2)
            cq = proj(self.cross_attn_q, h).view(b, s, self.num_heads, self.head_dim)
            c = native.dense_attention(cq, cross.k[layer], cross.v[layer], cross.lens,
                                       cross.max_len, self.scale, slot_ids=cross.slot_ids)
            x, h = add_norm(x, proj(self.cross_attn_out, c.view(b, s, hd)), self.norm3)
        else:
            x, h = add_norm(x, a, self.norm2)
        return x, mlp(self.mlp, h)

    # -- contiguous API of the reference (models.py:110-208) ---------------------
    def forward(self, x: torch.Tensor, past_key_values: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                encoder_hidden_states: Optional[torch.Tensor] = None,
                encoder_past_kv: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                attention_mask: Optional[torch.Tensor] = None,
                encoder_attention_mask: Optional[torch.Tensor] = None):
        b, s, _ = x.shape
        hd = self.num_heads * self.head_dim
        q, k, v = self._qkv(x)
        k = k.transpose(1, 2)
        v = v.transpose(1, 2)
        if past_key_values is not None:
            pk, pv = past_key_values
            k = torch.cat([pk.to(q.dtype), k], dim=2)
            v = torch.cat([pv.to(q.dtype), v], dim=2)
        else:
            k, v = k.contiguous(), v.contiguous()
        new_past = (k, v)
        t = k.shape[2]
        if attention_mask is not None:
            kk, vv, lens = _compact(k, v, _keep_mask(attention_mask, b, t))
        else:
            kk, vv = k, v
            lens = torch.full((b,), t, dtype=torch.int32, device=x.device)
        attn = native.dense_attention(q, kk, vv, lens, t, self.scale, causal=self.is_decoder and s > 1)
        x = x + proj(self.self_attn_out, attn.reshape(b, s, hd))

        new_cross = None
        used = encoder_hidden_states is not None or encoder_past_kv is not None
        if used:
            if encoder_past_kv is not None:
                ck, cv = encoder_past_kv
                ck, cv = ck.to(q.dtype), cv.to(q.dtype)
            else:
                enc = encoder_hidden_states
                te = enc.shape[1]
                ck = self.cross_attn_k(enc).view(b, te, self.num_heads, self.head_dim).transpose(1, 2)
                cv = self.cross_attn_v(enc).view(b, te, self.num_heads, self.head_dim).transpose(1, 2)
            new_cross = (ck, cv)
            if ck.stride(3) != 1 or ck.stride() != cv.stride():
                ck, cv = ck.contiguous(), cv.contiguous()
            te = ck.shape[2]
            if encoder_attention_mask is not None:
                ck, cv, clens = _compact(ck, cv, _keep_mask(encoder_attention_mask, b, te))
            else:
                clens = torch.full((b,), te, dtype=torch.int32, device=x.device)
            if ck.shape[0] == 1 and b > 1:
                ck, cv = ck.expand(b, -1, -1, -1), cv.expand(b, -1, -1, -1)
            c = native.dense_attention(self._cross_q(x), ck, cv, clens, te, self.scale)
            x = x + proj(self.cross_attn_out, c.reshape(b, s, hd))
        return self._finish(x, used), new_past, new_cross


# ---------------------------------------------------------------------------
# Model.
# ---------------------------------------------------------------------------
class WhisperClassSpeechEncoderDecoderModel(nn.Module):
    """Conv front-end + encoder layers + causal decoder with cross-attention."""

    def __init__(self, num_encoder_layers: int = 4, num_decoder_layers: int = 4, num_heads: int = 4,
                 hidden_dim: int = 256, mel_dim: int = 80, vocab_size: int = 51200,
                 head_dim: Optional[int] = None):
        super().__init__()
        self.num_encoder_layers = num_encoder_layers
        self.num_decoder_layers = num_decoder_layers
        self.num_heads = num_heads
        self.head_dim = head_dim if head_dim is not None else hidden_dim // num_heads
        self.hidden_dim = hidden_dim
        self.vocab_size = vocab_size

        class Config:
            pass

        self.config = Config()
        self.config.num_hidden_layers = num_decoder_layers
        self.config.num_attention_heads = num_heads
        self.config.num_key_value_heads = num_heads
        self.config.hidden_size = hidden_dim
        self.config.vocab_size = vocab_size
        self.config.encoder_num_layers = num_encoder_layers

        self.conv1 = nn.Conv1d(mel_dim, hidden_dim, kernel_size=3, padding=1)
        self.conv2 = nn.Conv1d(hidden_dim, hidden_dim, kernel_size=3, stride=2, padding=1)
        self.encoder_layers = nn.ModuleList(
            [DecoderLayer(hidden_dim, num_heads, self.head_dim, is_decoder=False) for _ in range(num_encoder_layers)])
        self.encoder_norm = nn.LayerNorm(hidden_dim)
        self.decoder_embed = nn.Embedding(vocab_size, hidden_dim)
        self.decoder_layers = nn.ModuleList(
            [DecoderLayer(hidden_dim, num_heads, self.head_dim, is_decoder=True) for _ in range(num_decoder_layers)])
        self.decoder_norm = nn.LayerNorm(hidden_dim)
        self.lm_head = nn.Linear(hidden_dim, vocab_size, bias=False)

    # -- initialisation used by the benchmark configs ------------------------------
    def init_normal_(self, std: float = 0.02, seed: int = 0,
                     draw_device: Optional[str] = None) -> "WhisperClassSpeechEncoderDecoderModel":
        """Weights of every Linear / Conv1d / Embedding ~ N(0, std), biases 0,
        LayerNorm 1 / 0. Draws are seeded on `draw_device` (default CPU, so every
        device gets the same values; a GPU draw is much faster for large models)."""
        return _init_normal(self, std, seed, draw_device)

    @property
    def dtype(self) -> torch.dtype:
        return self.decoder_norm.weight.dtype

    def _embed(self, ids: torch.Tensor) -> torch.Tensor:
        return self.decoder_embed(ids).to(dtype=self.decoder_norm.weight.dtype)

    # -- encoder (models.py:349-367) ---------------------------------------------------
    def encode(self, mel_features: torch.Tensor):
        x = F.gelu(self.conv1(mel_features))
        x = F.gelu(self.conv2(x)).transpose(1, 2)
        kv = []
        for layer in self.encoder_layers:
            x, (k, v), _ = layer(x)
            kv.append((k, v))
        return self.encoder_norm(x), kv

    def project_cross_kv(self, encoder_hidden_states: torch.Tensor) -> List[Tuple[torch.Tensor, torch.Tensor]]:
        """Per decoder layer (K, V) [B, H, T, D] = cross_attn_k/v(encoder states) (models.py:179-181)."""
        b, t, _ = encoder_hidden_states.shape
        out = []
        for layer in self.decoder_layers:
            k = layer.cross_attn_k(encoder_hidden_states).view(b, t, self.num_heads, self.head_dim)
            v = layer.cross_attn_v(encoder_hidden_states).view(b, t, self.num_heads, self.head_dim)
            out.append((k.transpose(1, 2).contiguous(), v.transpose(1, 2).contiguous()))
        return out

    # -- paged decode (the hot path) -------------------------------------------------
    def decode_step_paged(self, input_ids: torch.Tensor, kv: PagedKV, cross: Optional[CrossKV] = None,
                          last_only: bool = True) -> torch.Tensor:
        """Run the decoder on input_ids [B, Q] whose K/V go into the paged pool at
        positions ctx_lens-Q .. ctx_lens-1; returns logits [B, V] of the last
        position (or [B, Q, V])."""
        x = self._embed(input_ids)
        pending = None
        for l, layer in enumerate(self.decoder_layers):
            x, pending = layer.forward_paged(x, l, kv, cross, pending)
        if last_only:
            x = x[:, -1]
            pending = None if pending is None else pending[:, -1]
        _, h = add_norm(x, pending, self.decoder_norm)
        return proj(self.lm_head, h)

    # -- decode step, reference signature (models.py:369-423) ----------------------------
    def decode_step(self, input_ids: torch.Tensor, past_key_values: Optional[Any] = None,
                    encoder_past_kv_list: Optional[List[Tuple[torch.Tensor, torch.Tensor]]] = None,
                    encoder_hidden_states: Optional[torch.Tensor] = None,
                    attention_mask: Optional[torch.Tensor] = None,
                    encoder_attention_mask: Optional[torch.Tensor] = None,
                    position_ids: Optional[torch.Tensor] = None, use_cache: bool = True, **kwargs) -> ModelOutput:
        """Logits [B, S, V] of input_ids [B, S] and the updated cache.

        past_key_values: a PagedKVCache (the paged hot path), or contiguous past K/V as in the
        reference (an object with .layers[l].keys/.values, a list of (K, V) [B, H, T, D], or None).
        encoder_past_kv_list: per decoder layer (K, V) [B or 1, H, T_enc, D], row b of the batch
        attending row b; layers past the list's end use encoder_hidden_states (projected) or no
        cross-attention. Masks as in the reference (models.py:142-157, 186-199).
        logits_to_keep (keyword): when > 0, logits of the last logits_to_keep positions only."""
        if isinstance(past_key_values, PagedKVCache):
            return self._decode_step_paged_cache(input_ids, past_key_values, encoder_past_kv_list,
                                                 encoder_hidden_states, attention_mask, encoder_attention_mask,
                                                 int(kwargs.get("logits_to_keep", 0) or 0))
        x = self._embed(input_ids)
        cache = KVCache() if use_cache else None
        for i, layer in enumerate(self.decoder_layers):
            past = None
            if past_key_values is not None:
                if hasattr(past_key_values, "layers"):
                    if i < len(past_key_values.layers):
                        past = (past_key_values.layers[i].keys, past_key_values.layers[i].values)
                elif isinstance(past_key_values, (list, tuple)) and i < len(past_key_values):
                    past = past_key_values[i]
            enc_kv = encoder_past_kv_list[i] if encoder_past_kv_list is not None and i < len(
                encoder_past_kv_list) else None
            x, new_kv, _ = layer(x, past_key_values=past,
                                 encoder_hidden_states=encoder_hidden_states if enc_kv is None else None,
                                 encoder_past_kv=enc_kv, attention_mask=attention_mask,
                                 encoder_attention_mask=encoder_attention_mask)
            if use_cache:
                cache.layers.append(LayerKV(new_kv[0], new_kv[1]))
        keep = int(kwargs.get("logits_to_keep", 0) or 0)
        if keep > 0:
            x = x[:, -keep:]
        return ModelOutput(proj(self.lm_head, self.decoder_norm(x)), cache)

    def _decode_step_paged_cache(self, input_ids: torch.Tensor, cache: PagedKVCache,
                                 encoder_past_kv_list: Optional[List[Tuple[torch.Tensor, torch.Tensor]]],
                                 encoder_hidden_states: Optional[torch.Tensor],
                                 attention_mask: Optional[torch.Tensor],
                                 encoder_attention_mask: Optional[torch.Tensor], keep: int) -> ModelOutput:
        b = input_ids.shape[0]
        if attention_mask is not None:
            raise ValueError("decode_step: a PagedKVCache carries each row's length; attention_mask must be None")
        if cache.batch < b:
            raise ValueError(f"decode_step: the PagedKVCache holds {cache.batch} rows for a batch of {b}")
        cross = self._cross_kv(b, encoder_past_kv_list, encoder_hidden_states, encoder_attention_mask, cache)
        if keep == 1:
            logits = self.decode_step_paged(input_ids, cache.paged(), cross, last_only=True).unsqueeze(1)
        else:
            logits = self.decode_step_paged(input_ids, cache.paged(), cross, last_only=False)
            if keep > 1:
                logits = logits[:, -keep:]
        return ModelOutput(logits, cache)

    def _cross_kv(self, b: int, enc_list: Optional[List[Tuple[torch.Tensor, torch.Tensor]]],
                  enc_hidden: Optional[torch.Tensor], enc_mask: Optional[torch.Tensor],
                  cache: PagedKVCache) -> Optional[CrossKV]:
        """The decode_step's encoder inputs as per-layer [B, H, T, D] K/V and per-row lengths: the given
        (K, V) per layer, then (for the layers past the list) K/V projected from encoder_hidden_states
        (models.py:179-181, 398-406)."""
        n = self.num_decoder_layers
        ks: List[torch.Tensor] = []
        vs: List[torch.Tensor] = []
        dt = self.dtype
        for k, v in (enc_list or [])[:n]:
            if k.dim() != 4 or k.shape[1] != self.num_heads or k.shape[3] != self.head_dim or \
                    k.shape[0] not in (1, b) or v.shape != k.shape:
                raise ValueError(f"decode_step: encoder K/V must be [{b} or 1, {self.num_heads}, T, "
                                 f"{self.head_dim}], got {tuple(k.shape)} / {tuple(v.shape)}")
            k, v = k.to(dt), v.to(dt)
            if k.stride(3) != 1 or k.stride() != v.stride():
                k, v = k.contiguous(), v.contiguous()
            if k.shape[0] == 1 and b > 1:
                k, v = k.expand(b, -1, -1, -1), v.expand(b, -1, -1, -1)
            ks.append(k)
            vs.append(v)
        if enc_hidden is not None and len(ks) < n:
            h = enc_hidden.to(dt)
            te = h.shape[1]
            for layer in self.decoder_layers[len(ks):]:
                ks.append(layer.cross_attn_k(h).view(h.shape[0], te, self.num_heads, self.head_dim)
                          .transpose(1, 2).contiguous().expand(b, -1, -1, -1))
                vs.append(layer.cross_attn_v(h).view(h.shape[0], te, self.num_heads, self.head_dim)
                          .transpose(1, 2).contiguous().expand(b, -1, -1, -1))
        if not ks:
            return None
        t = ks[0].shape[2]
        if any(k.shape[2] != t for k in ks):
            raise ValueError("decode_step: every layer's encoder K/V must cover the same positions")
        if enc_mask is None:
            lens = torch.full((b,), t, dtype=torch.int32, device=ks[0].device)
        elif enc_mask is cache.cross_mask and cache.cross_lens is not None:
            lens = cache.cross_lens[:b]
        else:
            keep = _keep_mask(enc_mask, b, t)
            for i in range(len(ks)):
                ks[i], vs[i], lens = _compact(ks[i], vs[i], keep)
        return CrossKV(ks, vs, lens, t)

    # -- bucketed static-KV decode, reference signature (models.py:425-487) -------------
    def decode_step_graph_fixed(self, g_token_ids: torch.Tensor, g_positions: torch.Tensor, g_self_kv: torch.Tensor,
                                g_cross_kv: torch.Tensor, g_output_tokens: torch.Tensor, bucket: int,
                                max_slots: int, g_attn_mask: Optional[torch.Tensor] = None,
                                g_cross_mask: Optional[torch.Tensor] = None) -> None:
        """One decode step over static per-slot buffers g_self_kv [S, L, 2, H, bucket, D]
        and g_cross_kv [S, L, 2, H, T, D]; masks are additive with -10000 beyond each
        slot's length (graph_decode_buffers.py:527-537), turned into lengths by
        _bucket_mask_lens (a slot masked everywhere attends over every position, as the
        reference's softmax does). Writes argmax tokens."""
        x = self._embed(g_token_ids)
        dev = x.device
        if g_attn_mask is not None:
            self_lens = _bucket_mask_lens(g_attn_mask, max_slots, bucket, "g_attn_mask")
        else:
            self_lens = torch.full((max_slots,), bucket, dtype=torch.int32, device=dev)
        t_enc = g_cross_kv.shape[4]
        if g_cross_mask is not None:
            cross_lens = _bucket_mask_lens(g_cross_mask, max_slots, t_enc, "g_cross_mask")
        else:
            cross_lens = torch.full((max_slots,), t_enc, dtype=torch.int32, device=dev)
        pos = g_positions.view(max_slots).clamp(0, bucket - 1)
        hd = self.num_heads * self.head_dim
        for l, layer in enumerate(self.decoder_layers):
            q, k, v = layer._qkv(x)
            idx = pos.view(max_slots, 1, 1, 1).expand(max_slots, layer.num_heads, 1, layer.head_dim)
            g_self_kv[:, l, 0].scatter_(2, idx, k.transpose(1, 2))
            g_self_kv[:, l, 1].scatter_(2, idx, v.transpose(1, 2))
            a = native.dense_attention(q, g_self_kv[:, l, 0], g_self_kv[:, l, 1], self_lens, bucket, layer.scale)
            x = x + layer.self_attn_out(a.view(max_slots, 1, hd))
            c = native.dense_attention(layer._cross_q(x), g_cross_kv[:, l, 0], g_cross_kv[:, l, 1], cross_lens,
                                       t_enc, layer.scale)
            x = x + layer.cross_attn_out(c.view(max_slots, 1, hd))
            x = layer._finish(x, True)
        logits = proj(self.lm_head, self.decoder_norm(x[:, -1, :]))
        native.argmax(logits, out=g_output_tokens)


# ---------------------------------------------------------------------------
# Streaming multi-codebook TTS model (decoder-only, paged self-attention).
# ---------------------------------------------------------------------------
class MultiCodebookEmbedding(nn.Module):
    """Sum of K per-codebook embeddings (reference models.py:23-51, same parameter names)."""

    def __init__(self, num_codebooks: int, vocab_size: int, embed_dim: int):
        super().__init__()
        self.num_codebooks = num_codebooks
        self.vocab_size = vocab_size
        self.embed_dim = embed_dim
        self.embeddings = nn.ModuleList([nn.Embedding(vocab_size, embed_dim) for _ in range(num_codebooks)])

    def forward(self, input_codebooks: torch.Tensor) -> torch.Tensor:
        """[B, S, K] codes -> [B, S, embed_dim]: the K gathers and K - 1 adds of the reference in one
        launch, with the reference's left-to-right rounding."""
        if input_codebooks.shape[-1] != self.num_codebooks:
            raise ValueError(f"Expected {self.num_codebooks} codebooks, got {input_codebooks.shape[-1]}")
        return native.codebook_embed_sum(input_codebooks, [e.weight for e in self.embeddings])


class MultiCodebookHeads(nn.Module):
    """One bias-free linear head per codebook (reference models.py:54-77, same parameter
    names), computed as one GEMM over the concatenated head weights."""

    def __init__(self, num_codebooks: int, hidden_dim: int, vocab_size: int):
        super().__init__()
        self.num_codebooks = num_codebooks
        self.vocab_size = vocab_size
        self.heads = nn.ModuleList([nn.Linear(hidden_dim, vocab_size, bias=False) for _ in range(num_codebooks)])
        self._key = None
        self._w: Optional[torch.Tensor] = None

    def fused_weight(self) -> torch.Tensor:
        """[K * V, hidden], rebuilt when any head weight changes."""
        ws = tuple(h.weight for h in self.heads)
        key = tuple((w.data_ptr(), w._version, w.dtype) for w in ws)
        if key != self._key:
            self._w = torch.cat([w.detach() for w in ws], dim=0).contiguous()
            self._key = key
        return self._w

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        """[B, S, hidden] -> logits [B, S, K, V]."""
        b, s, _ = hidden_states.shape
        w = self.fused_weight()
        y = native.linear(hidden_states, w) if hidden_states.is_cuda else F.linear(hidden_states, w)
        return y.view(b, s, self.num_codebooks, self.vocab_size)


class StreamingMultiCodebookTTSModel(nn.Module):
    """Decoder-only model over K parallel codebook streams (reference models.py:211-295):
    summed codebook embeddings, DecoderLayer stack (self-attention only, so each MLP
    normalises with norm2), final LayerNorm, one head per codebook.

    Entry points:
        forward(input_codebooks, past_key_values, use_cache)  the reference signature,
            contiguous past K/V ([B, H, T, D] per layer) -> logits [B, S, K, V] + cache
        decode_step_paged(input_codebooks, PagedKV)  the paged hot path: per layer one
            fused launch appends the new frames' K/V through the block table and attends
    """

    def __init__(self, num_layers: int = 4, num_heads: int = 4, hidden_dim: int = 256, num_codebooks: int = 4,
                 vocab_size: int = 1024):
        super().__init__()
        self.num_layers = num_layers
        self.num_heads = num_heads
        self.head_dim = hidden_dim // num_heads
        self.hidden_dim = hidden_dim
        self.num_codebooks = num_codebooks
        self.vocab_size = vocab_size

        class Config:
            pass

        self.config = Config()
        self.config.num_hidden_layers = num_layers
        self.config.num_attention_heads = num_heads
        self.config.num_key_value_heads = num_heads
        self.config.hidden_size = hidden_dim
        self.config.vocab_size = vocab_size

        self.embeddings = MultiCodebookEmbedding(num_codebooks, vocab_size, hidden_dim)
        self.layers = nn.ModuleList(
            [DecoderLayer(hidden_dim, num_heads, self.head_dim, is_decoder=True) for _ in range(num_layers)])
        self.norm = nn.LayerNorm(hidden_dim)
        self.heads = MultiCodebookHeads(num_codebooks, hidden_dim, vocab_size)

    def init_normal_(self, std: float = 0.02, seed: int = 0,
                     draw_device: Optional[str] = None) -> "StreamingMultiCodebookTTSModel":
        """Weights of every Linear / Embedding ~ N(0, std), LayerNorm 1 / 0 (seeded)."""
        return _init_normal(self, std, seed, draw_device)

    @property
    def dtype(self) -> torch.dtype:
        return self.norm.weight.dtype

    def forward(self, input_codebooks: torch.Tensor, past_key_values: Optional[Any] = None,
                use_cache: bool = True, logits_to_keep: int = 0) -> ModelOutput:
        """Logits [B, S, K, V] of input_codebooks [B, S, K] and the updated cache. With a PagedKVCache as
        past_key_values this is the paged step (the frames' K/V go into the pool through the block
        tables); otherwise past K/V are contiguous, as in the reference. logits_to_keep > 0 keeps the
        logits of the last logits_to_keep frames only."""
        if isinstance(past_key_values, PagedKVCache):
            if logits_to_keep == 1:
                logits = self.decode_step_paged(input_codebooks, past_key_values.paged(), last_only=True)
                return ModelOutput(logits.unsqueeze(1), past_key_values)
            logits = self.decode_step_paged(input_codebooks, past_key_values.paged(), last_only=False)
            return ModelOutput(logits[:, -logits_to_keep:] if logits_to_keep > 0 else logits, past_key_values)
        x = self.embeddings(input_codebooks)
        cache = KVCache() if use_cache else None
        for i, layer in enumerate(self.layers):
            past = None
            if past_key_values is not None:
                if hasattr(past_key_values, "layers"):
                    if i < len(past_key_values.layers):
                        past = (past_key_values.layers[i].keys, past_key_values.layers[i].values)
                elif isinstance(past_key_values, (list, tuple)) and i < len(past_key_values):
                    past = past_key_values[i]
            x, new_kv, _ = layer(x, past_key_values=past)
            if use_cache:
                cache.layers.append(LayerKV(new_kv[0], new_kv[1]))
        if logits_to_keep > 0:
            x = x[:, -logits_to_keep:]
        return ModelOutput(self.heads(self.norm(x)), cache)

    def decode_step_paged(self, input_codebooks: torch.Tensor, kv: PagedKV, last_only: bool = True) -> torch.Tensor:
        """Run the model on input_codebooks [B, Q, K] whose K/V go into the paged pool at
        positions ctx_lens-Q .. ctx_lens-1 (causal among the Q frames); returns the logits
        of the last frame [B, K, V] (or of every frame, [B, Q, K, V])."""
        x = self.embeddings(input_codebooks)
        pending = None
        for l, layer in enumerate(self.layers):
            x, pending = layer.forward_paged(x, l, kv, None, pending)
        if last_only:
            x = x[:, -1:]
            pending = None if pending is None else pending[:, -1:]
        _, h = add_norm(x, pending, self.norm)
        logits = self.heads(h)
        return logits[:, 0] if last_only else logits
