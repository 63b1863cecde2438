"""Reduced-precision error model of the synthetic Whisper-class decoder — TEST INFRASTRUCTURE ONLY.

The reference runs its decoder in fp16 / bf16 tensors: every op's output is rounded to the tensor
dtype (speech_serving/models.py:110-208 DecoderLayer.forward, :369-423 decode_step; the GEMMs, the
softmax and the LayerNorm compute internally in fp32). Two implementations that round at different
places (or accumulate in a different order) give logits that differ by a sum of rounding errors. This
module gives that difference a derived size, with no constant fitted to measurements:

- Decoder64 restates decode_step over a whole teacher-forced token sequence (one causal pass: the
  prompt and every later step's token, which is what prefill + cached decode steps compute row by row)
  in float64 torch, and records each *rounding site*: an op output the reference rounds to its dtype.
- A rounding of an exact value y to the dtype adds an error uniform in [-ulp(y)/2, ulp(y)/2]
  (variance ulp(y)^2 / 12). To first order, a logit z moves by sum_s g_s * delta_s with
  g_s = dz/dy_s (autograd through the float64 pass). Taking the errors as independent,
  var(z) = sum over sites and elements of g^2 ulp^2 / 12.
- rounding_sigma sums that variance over the sites of two placements: the reference's (every op
  output, incl. the attention scores and probabilities) and the paged path's (the fused attention
  kernel rounds only its output). Sites both implementations round count twice (their errors are
  taken as independent, which overstates the difference), so the sigma bounds the spread of
  z_paged - z_reference, and of either against float64 math.
- seeded_state / seeded_cross_kv regenerate the fixtures' weights and encoder K/V from seeds, by
  parameter name, so the reference run and the GPU run use identical inputs.

- MultiCodebook64 does the same for the streaming multi-codebook TTS model (models.py:23-77, 211-295):
  the K codebook embeddings summed left to right (each partial sum a site), the same layers without
  cross-attention, the final norm and K heads, with the K heads' logits laid out as one row.

Parity pins: Decoder64's float64 logits equal oracle/decoder.py (itself pinned by the reference's
golden vectors) on the golden model; the reference's own fp16/bf16 logits (tests/golden/
whisper_lowp_golden.npz) lie within 5 sigma of Decoder64's float64 logits at every checked step
(tests/test_lowp_oracle.py). MultiCodebook64 equals oracle/tts.py (pinned by the reference's TTS golden
vectors) on the golden TTS model, and the reference's own fp16/bf16 TTS logits (tests/golden/
tts_lowp_golden.npz) lie within 5 sigma of it (tests/test_tts_lowp_oracle.py).
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

# Sites rounded by the reference in each decoder layer, in the order they are computed, and those the
# paged path rounds (its attention kernels keep scores and probabilities in fp32 registers).
LAYER_SITES = ("norm1", "q", "k", "v", "scores", "probs", "attn", "attn_out", "res1",
               "norm2", "cq", "cscores", "cprobs", "cattn", "cattn_out", "res2",
               "norm3", "fc1", "gelu", "fc2", "res3")
FINAL_SITES = ("final_norm", "logits")
PAGED_SKIPS = frozenset(("scores", "probs", "cscores", "cprobs"))
PLACEMENTS = ("reference", "paged")

MANTISSA_BITS = {torch.float16: 11, torch.bfloat16: 8}  # significand bits incl. the implicit one
MIN_NORMAL_EXP = {torch.float16: -14, torch.bfloat16: -126}


def seeded_state(shapes: Dict[str, Tuple[int, ...]], seed: int, std: float = 0.02) -> Dict[str, torch.Tensor]:
    """float32 parameters drawn by name (sorted), from one numpy PCG64 generator (the same stream on every
    host; torch's CPU normal fill takes vector paths that depend on the host's instruction set):
    Linear / Conv / Embedding weights N(0, std), biases N(0, std), LayerNorm weights 1 + 0.2 N(0, 1) and
    biases 0.2 N(0, 1) (so that norm1 / norm2 / norm3 differ)."""
    g = np.random.default_rng(seed)
    out = {}
    for name in sorted(shapes):
        z = torch.from_numpy(g.standard_normal(shapes[name], dtype=np.float32))
        is_norm = "norm" in name.split(".")[-2] if "." in name else False
        if is_norm and name.endswith(".weight"):
            out[name] = 1.0 + 0.2 * z
        elif is_norm:
            out[name] = 0.2 * z
        else:
            out[name] = std * z
    return out


def seeded_cross_kv(layers: int, heads: int, t: int, d: int, seed: int, std: float) -> List[Tuple[torch.Tensor, ...]]:
    """Per decoder layer (K, V) [1, heads, t, d] float32 ~ N(0, std^2): encoder K/V of the magnitude
    cross_attn_k/v gives N(0, 1) encoder states."""
    g = np.random.default_rng(seed)
    shape = (1, heads, t, d)
    return [(std * torch.from_numpy(g.standard_normal(shape, dtype=np.float32)),
             std * torch.from_numpy(g.standard_normal(shape, dtype=np.float32))) for _ in range(layers)]


def checksums(state: Dict[str, torch.Tensor]) -> torch.Tensor:
    """Two exact integer sums over each tensor's raw bits (the plain sum, and the sum weighted by
    (index mod 65521) + 1), in sorted-name order: [n, 2] int64. Integer sums do not depend on the
    order a threaded reduction adds in, so every host computes the same values."""
    rows = []
    for k in sorted(state):
        t = state[k].detach().contiguous().cpu()
        bits = t.view({2: torch.int16, 4: torch.int32}[t.element_size()]).reshape(-1).to(torch.int64)
        w = torch.arange(bits.numel(), dtype=torch.int64) % 65521 + 1
        rows.append([int(bits.sum()), int((bits * w).sum())])
    return torch.tensor(rows, dtype=torch.int64)


def ulp(y: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Spacing of the dtype's values at |y| (the subnormal spacing below the smallest normal)."""
    p, emin = MANTISSA_BITS[dtype], MIN_NORMAL_EXP[dtype]
    e = torch.floor(torch.log2(y.abs().clamp_min(2.0 ** emin)))
    return torch.exp2(e - (p - 1))


def _ln(x, w, b):
    return torch.nn.functional.layer_norm(x, (x.shape[-1],), w, b, 1e-5)


def _layers(x: torch.Tensor, n_layers: int, h: int, d: int, layer_w, cross, site) -> torch.Tensor:
    """The decoder layers of models.py:110-208 over one request's sequence x [S, hidden] (causal
    self-attention, cross-attention over cross[i] where given, GELU MLP): layer_w(i, name) gives a
    weight, site(i, name, y) takes each rounding site's value and returns what the layer goes on with
    (the value itself, or the value rounded)."""
    s = x.shape[0]
    scale = 1.0 / math.sqrt(d)
    causal = torch.triu(torch.full((s, s), float("-inf"), dtype=torch.float64), diagonal=1)
    for i in range(n_layers):
        L = lambda n, i=i: layer_w(i, n)  # noqa: E731
        r = lambda n, y, i=i: site(i, n, y)  # noqa: E731
        h1 = r("norm1", _ln(x, L("norm1.weight"), L("norm1.bias")))
        q = r("q", h1 @ L("self_attn_q.weight").T).view(s, h, d).transpose(0, 1)
        k = r("k", h1 @ L("self_attn_k.weight").T).view(s, h, d).transpose(0, 1)
        v = r("v", h1 @ L("self_attn_v.weight").T).view(s, h, d).transpose(0, 1)
        w = r("scores", q @ k.transpose(1, 2)) * scale + causal
        pr = r("probs", torch.softmax(w, dim=-1))
        o = r("attn", pr @ v).transpose(0, 1).reshape(s, h * d)
        x = r("res1", x + r("attn_out", o @ L("self_attn_out.weight").T))
        used = cross is not None and i < len(cross)
        if used:
            ck, cv = cross[i]
            h2 = r("norm2", _ln(x, L("norm2.weight"), L("norm2.bias")))
            cq = r("cq", h2 @ L("cross_attn_q.weight").T).view(s, h, d).transpose(0, 1)
            cw = r("cscores", cq @ ck.transpose(1, 2)) * scale
            cp = r("cprobs", torch.softmax(cw, dim=-1))
            co = r("cattn", cp @ cv).transpose(0, 1).reshape(s, h * d)
            x = r("res2", x + r("cattn_out", co @ L("cross_attn_out.weight").T))
        n = "norm3" if used else "norm2"
        hm = r(n, _ln(x, L(f"{n}.weight"), L(f"{n}.bias")))
        f1 = r("fc1", hm @ L("mlp.0.weight").T + L("mlp.0.bias"))
        gl = r("gelu", torch.nn.functional.gelu(f1))
        x = r("res3", x + r("fc2", gl @ L("mlp.2.weight").T + L("mlp.2.bias")))
    return x


class Decoder64:
    """Float64 restatement of the reference decoder (models.py:110-208, 369-423) over one request's whole
    token sequence, causal, with per-layer cross-attention over given encoder K/V."""

    layer_prefix = "decoder_layers"

    def __init__(self, state: Dict[str, torch.Tensor], num_heads: int, head_dim: int):
        self.p = {k: v.detach().to(torch.float64) for k, v in state.items()}
        self.h, self.d = num_heads, head_dim
        self.layers = len({k.split(".")[1] for k in state if k.startswith(self.layer_prefix + ".")})

    _ln = staticmethod(_ln)

    # The model's two ends: the input rows, and the logits as a [S, V] matrix (the multi-codebook model
    # flattens its K heads into [S, K * V]). W(name) gives a weight, site(name, y) takes a rounding site,
    # start(x) takes the first gathered rows (a graph leaf when sites are recorded).
    def embed(self, ids, W, site, start) -> torch.Tensor:
        return start(W("decoder_embed.weight")[torch.as_tensor(list(ids))])

    def head(self, x, W, site) -> torch.Tensor:
        hf = site("final_norm", _ln(x, W("decoder_norm.weight"), W("decoder_norm.bias")))
        return site("logits", hf @ W("lm_head.weight").T)

    def run(self, ids, cross, site, W, cast=lambda t: t, leaf: bool = False) -> torch.Tensor:
        """The pass with site(name, y) at every rounding site ("<layer>.<site>" inside the layers), weights
        from W, the input rows and encoder K/V through cast; leaf: the input rows become a graph leaf."""
        start = (lambda t: cast(t).clone().requires_grad_(True)) if leaf else cast
        x = cast(self.embed(ids, W, site, start))
        cr = None if cross is None else [tuple(cast(t.detach().to(torch.float64)[0]) for t in kv) for kv in cross]
        x = _layers(x, self.layers, self.h, self.d, lambda i, n: W(f"{self.layer_prefix}.{i}.{n}"), cr,
                    lambda i, n, y: site(f"{i}.{n}", y))
        return self.head(x, W, site)

    def forward(self, ids: Sequence, cross: Optional[Sequence[Tuple[torch.Tensor, torch.Tensor]]],
                sites: Optional[Dict[str, torch.Tensor]] = None) -> torch.Tensor:
        """logits [S, V] of the token sequence ids (row t: the step that sees tokens 0..t). With `sites`,
        every rounding site's float64 value is recorded under "<layer>.<site>" (kept in the graph)."""
        if sites is None:
            return self.run(ids, cross, lambda n, y: y, self.p.__getitem__)
        return self.run(ids, cross, lambda n, y: sites.__setitem__(n, y) or y, self.p.__getitem__, leaf=True)


class MultiCodebook64(Decoder64):
    """Float64 restatement of the reference's streaming multi-codebook TTS model (models.py:23-77,
    211-295): the frame's input is the sum of its K codebook embeddings, added left to right (each
    partial sum a rounding site, "emb<k>"), the decoder layers without cross-attention, the final norm
    ("norm") and K linear heads. A sequence is a list of frames (K codes each); the logits of the K
    heads are laid out as one row [K * V] per position (head k's token j at k * V + j)."""

    layer_prefix = "layers"

    def embed(self, frames, W, site, start) -> torch.Tensor:
        codes = torch.as_tensor([list(f) for f in frames])
        k_n = codes.shape[1]
        x = start(W("embeddings.embeddings.0.weight")[codes[:, 0]])
        for k in range(1, k_n):
            x = site(f"emb{k}", x + W(f"embeddings.embeddings.{k}.weight")[codes[:, k]])
        return x

    def head(self, x, W, site) -> torch.Tensor:
        hf = site("final_norm", _ln(x, W("norm.weight"), W("norm.bias")))
        k_n = len([n for n in self.p if n.startswith("heads.heads.")])
        return site("logits", torch.cat([hf @ W(f"heads.heads.{k}.weight").T for k in range(k_n)], dim=-1))


def _site_kind(name: str) -> str:
    return name.split(".", 1)[1] if "." in name else name


def rounding_sigma(model: Decoder64, ids: Sequence[int], cross, dtype: torch.dtype, positions: Sequence[int],
                   pairs: Sequence[Tuple[int, Optional[int]]],
                   placements: Sequence[str] = PLACEMENTS) -> Tuple[torch.Tensor, torch.Tensor]:
    """For each position t (a row of the teacher-forced sequence) and (a, b) token pair: the standard
    deviation of the rounding error of z_t[a] - z_t[b] (b None: of z_t[a] alone), summed over the
    rounding sites of the given placements. Returns (sigmas [len(positions)], float64 logits [S, V])."""
    sites: Dict[str, torch.Tensor] = {}
    logits = model.forward(ids, cross, sites)
    names = list(sites)
    ulps = {n: ulp(sites[n].detach(), dtype) for n in names}
    sig = []
    for t, (a, b) in zip(positions, pairs):
        target = logits[t, a] - (logits[t, b] if b is not None else 0.0)
        grads = torch.autograd.grad(target, [sites[n] for n in names], retain_graph=True, allow_unused=True)
        var = 0.0
        for n, g in zip(names, grads):
            if g is None:
                continue
            per = float(((g.detach() * ulps[n]) ** 2).sum()) / 12.0
            kind = _site_kind(n)
            for pl in placements:
                if pl == "paged" and kind in PAGED_SKIPS:
                    continue
                var += per
        sig.append(math.sqrt(var))
    return torch.tensor(sig, dtype=torch.float64), logits.detach()


def round_through(model: Decoder64, ids: Sequence, cross, dtype: torch.dtype, placement: str) -> torch.Tensor:
    """The float64 pass with every site of `placement` rounded to dtype (round to nearest even) where it
    is produced, from weights, input rows and encoder K/V in dtype: an emulation of that implementation's
    arithmetic up to its fp32 accumulation order."""
    skip = PAGED_SKIPS if placement == "paged" else frozenset()
    rt = lambda y: y.to(dtype).to(torch.float64)  # noqa: E731
    return model.run(ids, cross, lambda n, y: y if _site_kind(n) in skip else rt(y), lambda n: rt(model.p[n]), rt)
