"""Write golden vectors of the reference's streaming multi-codebook TTS model and engine.

Run in the development container, where the reference repository is mounted:
    python tests/golden/make_tts_golden.py [/path/to/reference]          # float32 vectors
    python tests/golden/make_tts_golden.py [/path/to/reference] --lowp   # fp16 / bf16 greedy frames

--lowp writes tests/golden/tts_lowp_golden.npz: the reference's own reduced-precision greedy decode
(its StreamingMultiCodebookTTSModel cast to float16 and to bfloat16 on the CPU, model(...) with a
DynamicCache per frame, argmax per codebook) for two shapes, the float32 golden shape below and the
reference model's default shape (4 layers, 4 heads x 64, 4 codebooks, vocab 1024), two requests each:
per frame the K codes and each codebook's top-16 logits (for the small shape every logit). Weights and
prompts are drawn from seeds by name (oracle/rounding.seeded_state, numpy PCG64), so a run that
regenerates them checks the recorded checksums.

The float32 mode imports speech_serving.models.StreamingMultiCodebookTTSModel and
speech_serving.tts_engine.StreamingTTSEngine from the reference (CPU,
float32), builds a small seeded model with the shapes of the reference's own
TTS test (test_speech_engine.py:35-91), and saves to
tests/golden/tts_small_golden.npz (numpy arrays only, no pickles):
    param.*                 the model's state_dict
    prompts                 [R, P, K] int64 prompt codebook frames
    prefill_logits{r}       model(prompt r) logits [1, P, K, V]
    prefill_k{l}/v{l}       request 0's prefill K/V per layer [1, H, P, D]
    step_logits{r}          the last-position logits of every generated frame
                            of request r, from the model run incrementally
                            with its contiguous past [F, K, V]
    engine_frames{r}        the reference engine's frames for request r [F, K]
    engine_blocks           allocated / free block counts after the run
The oracle (oracle/tts.py) is checked against this file by
tests/test_tts_oracle.py, and the HIP engine by tests/test_tts_gpu.py.
No test, benchmark or library code reads the reference; the tests read only this file.
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "tts_small_golden.npz")

CONFIG = dict(num_layers=2, num_heads=4, hidden_dim=64, num_codebooks=4, vocab_size=128)
BLOCK_SIZE = 8
NUM_BLOCKS = 32
MAX_BATCH = 2
REQUESTS = 3
PROMPT_LEN = 10
FRAMES = 15
MIN_MARGIN = 1e-3  # smallest top-1 minus top-2 logit gap the chosen seed must keep


def build(seed, TTSModel):
    torch.manual_seed(seed)
    model = TTSModel(**CONFIG).eval()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        # Distinct LayerNorm parameters so norm1 / norm2 / final norm are distinguishable.
        for mod in model.modules():
            if isinstance(mod, torch.nn.LayerNorm):
                mod.weight.add_(0.2 * torch.randn(mod.weight.shape, generator=g))
                mod.bias.add_(0.2 * torch.randn(mod.bias.shape, generator=g))
    prompts = torch.randint(0, CONFIG["vocab_size"], (REQUESTS, PROMPT_LEN, CONFIG["num_codebooks"]), generator=g)
    return model, prompts


def incremental(model, prompt, frames):
    """Prefill, then one frame per step with the contiguous past: last-position logits per frame."""
    out = model(input_codebooks=prompt[None], use_cache=True)
    logits = []
    for _ in range(frames):
        last = out.logits[0, -1]  # [K, V]
        logits.append(last.clone())
        nxt = torch.argmax(last, dim=-1)[None, None]  # [1, 1, K]
        out = model(input_codebooks=nxt, past_key_values=out.past_key_values, use_cache=True)
    return torch.stack(logits)


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from speech_serving.models import StreamingMultiCodebookTTSModel  # noqa: E402  (reference)
    from speech_serving.tts_engine import StreamingTTSEngine  # noqa: E402  (reference)
    from paged_kv_cache.block_manager import BlockManager  # noqa: E402  (reference)

    for seed in range(2024, 2124):
        model, prompts = build(seed, StreamingMultiCodebookTTSModel)
        with torch.no_grad():
            steps = [incremental(model, prompts[r], FRAMES) for r in range(REQUESTS)]
        top2 = torch.stack(steps).topk(2, dim=-1).values
        margin = float((top2[..., 0] - top2[..., 1]).min())
        if margin >= MIN_MARGIN:
            break
    else:
        raise SystemExit("no seed in range keeps every greedy margin above MIN_MARGIN")

    out = {f"param.{k}": v.detach().numpy().copy() for k, v in model.state_dict().items()}
    out["prompts"] = prompts.numpy().astype(np.int64)
    with torch.no_grad():
        for r in range(REQUESTS):
            pre = model(input_codebooks=prompts[r][None], use_cache=True)
            out[f"prefill_logits{r}"] = pre.logits.numpy()
            if r == 0:
                for l in range(CONFIG["num_layers"]):
                    out[f"prefill_k{l}"] = pre.past_key_values.layers[l].keys.numpy()
                    out[f"prefill_v{l}"] = pre.past_key_values.layers[l].values.numpy()
            out[f"step_logits{r}"] = steps[r].numpy()

        bm = BlockManager(num_layers=CONFIG["num_layers"], num_kv_heads=CONFIG["num_heads"],
                          head_dim=CONFIG["hidden_dim"] // CONFIG["num_heads"], block_size=BLOCK_SIZE,
                          num_blocks=NUM_BLOCKS, dtype=torch.float32, device="cpu")
        engine = StreamingTTSEngine(model, bm, max_batch_size=MAX_BATCH, device="cpu")
        for r in range(REQUESTS):
            engine.submit(prompts[r], max_new_frames=FRAMES)
        done = sorted(engine.run_until_done(), key=lambda q: q.id)
    for q in done:
        frames = torch.stack(q.generated_frames).numpy().astype(np.int64)
        out[f"engine_frames{q.id}"] = frames
        # The engine's frames are the argmax of the incremental model's logits.
        assert (frames == steps[q.id].argmax(-1).numpy()).all(), f"engine and incremental model differ (req {q.id})"
    out["engine_blocks"] = np.array([bm.allocated_block_count, bm.num_free_blocks], dtype=np.int64)
    out["config_json"] = np.frombuffer(json.dumps(dict(
        CONFIG, seed=seed, block_size=BLOCK_SIZE, num_blocks=NUM_BLOCKS, max_batch=MAX_BATCH,
        requests=REQUESTS, prompt_len=PROMPT_LEN, frames=FRAMES, min_margin=margin)).encode(), dtype=np.uint8)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(out)} arrays), seed {seed}, min margin {margin:.4g}")


LOWP_OUT = os.path.join(HERE, "tts_lowp_golden.npz")
LOWP_SHAPES = {
    # layers, heads, hidden, codebooks, vocab, prompt frames, generated frames, weight std, seeds
    "small": dict(num_layers=2, num_heads=4, hidden_dim=64, num_codebooks=4, vocab_size=128, prompt_len=8,
                  frames=16, std=0.1, seed=3101, prompt_seeds=[3102, 3103]),
    "default": dict(num_layers=4, num_heads=4, hidden_dim=256, num_codebooks=4, vocab_size=1024, prompt_len=8,
                    frames=16, std=0.05, seed=3201, prompt_seeds=[3202, 3203]),
}
LOWP_DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}
TOPK = 16


def lowp_prompt(cfg, seed):
    """[P, K] int64 prompt frames, uniform codes from one numpy PCG64 stream."""
    g = np.random.default_rng(seed)
    return g.integers(0, cfg["vocab_size"], size=(cfg["prompt_len"], cfg["num_codebooks"]), dtype=np.int64)


def write_lowp(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))  # the repository root, for oracle/
    from speech_serving.models import StreamingMultiCodebookTTSModel  # noqa: E402  (reference)

    from oracle.rounding import checksums, seeded_state  # noqa: E402

    out = {}
    for shape, cfg in LOWP_SHAPES.items():
        args = {k: cfg[k] for k in ("num_layers", "num_heads", "hidden_dim", "num_codebooks", "vocab_size")}
        for dname, dtype in LOWP_DTYPES.items():
            model = StreamingMultiCodebookTTSModel(**args)
            state = seeded_state({k: tuple(v.shape) for k, v in model.state_dict().items()}, cfg["seed"], cfg["std"])
            model.load_state_dict(state)
            model = model.to(dtype).eval()
            out[f"{shape}.{dname}.param_checksums"] = checksums({k: v.to(dtype) for k, v in state.items()}).numpy()
            for r, pseed in enumerate(cfg["prompt_seeds"]):
                key = f"{shape}.{dname}.r{r}"
                prompt = lowp_prompt(cfg, pseed)
                frames, tk_i, tk_v, full = [], [], [], []
                with torch.no_grad():
                    cur = model(input_codebooks=torch.from_numpy(prompt)[None], use_cache=True)
                    for _ in range(cfg["frames"]):
                        last = cur.logits[0, -1]  # [K, V]
                        vals, idx = torch.topk(last.float(), TOPK, dim=-1)
                        tk_i.append(idx.numpy())
                        tk_v.append(vals.numpy())
                        if shape == "small":
                            full.append(last.float().numpy())
                        nxt = torch.argmax(last, dim=-1)
                        frames.append(nxt.numpy())
                        cur = model(input_codebooks=nxt[None, None], past_key_values=cur.past_key_values,
                                    use_cache=True)
                out[f"{key}.prompt"] = prompt
                out[f"{key}.frames"] = np.stack(frames).astype(np.int64)
                out[f"{key}.topk_idx"] = np.stack(tk_i).astype(np.int64)
                out[f"{key}.topk_val"] = np.stack(tk_v).astype(np.float32)
                if full:
                    out[f"{key}.logits"] = np.stack(full).astype(np.float32)
                print(f"  {key}: frames {[f.tolist() for f in frames[:4]]} ... distinct codes "
                      f"{len(set(np.stack(frames).reshape(-1).tolist()))}")
    out["config_json"] = np.frombuffer(json.dumps(dict(shapes=LOWP_SHAPES, dtypes=list(LOWP_DTYPES),
                                                       topk=TOPK)).encode(), dtype=np.uint8)
    np.savez_compressed(LOWP_OUT, **out)
    print(f"wrote {LOWP_OUT} ({os.path.getsize(LOWP_OUT)} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    root = args[0] if args else "/root/reference"
    if "--lowp" in sys.argv[1:]:
        write_lowp(root)
    else:
        main(root)
