"""Benchmark of the decoder KV-cache hot path on one MI355X.

Main workload (the JSON line's value): paged decode attention for one decoder
layer, fp16, 32 heads x 64, block size 16, batch 64, per-sequence context
U[1, 448], block tables a seeded random permutation of a 4096-block pool,
Q/K/V ~ N(0, 1). One step = one fused launch that appends the batch's new
token K/V into the pool through each sequence's block table and attends over
the sequence's context (new token included). Inputs are resident in HBM
before timing. Steps rotate over independent pool/table sets whose combined
footprint exceeds the 256 MB last-level cache, so every step streams its K/V
from HBM.

Extra fields (same JSON line), Whisper-large-v3 decoder shapes (bf16, 20 heads
x 64, batch 64):
  large_v3_paged_attention  the same fused kernel at ctx U[1, 452] (and at batch 128,
                            the large-v3 serving configuration's slot count)
  large_v3_cross_attention  attention over 1500 contiguous encoder positions
  large_v3_append / _gather the standalone append (encoder K/V store) and block-table
                            gather kernels
  large_v3_prefill_cross_attention  the prompt prefill's cross-attention, 128 requests x q_len
                            1 / 4 / 16 (multi-query matrix-core kernel for q_len >= 2)
  large_v3_encoder_attention  encoder attention over paged blocks (1500 queries, 64-query tiles)
  large_v3_argmax           greedy tokens of a decode step (64 x 51866 logits) with slot feedback
  large_v3_cross_copy       one request's encoder K/V (32 layers) into its decode slot
  tts_decode                the streaming multi-codebook TTS engine (reference TTS
                            model's default shape, 64 requests x 256 frames)
  config1_decode            the Whisper-tiny-shaped decoder of config 1 (4 requests x 64 greedy
                            tokens, fp32): GPU graph and eager decode tokens/s beside the
                            reference's eager path on the host
  large_v3_decode           end-to-end greedy decode through the scheduler's
                            captured graphs: 32 layers, d_model 1280, vocab
                            51866, N(0, 0.02) weights, 64 requests x 448 tokens,
                            random N(0,1) encoder states projected by cross_attn_k/v.
  large_v3_serving          the large-v3 serving scenario: 128 graph slots, a burst of
                            256 requests x 448 tokens at t=0, a decoder pool that holds
                            the 128 slots' blocks but not the burst's, so admission waits
                            for freed blocks and recycles them.

Every cpu_baseline block times oracle/cpu_path.py (the reference's eager path restated in float32
torch) on torch's host threads and records the thread count and the CPU model.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--no-cpu-baseline] [--no-large-v3]
    python bench.py --mode copy    # known-size copy for PMC counter scaling
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "inference-speech-model_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E peak
LLC_BYTES = 256 << 20  # MI355X Infinity Cache


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--heads", type=int, default=32)
    ap.add_argument("--head-dim", type=int, default=64)
    ap.add_argument("--block-size", type=int, default=16)
    ap.add_argument("--pool-blocks", type=int, default=4096)
    ap.add_argument("--max-ctx", type=int, default=448)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--chunk", type=int, default=0, help="split-K chunk (0 = library default)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-large-v3", action="store_true", help="skip the large-v3 kernel and decode measurements")
    ap.add_argument("--no-decode", action="store_true", help="skip the large-v3 decode (keep its kernel measurements)")
    ap.add_argument("--no-tts", action="store_true", help="skip the streaming TTS engine measurement")
    ap.add_argument("--no-config1", action="store_true", help="skip the Whisper-tiny config-1 decode")
    ap.add_argument("--decode-batch", type=int, default=64)
    ap.add_argument("--decode-tokens", type=int, default=448)
    ap.add_argument("--decode-layers", type=int, default=32)
    ap.add_argument("--no-serving", action="store_true", help="skip the large-v3 256-request serving burst")
    ap.add_argument("--mode", choices=["attention", "copy", "decode", "decode-eager", "serving", "tts", "config1", "prefill",
                                       "copies"],
                    default="attention",
                    help="copy: plain device copy of --copy-mib MiB, a known-traffic kernel for counter scaling; "
                         "decode: only the large-v3-shaped greedy decode; serving: only the large-v3 serving "
                         "burst; tts: only the streaming TTS engine; copies: only the large-v3 append, gather, "
                         "slot handoff copy and argmax")
    ap.add_argument("--copy-mib", type=int, default=512)
    return ap.parse_args()


def copy_calibration(a):
    """Copy a buffer of known size --steps times (reads and writes copy-mib MiB each)."""
    import torch

    n = a.copy_mib << 20
    src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / a.steps
    print(json.dumps({"mode": "copy", "bytes_read_per_launch": n, "bytes_written_per_launch": n,
                      "launches": a.steps + 3, "us_per_copy": round(dt * 1e6, 2),
                      "GBps_read_plus_write": round(2 * n / dt / 1e9, 1)}), flush=True)


def measured_traffic(a, digest):
    """HBM bytes per launch from the committed rocprofv3 PMC summary of this exact config, measured
    with a library built from these exact sources (same src digest), else None."""
    key = (f"fp16/b{a.batch}/h{a.heads}/d{a.head_dim}/bs{a.block_size}/nb{a.pool_blocks}/"
           f"ctx{a.max_ctx}/seed{a.seed}")
    path = os.path.join(ROOT, "profiles", "paged_attention_config2.md")
    if a.chunk or not os.path.exists(path):
        return None
    for line in open(path):
        if not line.startswith("traffic_bytes_per_launch="):
            continue
        fields = dict(f.split("=", 1) for f in line.split() if "=" in f)
        if fields.get("config") == key and fields.get("src") == digest:
            return int(fields["traffic_bytes_per_launch"])
    return None


def attention_bytes(ctx, heads, d, elt, bs):
    """Algorithmic bytes of one paged attention launch: K+V rows read, q read,
    out written, block-table entries and the length read."""
    return sum(2 * c * heads * d * elt + 2 * heads * d * elt + 4 * math.ceil(c / bs) + 4 for c in ctx)


def append_write_bytes(batch, heads, d, elt):
    """Pool bytes the fused append writes (the new rows themselves are read as keys)."""
    return batch * 2 * heads * d * elt


def append_bytes(batch, heads, d, elt):
    """Standalone append: read the new rows, write them, read the slot ids."""
    return batch * (2 * heads * d * elt + 2 * heads * d * elt + 8)


class ProblemSet:
    """One independent copy of a paged-attention workload: pool, tables, lengths, inputs.

    Rows are laid out longest-first, as the engine lays out its decode batch
    (sorted=False keeps the drawn order).
    """

    def __init__(self, torch, seed, device, dtype, batch, heads, d, bs, nb, max_ctx, sorted_rows=True):
        g = torch.Generator().manual_seed(seed)
        self.ctx = torch.randint(1, max_ctx + 1, (batch,), generator=g)  # keys incl. the new token
        if sorted_rows:
            self.ctx = self.ctx.sort(descending=True).values
        maxblk = math.ceil(max_ctx / bs)
        perm = torch.randperm(nb, generator=g)[: batch * maxblk]
        self.tables_cpu = perm.view(batch, maxblk).to(torch.int32)
        self.k_pool = torch.randn(nb, bs, heads, d, generator=g).to(device, dtype)
        self.v_pool = torch.randn(nb, bs, heads, d, generator=g).to(device, dtype)
        self.q = torch.randn(batch, heads, d, generator=g).to(device, dtype)
        self.k_new = torch.randn(batch, heads, d, generator=g).to(device, dtype)
        self.v_new = torch.randn(batch, heads, d, generator=g).to(device, dtype)
        pos = (self.ctx - 1).tolist()
        self.slots = [int(self.tables_cpu[i, p // bs]) * bs + p % bs for i, p in enumerate(pos)]
        self.tables = self.tables_cpu.to(device)
        self.ctx_dev = self.ctx.to(torch.int32).to(device)
        self.out = torch.empty_like(self.q)
        elt = torch.empty((), dtype=dtype).element_size()
        self.bytes = attention_bytes(self.ctx.tolist(), heads, d, elt, bs) + append_write_bytes(batch, heads, d, elt)


GRAPH_STEPS = 32  # steps per captured graph in the timed region: the large-v3 decoder's layers per token step


def graph_launch_us(torch, fns, per_fn=8, replays=7):
    """Average duration of one launch, from HIP events around replays of a captured graph that
    holds per_fn back-to-back launches of every fn (rotating through fns). The events sit on the
    stream the graph is replayed on; the gap between dependent launches is included."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for f in fns:
            f()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    n = per_fn * len(fns)
    with torch.cuda.graph(g):
        for i in range(n):
            fns[i % len(fns)]()
    # Warm-up replays for at least ~0.2 s of GPU time, so the timed replays see the GPU's
    # steady-state clocks rather than the ramp after an idle host phase.
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 0.2:
        for _ in range(4):
            g.replay()
        torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    per = []
    for _ in range(replays):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(cur)
        g.replay()
        b.record(cur)
        b.synchronize()
        per.append(a.elapsed_time(b) * 1e3 / n)
    del g
    per.sort()
    return per[len(per) // 2]


def paged_sets(torch, native, dev, dtype, batch, heads, d, bs, nb, max_ctx, seed, chunk, sorted_rows=True):
    one = ProblemSet(torch, seed, dev, dtype, batch, heads, d, bs, nb, max_ctx, sorted_rows)
    nsets = max(2, math.ceil(2 * LLC_BYTES / one.bytes) + 1)
    sets = [one] + [ProblemSet(torch, seed + i, dev, dtype, batch, heads, d, bs, nb, max_ctx, sorted_rows)
                    for i in range(1, nsets)]
    native.reserve_attention(batch, heads, d, max_ctx, dtype, dev, chunk)
    return sets


def host_cpu():
    """(threads torch uses, CPU model, logical CPUs the OS reports). The threads are torch's own count,
    i.e. OMP_NUM_THREADS where it is set (the process's share of the host), else every core."""
    import torch

    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return torch.get_num_threads(), model, os.cpu_count()


def baseline_record(value, unit, sample, **extra):
    threads, model, cpus = host_cpu()
    return {"value": value, "unit": unit, "cores": threads, "kind": "port", "dtype": "fp32",
            "cpu_model": model, "host_logical_cpus": cpus,
            "path": "the reference's eager path restated in float32 torch (oracle/cpu_path.py)",
            "sample": sample, **extra}


def cpu_baseline(s, a, scale, budget_s):
    """The paged-attention microbench step (fp16, 32 heads, batch 64) on the host: append + block-table gather into a zero-padded batch + masked
    attention in float32 torch on torch's threads (oracle/cpu_path.paged_attention_step). value is
    the GPU workload's algorithmic bytes (fp16 element size) per CPU call time, so the two values
    compare as the inverse of their times."""
    import torch

    from oracle import cpu_path as C

    kp = s.k_pool.float().cpu()
    vp = s.v_pool.float().cpu()
    q = s.q.float().cpu()
    kn, vn = s.k_new.float().cpu(), s.v_new.float().cpu()
    tables = s.tables_cpu.long()
    ctx = s.ctx.tolist()
    nbytes = attention_bytes(ctx, a.heads, a.head_dim, 2, a.block_size) + append_write_bytes(a.batch, a.heads,
                                                                                             a.head_dim, 2)
    times = []
    with torch.no_grad():
        C.paged_attention_step(q, kp, vp, tables, ctx, kn, vn, scale)  # warm-up
        t_end = time.perf_counter() + budget_s
        while time.perf_counter() < t_end or len(times) < 10:
            t0 = time.perf_counter()
            C.paged_attention_step(q, kp, vp, tables, ctx, kn, vn, scale)
            times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return baseline_record(round(nbytes / med / 1e9, 4), "GB/s",
                           f"{len(times)} calls of the whole microbench batch (B={a.batch}, fused append + gather + "
                           f"attention), median {med * 1e3:.2f} ms per call",
                           ms_per_step=round(med * 1e3, 3))


def large_v3_kernels(torch, native, dev, a):
    """Fused paged attention and cross-attention at Whisper-large-v3 decoder shapes, batch 64, bf16."""
    dt, b, h, d = torch.bfloat16, 64, 20, 64
    out = {}
    # Rows longest-first with SKV_ATTN_ROWS_LONGEST_FIRST (the graph decode's layout), the same rows
    # without the flag (the launch checks their order itself), and rows in drawn order (ranked in the launch).
    for sorted_rows, flag in ((True, True), (True, False), (False, False)):
        sets = paged_sets(torch, native, dev, dt, b, h, d, 16, 4096, 452, a.seed + 100, 0, sorted_rows)
        fns = [lambda s=s: native.paged_attention(s.q, s.k_pool, s.v_pool, s.tables, s.ctx_dev, 452, 0.125,
                                                  out=s.out, k_new=s.k_new, v_new=s.v_new, rows_longest_first=flag)
               for s in sets]
        avg = graph_launch_us(torch, fns)
        byts = sum(s.bytes for s in sets) / len(sets)
        if flag:
            out["large_v3_paged_attention"] = {
                "shape": "bf16, 20 heads x 64, batch 64, block size 16, ctx U[1,452], fused append, "
                         "rows longest-first (flagged SKV_ATTN_ROWS_LONGEST_FIRST, as the graph decode does)",
                "avg_launch_us": round(avg, 3), "algorithmic_bytes_per_launch": int(byts),
                "achieved_GBps": round(byts / (avg * 1e-6) / 1e9, 1),
                "frac": round(byts / (avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        elif sorted_rows:
            r = out["large_v3_paged_attention"]
            r["longest_first_unflagged_avg_launch_us"] = round(avg, 3)
            r["longest_first_unflagged_frac"] = round(byts / (avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
        else:
            r = out["large_v3_paged_attention"]
            r["unsorted_rows_avg_launch_us"] = round(avg, 3)
            r["unsorted_rows_frac"] = round(byts / (avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
        del sets, fns
        torch.cuda.empty_cache()
    # The same kernel at batch 128 (the large-v3 serving configuration's slot count): rows longest-first
    # (flagged), and rows in drawn order (ranked in the launch).
    for sorted_rows in (True, False):
        sets = paged_sets(torch, native, dev, dt, 128, h, d, 16, 4096, 452, a.seed + 150, 0, sorted_rows)
        fns = [lambda s=s: native.paged_attention(s.q, s.k_pool, s.v_pool, s.tables, s.ctx_dev, 452, 0.125,
                                                  out=s.out, k_new=s.k_new, v_new=s.v_new,
                                                  rows_longest_first=sorted_rows)
               for s in sets]
        avg = graph_launch_us(torch, fns)
        byts = sum(s.bytes for s in sets) / len(sets)
        if sorted_rows:
            out["large_v3_paged_attention"]["batch128"] = {
                "avg_launch_us": round(avg, 3), "algorithmic_bytes_per_launch": int(byts),
                "frac": round(byts / (avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        else:
            r = out["large_v3_paged_attention"]["batch128"]
            r["unsorted_rows_avg_launch_us"] = round(avg, 3)
            r["unsorted_rows_frac"] = round(byts / (avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
        del sets, fns
        torch.cuda.empty_cache()
    t = 1500
    kvs = []
    for i in range(2):  # 2 x 491 MB > 256 MB last-level cache
        g = torch.Generator(device=dev).manual_seed(a.seed + 200 + i)
        kvs.append((torch.randn(b, 2, h, t, d, generator=g, device=dev, dtype=dt),
                    torch.randn(b, h, d, generator=g, device=dev, dtype=dt)))
    lens = torch.full((b,), t, dtype=torch.int32, device=dev)
    res = torch.empty(b, h, d, dtype=dt, device=dev)
    native.reserve_attention(b, h, d, t, dt, dev)
    fns = [lambda kv=kv: native.dense_attention(kv[1], kv[0][:, 0], kv[0][:, 1], lens, t, 0.125, out=res)
           for kv in kvs]
    avg = graph_launch_us(torch, fns, per_fn=4, replays=5)
    byts = b * (2 * t * h * d * 2 + 2 * h * d * 2 + 4)
    out["large_v3_cross_attention"] = {
        "shape": "bf16, 20 heads x 64, batch 64, 1500 encoder positions (g_cross_kv slot-major layer slice)",
        "avg_launch_us": round(avg, 3), "algorithmic_bytes_per_launch": int(byts),
        "achieved_GBps": round(byts / (avg * 1e-6) / 1e9, 1), "frac": round(byts / (avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    del kvs, fns
    torch.cuda.empty_cache()
    return out


def large_v3_prefill_cross(torch, native, dev, a):
    """The prompt prefill's cross-attention at the large-v3 serving shape: 128 requests x q_len prompt
    tokens against each request's 1500 contiguous encoder positions (bf16, 20 heads x 64, the
    slot-major g_cross_kv layer slice). q_len >= 2 runs the multi-query matrix-core kernel (K/V read
    once per request); q_len 1 and the one-query-per-row form of q_len 4 (every query row re-reads
    its request's K/V, the kernel used for prompts before) run the decode kernel. Bytes: K/V of
    every request once, plus q and out."""
    dt, b, h, d, t = torch.bfloat16, 128, 20, 64, 1500
    kvs = []
    for i in range(2):  # 2 x 983 MB > the 256 MB last-level cache
        g = torch.Generator(device=dev).manual_seed(a.seed + 400 + i)
        kvs.append(torch.randn(b, 2, h, t, d, generator=g, device=dev, dtype=dt))
    lens = torch.full((b,), t, dtype=torch.int32, device=dev)
    out = {"shape": "bf16, 20 heads x 64, 128 requests, 1500 encoder positions each (g_cross_kv slot-major layer "
                    "slice)"}
    for q_len in (1, 4, 16):
        g = torch.Generator(device=dev).manual_seed(a.seed + 410 + q_len)
        q = torch.randn(b, q_len, h, d, generator=g, device=dev, dtype=dt)
        res = torch.empty_like(q)
        native.reserve_attention(b * q_len, h, d, t, dt, dev)
        fns = [lambda kv=kv: native.dense_attention(q, kv[:, 0], kv[:, 1], lens, t, 0.125, out=res) for kv in kvs]
        us = graph_launch_us(torch, fns, per_fn=4, replays=5)
        byts = b * (2 * t * h * d * 2 + q_len * 2 * h * d * 2 + 4)
        out[f"q{q_len}"] = {"avg_launch_us": round(us, 3), "algorithmic_bytes_per_launch": byts,
                            "achieved_GBps": round(byts / (us * 1e-6) / 1e9, 1),
                            "frac": round(byts / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        if q_len == 4:  # the same 4 queries as one-query rows (K/V re-read per query)
            q1 = q.reshape(b * q_len, 1, h, d)
            r1 = torch.empty_like(q1)
            slots = torch.arange(b, dtype=torch.int32, device=dev).repeat_interleave(q_len)
            lens1 = torch.full((b * q_len,), t, dtype=torch.int32, device=dev)
            native.reserve_attention(b * q_len, h, d, t, dt, dev)
            fns = [lambda kv=kv: native.dense_attention(q1, kv[:, 0], kv[:, 1], lens1, t, 0.125, slot_ids=slots,
                                                        out=r1) for kv in kvs]
            out["q4_one_query_rows_avg_launch_us"] = round(graph_launch_us(torch, fns, per_fn=4, replays=5), 3)
            torch.cuda.synchronize()
            out["q4_max_abs_diff_vs_one_query_rows"] = float((res.float() - r1.view_as(res).float()).abs().max())
    del kvs
    torch.cuda.empty_cache()
    return out


def large_v3_encoder_attention(torch, native, dev, a):
    """EncoderAttentionBackend at the large-v3 encoder shape: 1500 queries x 20 heads x 64 of one
    request attending its 1500 encoder positions in 94 pool blocks of 16 (bf16, non-causal). The
    multi-query kernel reads the blocks once per 16 queries; the one-query-per-row form (the path
    this call took before) reads them once per query. Compute-bound: 4 * 1500 * 1500 * 64 * 20 flops."""
    dt, h, d, t, bs = torch.bfloat16, 20, 64, 1500, 16
    nblk = -(-t // bs)
    g = torch.Generator(device=dev).manual_seed(a.seed + 500)
    kp = torch.randn(4 * nblk, bs, h, d, generator=g, device=dev, dtype=dt)
    vp = torch.randn(4 * nblk, bs, h, d, generator=g, device=dev, dtype=dt)
    table = torch.randperm(4 * nblk, generator=torch.Generator().manual_seed(a.seed + 501))[:nblk].tolist()
    q = torch.randn(1, t, h, d, generator=g, device=dev, dtype=dt)
    flops = 4 * t * t * d * h
    tbl = torch.tensor([table], dtype=torch.int32, device=dev)
    one = torch.full((1,), t, dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    native.reserve_attention(t, h, d, t, dt, dev)
    # The call EncoderAttentionBackend.forward makes (one shared table row, non-causal).
    fns = [lambda: native.paged_attention(q, kp, vp, tbl, one, t, 0.125, out=out)]
    us = graph_launch_us(torch, fns, per_fn=8, replays=5)
    q1 = q.reshape(t, 1, h, d)
    rows = torch.zeros(t, dtype=torch.int32, device=dev)
    lens = torch.full((t,), t, dtype=torch.int32, device=dev)
    fns1 = [lambda: native.paged_attention(q1, kp, vp, tbl, lens, t, 0.125, table_rows=rows)]
    us1 = graph_launch_us(torch, fns1, per_fn=4, replays=5)
    return {"shape": "bf16, one request, 1500 queries x 20 heads x 64 over 1500 positions in 94 pool blocks",
            "avg_launch_us": round(us, 3), "tflops": round(flops / (us * 1e-6) / 1e12, 1),
            "frac_of_bf16_mfma_peak": round(flops / (us * 1e-6) / 2.5e15, 4),
            "one_query_rows_avg_launch_us": round(us1, 3)}


def large_v3_append_gather(torch, native, dev, a):
    """Standalone append and block-table gather at Whisper-large-v3 shapes (bf16, 20 heads x 64).

    append: one layer's K and V rows of 64 requests x 1500 encoder positions into a paged pool through
    a seeded permutation of its slots (the encoder K/V store); bytes = rows read + rows written + slots.
    gather: the decoder pool of a batch of 64 (ctx U[1,452], longest-first) into zero-padded
    [64, 20, 452, 64] K and V; bytes = pool rows read + padded output written + table entries."""
    dt, h, d, bs = torch.bfloat16, 20, 64, 16
    out = {}
    n = 64 * 1500
    g = torch.Generator(device=dev).manual_seed(a.seed + 300)
    kn = torch.randn(n, h, d, generator=g, device=dev, dtype=dt)
    vn = torch.randn(n, h, d, generator=g, device=dev, dtype=dt)
    nb = n // bs
    kp = torch.zeros(nb, bs, h, d, device=dev, dtype=dt)
    vp = torch.zeros_like(kp)
    slots = torch.randperm(nb, generator=torch.Generator().manual_seed(a.seed + 301))
    slots = (slots[:, None] * bs + torch.arange(bs)[None]).reshape(-1).to(dev)
    avg = graph_launch_us(torch, [lambda: native.append(kn, vn, kp, vp, slots)], per_fn=4, replays=5)
    byts = n * (2 * h * d * 2 + 2 * h * d * 2 + 8)
    out["large_v3_append"] = {
        "shape": "bf16, 20 heads x 64, 64 requests x 1500 encoder positions (one layer's K and V) into a paged "
                 "pool through a permuted slot mapping",
        "avg_launch_us": round(avg, 3), "algorithmic_bytes_per_launch": int(byts),
        "achieved_GBps": round(byts / (avg * 1e-6) / 1e9, 1), "frac": round(byts / (avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    del kn, vn, kp, vp, slots
    torch.cuda.empty_cache()

    sets = paged_sets(torch, native, dev, dt, 64, h, d, bs, 4096, 452, a.seed + 100, 0, True)
    outs = (torch.empty(64, h, 452, d, device=dev, dtype=dt), torch.empty(64, h, 452, d, device=dev, dtype=dt))
    fns = [lambda s=s: native.gather(s.k_pool, s.v_pool, s.tables, s.ctx_dev, 452, k_out=outs[0], v_out=outs[1])
           for s in sets]
    avg = graph_launch_us(torch, fns)
    byts = sum(2 * sum(s.ctx.tolist()) * h * d * 2 + 2 * 64 * h * 452 * d * 2 +
               4 * sum(math.ceil(c / bs) for c in s.ctx.tolist()) + 4 * 64 for s in sets) / len(sets)
    out["large_v3_gather"] = {
        "shape": "bf16, 20 heads x 64, batch 64, ctx U[1,452] longest-first, block size 16, into zero-padded "
                 "[64, 20, 452, 64] K and V",
        "avg_launch_us": round(avg, 3), "algorithmic_bytes_per_launch": int(byts),
        "achieved_GBps": round(byts / (avg * 1e-6) / 1e9, 1), "frac": round(byts / (avg * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    del sets, fns, outs
    torch.cuda.empty_cache()
    return out


def large_v3_cross_copy(torch, native, dev, a):
    """Encoder K/V into a decode slot (the graph decode's slot handoff) at the large-v3 shape: one request's
    32 layers of K and V, 20 heads x 1500 positions x 64 bf16 each, into the slot's region of the
    slot-major cross-attention buffer, one launch. Two rotating request/slot pairs (2 x 492 MB moved >
    the 256 MB last-level cache). Bytes: every element read once and written once."""
    L, h, t, d, dt = 32, 20, 1500, 64, torch.bfloat16
    pairs = []
    for i in range(2):
        g = torch.Generator(device=dev).manual_seed(a.seed + 700 + i)
        ks = [torch.randn(h, t, d, generator=g, device=dev, dtype=dt) for _ in range(L)]
        vs = [torch.randn(h, t, d, generator=g, device=dev, dtype=dt) for _ in range(L)]
        pairs.append((ks, vs, torch.empty(L, 2, h, t, d, device=dev, dtype=dt)))
    fns = [lambda pr=pr: native.copy_cross_kv(pr[0], pr[1], pr[2], t) for pr in pairs]
    us = graph_launch_us(torch, fns, per_fn=4, replays=5)
    ks, vs, dst = pairs[0]
    if not (torch.equal(dst[0, 0], ks[0]) and torch.equal(dst[L - 1, 1], vs[L - 1])):
        raise RuntimeError("large_v3_cross_copy: slot contents differ from the sources")
    byts = 2 * L * 2 * h * t * d * 2
    del pairs, fns, ks, vs, dst
    torch.cuda.empty_cache()
    return {"shape": "bf16, one request's 32 layers x (K, V) x 20 heads x 1500 positions x 64 into its decode slot",
            "avg_launch_us": round(us, 3), "algorithmic_bytes_per_launch": byts,
            "achieved_GBps": round(byts / (us * 1e-6) / 1e9, 1), "frac": round(byts / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def large_v3_argmax(torch, native, dev, a):
    """Greedy token selection of a large-v3 decode step: the first maximum of each of 64 rows of
    51866 bf16 logits (the LM head's output, which the decode reads right after writing it, so it
    is timed cache-resident), with the slot feedback the graph decode uses (next-step tokens, EOS
    flags and count). Bytes: the logits read plus the token outputs."""
    rows, vocab = 64, 51866
    g = torch.Generator(device=dev).manual_seed(a.seed + 600)
    logits = torch.randn(rows, vocab, generator=g, device=dev, dtype=torch.bfloat16)
    out = torch.empty(rows, dtype=torch.int64, device=dev)
    row_slots = torch.arange(rows, dtype=torch.int32, device=dev)
    slot_tokens = torch.zeros(rows, dtype=torch.int64, device=dev)
    slot_eos = torch.full((rows,), 50257, dtype=torch.int64, device=dev)
    slot_finished = torch.zeros(rows, dtype=torch.int32, device=dev)
    finished = torch.zeros(1, dtype=torch.int64, device=dev)
    fns = [lambda: native.argmax(logits, out=out, row_slots=row_slots, slot_tokens=slot_tokens, slot_eos=slot_eos,
                                 slot_finished=slot_finished, finished_count=finished)]
    us = graph_launch_us(torch, fns, per_fn=8, replays=5)
    if not torch.equal(out, torch.argmax(logits.float(), dim=-1)):
        raise RuntimeError("large_v3_argmax: tokens differ from torch.argmax")
    byts = rows * vocab * 2 + rows * 8 * 2
    return {"shape": "bf16, 64 rows x 51866 logits, slot feedback (tokens, EOS flags and count)",
            "avg_launch_us": round(us, 3), "algorithmic_bytes_per_launch": byts,
            "achieved_GBps": round(byts / (us * 1e-6) / 1e9, 1), "frac": round(byts / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def large_v3_decode(torch, dev, a, graph=True):
    """Greedy decode of decode_batch requests x decode_tokens tokens through the scheduler: its captured
    graphs (graph_decode=True), or its eager decode (the reference scheduler's default)."""
    from speech_serving import (BlockManager, DualCacheManager, EncoderBlockManager, MemoryGuard,
                                PhaseAwareSpeechScheduler, WhisperClassSpeechEncoderDecoderModel)
    from speech_serving.phase_aware_scheduler import WHISPER_DEFAULT_PREFIX_TOKENS

    dt, L, dm, h, vocab, t_enc, bs = torch.bfloat16, a.decode_layers, 1280, 20, 51866, 1500, 16
    b, n = a.decode_batch, a.decode_tokens
    model = WhisperClassSpeechEncoderDecoderModel(0, L, h, dm, 128, vocab, head_dim=64).to(dev, dt).eval()
    model.init_normal_(0.02, seed=a.seed, draw_device=str(dev))
    per_req = math.ceil((len(WHISPER_DEFAULT_PREFIX_TOKENS) + n) / bs)
    dec = BlockManager(L, h, 64, bs, num_blocks=b * per_req + 8, dtype=dt, device=str(dev))
    enc = EncoderBlockManager(1, h, 64, bs, num_blocks=8, dtype=dt, device=str(dev))
    sched = PhaseAwareSpeechScheduler(model, DualCacheManager(enc, dec), MemoryGuard(high_water_mark_pct=101.0),
                                      max_batch_size=b, device=str(dev), eos_token_id=-1, graph_decode=graph,
                                      **(dict(graph_readback_k=4, graph_direct_encoder_kv=True, graph_max_enc_len=t_enc)
                                         if graph else {}))
    g = torch.Generator(device=dev).manual_seed(a.seed + 7)
    with torch.no_grad():
        for _ in range(b):
            states = torch.randn(1, t_enc, dm, generator=g, device=dev, dtype=dt)
            sched.submit_encoded(model.project_cross_kv(states),
                                 prompt_token_ids=torch.tensor([WHISPER_DEFAULT_PREFIX_TOKENS]), max_new_tokens=n)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    done = sched.run_until_done()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    decode_tokens = sum(len(r.generated_tokens) - 1 for r in done)  # first token of each comes from prefill
    ok = len(done) == b and all(len(r.generated_tokens) == n for r in done) and dec.allocated_block_count == 0
    res = {
        "workload": f"Whisper-large-v3-shaped greedy decode: {L} layers, d_model {dm}, {h} heads x 64, vocab "
                    f"{vocab}, bf16 N(0,0.02) weights, {b} requests x {n} tokens from the 4-token prompt, "
                    f"{t_enc} N(0,1) encoder positions projected by cross_attn_k/v, block size {bs}, "
                    + (f"graph decode (batch bucket {b}, readback every 4 steps)" if graph else
                       "eager decode (decode_step with a PagedKVCache each step, the reference's default mode)"),
        "decode_tokens_per_s": round(decode_tokens / sched.decode_time_s, 1),
        "ms_per_decode_step": round(sched.decode_time_s / max(sched.decode_steps, 1) * 1e3, 3),
        "decode_steps": sched.decode_steps,
        "decode_tokens": decode_tokens,
        "wall_s_incl_prefill": round(wall, 3),
        "completed_ok": ok,
    }
    del sched, dec, enc
    torch.cuda.empty_cache()
    if graph and not a.no_cpu_baseline:
        res["cpu_baseline"] = decode_cpu_baseline(model, a.seed + 7, b, WHISPER_DEFAULT_PREFIX_TOKENS, 15.0)
    del model
    return res


def large_v3_serving(torch, dev, a):
    """The large-v3 serving scenario: 128 graph slots, a burst of 256 requests x 448 greedy tokens at
    t=0, a decoder pool of 128 x 29 + 100 blocks (the graph path reserves ceil((4 + 448) / 16) = 29
    blocks per request up front), so the second half of the burst is admitted as blocks free up."""
    from speech_serving import (BlockManager, DualCacheManager, EncoderBlockManager, MemoryGuard,
                                PhaseAwareSpeechScheduler, WhisperClassSpeechEncoderDecoderModel)
    from speech_serving.phase_aware_scheduler import WHISPER_DEFAULT_PREFIX_TOKENS

    dt, L, dm, h, vocab, t_enc, bs = torch.bfloat16, a.decode_layers, 1280, 20, 51866, 1500, 16
    slots, burst, n, distinct = 128, 256, a.decode_tokens, 16
    model = WhisperClassSpeechEncoderDecoderModel(0, L, h, dm, 128, vocab, head_dim=64).to(dev, dt).eval()
    model.init_normal_(0.02, seed=a.seed, draw_device=str(dev))
    per_req = math.ceil((len(WHISPER_DEFAULT_PREFIX_TOKENS) + n) / bs)
    pool = slots * per_req + 100
    dec = BlockManager(L, h, 64, bs, num_blocks=pool, dtype=dt, device=str(dev))
    enc = EncoderBlockManager(1, h, 64, bs, num_blocks=8, dtype=dt, device=str(dev))
    # Admission backpressure off: every request queues and waits for a slot and for blocks.
    sched = PhaseAwareSpeechScheduler(model, DualCacheManager(enc, dec), MemoryGuard(high_water_mark_pct=1e9),
                                      max_batch_size=slots, device=str(dev), eos_token_id=-1, graph_decode=True,
                                      graph_readback_k=4, graph_direct_encoder_kv=True, graph_max_enc_len=t_enc)
    g = torch.Generator(device=dev).manual_seed(a.seed + 11)
    with torch.no_grad():
        # The burst shares 16 distinct encoder outputs (each request still gets its own slot copy).
        kvs = [model.project_cross_kv(torch.randn(1, t_enc, dm, generator=g, device=dev, dtype=dt))
               for _ in range(distinct)]
        for i in range(burst):
            sched.submit_encoded(kvs[i % distinct], prompt_token_ids=torch.tensor([WHISPER_DEFAULT_PREFIX_TOKENS]),
                                 max_new_tokens=n)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    peak = 0
    while sched.step():
        peak = max(peak, dec.allocated_block_count)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    done = sched.completed
    generated = sum(len(r.generated_tokens) for r in done)
    decode_tokens = sum(len(r.generated_tokens) - 1 for r in done)
    ok = (len(done) == burst and all(len(r.generated_tokens) == n for r in done) and peak <= pool
          and dec.allocated_block_count == 0 and any(r.graph_slot_reused for r in done))
    res = {
        "workload": f"Whisper-large-v3-shaped serving burst: {L} layers, d_model {dm}, {h} heads x 64, vocab {vocab}, "
                    f"bf16 N(0,0.02) weights, {slots} graph slots (buckets 1/8/16/32/64/128), {burst} requests x "
                    f"{n} tokens submitted at t=0 (4-token prompt, {t_enc} encoder positions, {distinct} distinct "
                    f"N(0,1) encoder outputs), decoder pool {pool} blocks of {bs} (< {burst} x {per_req}), "
                    f"readback every 4 steps",
        "decode_tokens_per_s": round(decode_tokens / sched.decode_time_s, 1),
        "ms_per_decode_step": round(sched.decode_time_s / max(sched.decode_steps, 1) * 1e3, 3),
        "decode_steps": sched.decode_steps,
        "tokens_per_s_incl_admission": round(generated / wall, 1),
        "wall_s": round(wall, 3),
        "peak_blocks": peak,
        "pool_blocks": pool,
        "completed_ok": ok,
    }
    del sched, dec, enc, kvs, model
    torch.cuda.empty_cache()
    return res


def decode_cpu_baseline(model, seed, batch, prompt, budget_s, t_enc=1500):
    """The reference's eager decode on the host at the GPU figure's batch: float32 torch on torch's
    threads (oracle/cpu_path.EagerDecode), the same weights and the same per-request encoder states
    (regenerated from the GPU run's seed, projected on the GPU, copied to host float32). Decode
    tokens/s over the decode steps that fit in budget_s (the prompt's prefill is not timed)."""
    import torch

    from oracle import cpu_path as C

    dev = model.decoder_norm.weight.device
    dm, layers = model.hidden_dim, model.num_decoder_layers
    g = torch.Generator(device=dev).manual_seed(seed)
    shape = (batch, model.num_heads, t_enc, model.head_dim)
    cross = [(torch.empty(shape), torch.empty(shape)) for _ in range(layers)]
    with torch.no_grad():
        for i in range(batch):
            states = torch.randn(1, t_enc, dm, generator=g, device=dev, dtype=model.dtype)
            for l, (k, v) in enumerate(model.project_cross_kv(states)):
                cross[l][0][i].copy_(k[0].float())
                cross[l][1][i].copy_(v[0].float())
    dec = C.Decoder(model.state_dict(), model.num_heads, model.head_dim)
    run = C.EagerDecode(dec, cross, batched=True)
    with torch.no_grad():
        _, steps, busy = run.run(prompt, 64, budget_s=budget_s)
    rec = baseline_record(round(batch * steps / busy, 3), "tokens/s",
                          f"{steps} decode steps of {batch} requests (context {len(prompt) + 1}.."
                          f"{len(prompt) + steps}, {t_enc} encoder positions each, batched as the reference's "
                          f"eager scheduler batches them), {busy / max(steps, 1) * 1e3:.0f} ms per step",
                          batch=batch,
                          context_band=f"short-context sample: the first {steps} of the GPU run's 447 decode steps; "
                                       "the CPU path's per-step cost grows with the context (its self-attention "
                                       "gathers and pads every step), so later steps run slower than this rate")
    del run, dec, cross
    return rec


def tts_decode(torch, dev, a):
    """Streaming multi-codebook TTS on the paged engine: the reference TTS model's default shape
    (4 layers, 4 heads x 64, 4 codebooks, vocab 1024), bf16, 64 concurrent requests with
    32-frame prompts, 256 frames each, block size 16. Admission (prompt prefill of all 64
    requests and their first frame) is timed apart from the steady decode."""
    from speech_serving import BlockManager, StreamingMultiCodebookTTSModel, StreamingTTSEngine

    layers, heads, hidden, books, vocab, bs = 4, 4, 256, 4, 1024, 16
    batch, prompt_len, frames = 64, 32, 256
    model = StreamingMultiCodebookTTSModel(layers, heads, hidden, books, vocab).init_normal_(0.02, seed=a.seed)
    model = model.to(dev, torch.bfloat16).eval()
    g = torch.Generator().manual_seed(a.seed + 7)

    def engine_for(n, f):
        bm = BlockManager(layers, heads, hidden // heads, bs, num_blocks=n * math.ceil((prompt_len + f) / bs),
                          dtype=torch.bfloat16, device=str(dev))
        eng = StreamingTTSEngine(model, bm, max_batch_size=n, device=str(dev))
        for _ in range(n):
            eng.submit(torch.randint(0, vocab, (prompt_len, books), generator=g), max_new_frames=f)
        return eng, bm

    eng, _ = engine_for(4, 8)  # warm-up
    eng.run_until_done()
    eng, bm = engine_for(batch, frames)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    eng.step()  # admission: 64 prefills + first frames, then one decode step
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    steps = 0
    while eng.active or eng.queue:
        eng.step()
        steps += 1
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    done = eng.completed
    ok = len(done) == batch and all(q.generated_count == frames for q in done) and bm.allocated_block_count == 0
    decoded = batch * steps
    cpu = None
    if not a.no_cpu_baseline:
        cpu = tts_cpu_baseline(model, prompt_len, books, vocab, batch, a.seed, 5.0)
    return {"workload": f"StreamingTTSEngine, bf16, {layers} layers, d_model {hidden}, {heads} heads x "
                        f"{hidden // heads}, {books} codebooks x vocab {vocab}, {batch} requests x {frames} frames "
                        f"from {prompt_len}-frame prompts, block size {bs}",
            "decode_frames_per_s": round(decoded / (t2 - t1), 1),
            "decode_codebook_tokens_per_s": round(decoded * books / (t2 - t1), 1),
            "ms_per_decode_step": round((t2 - t1) / steps * 1e3, 3), "decode_steps": steps,
            "admission_s": round(t1 - t0, 3), "completed_ok": ok, "cpu_baseline": cpu}


def tts_cpu_baseline(model, prompt_len, books, vocab, batch, seed, budget_s):
    """The reference TTS engine's step on the host: each active request in turn gathers its past from
    the pool, runs one frame and scatters its new K/V (oracle/cpu_path.tts_step), float32 torch on
    torch's threads, the GPU run's weights and batch; decode frames/s over the engine steps that fit
    in budget_s (the prompts' prefill is not timed)."""
    import torch

    from oracle import cpu_path as C

    m = C.TTSModel(model.state_dict(), model.num_heads, model.head_dim)
    bs, frames_cap = 16, 256
    per = -(-(prompt_len + frames_cap) // bs)
    h, d = model.num_heads, model.head_dim
    pools = [(torch.zeros(batch * per, bs, h, d), torch.zeros(batch * per, bs, h, d)) for _ in range(m.core.n)]
    g = torch.Generator().manual_seed(seed)
    state = []
    with torch.no_grad():
        for r in range(batch):  # prefill (not timed): the prompt's K/V into the request's blocks
            table = list(range(r * per, (r + 1) * per))
            logits, kv = m.forward(torch.randint(0, vocab, (1, prompt_len, books), generator=g))
            for (kp, vp), (k, v) in zip(pools, kv):
                for pos in range(prompt_len):
                    kp[table[pos // bs], pos % bs] = k[0, :, pos]
                    vp[table[pos // bs], pos % bs] = v[0, :, pos]
            state.append([table, prompt_len, logits[0, -1].argmax(-1)])
        steps, busy = 0, 0.0
        while busy < budget_s and steps < frames_cap - 1:
            t0 = time.perf_counter()
            for st in state:
                st[2] = C.tts_step(m, pools, st[0], st[1], st[2][None, None])
                st[1] += 1
            steps += 1
            busy += time.perf_counter() - t0
    return baseline_record(round(batch * steps / busy, 2), "frames/s",
                           f"{steps} engine steps over {batch} requests one at a time (context {prompt_len}.."
                           f"{prompt_len + steps}), {busy / max(steps, 1) * 1e3:.1f} ms per engine step")


def config1_decode(torch, dev, a):
    """Config 1: the Whisper-tiny-shaped decoder (4 layers, d_model 384, 4 heads x 64, vocab 51865,
    float32 N(0, 0.02) weights), 4 requests with 1500 N(0,1) encoder positions projected by
    cross_attn_k/v, 64 greedy tokens each from the 4-token prompt, block size 16: decode tokens/s of
    the scheduler's graph decode and eager decode on the GPU, and of the reference's eager path on
    the host (float32 torch, oracle/cpu_path.EagerDecode) with the same weights and encoder K/V."""
    from speech_serving import (BlockManager, DualCacheManager, EncoderBlockManager, MemoryGuard,
                                PhaseAwareSpeechScheduler, WhisperClassSpeechEncoderDecoderModel)
    from speech_serving.phase_aware_scheduler import WHISPER_DEFAULT_PREFIX_TOKENS

    from oracle import cpu_path as C

    L, dm, h, vocab, b, n, t_enc = 4, 384, 4, 51865, 4, 64, 1500
    model = WhisperClassSpeechEncoderDecoderModel(1, L, h, dm, 80, vocab, head_dim=64)
    model = model.init_normal_(0.02, seed=a.seed + 1, draw_device=str(dev)).to(dev).eval()
    g = torch.Generator(device=dev).manual_seed(a.seed + 2)
    with torch.no_grad():
        kvs = [model.project_cross_kv(torch.randn(1, t_enc, dm, generator=g, device=dev)) for _ in range(b)]
    out = {"workload": f"Whisper-tiny-shaped decoder: {L} layers, d_model {dm}, {h} heads x 64, vocab {vocab}, "
                       f"fp32 N(0,0.02) weights, {b} requests x {n} greedy tokens from the 4-token prompt, {t_enc} "
                       f"N(0,1) encoder positions projected by cross_attn_k/v, block size 16"}
    tokens = {}
    for mode in ("graph", "eager"):
        dec = BlockManager(L, h, 64, 16, num_blocks=b * 5 + 8, dtype=torch.float32, device=str(dev))
        enc = EncoderBlockManager(1, h, 64, 16, num_blocks=8, dtype=torch.float32, device=str(dev))
        kw = dict(graph_decode=True, graph_readback_k=4, graph_direct_encoder_kv=True, graph_max_enc_len=t_enc) \
            if mode == "graph" else {}
        best = None
        for _ in range(2):  # the better of two runs: the first also pays one-time warm-up
            sched = PhaseAwareSpeechScheduler(model, DualCacheManager(enc, dec), MemoryGuard(high_water_mark_pct=1e9),
                                              max_batch_size=b, device=str(dev), eos_token_id=-1, **kw)
            for kv in kvs:
                sched.submit_encoded(kv, prompt_token_ids=torch.tensor([WHISPER_DEFAULT_PREFIX_TOKENS]),
                                     max_new_tokens=n)
            torch.cuda.synchronize()
            done = sorted(sched.run_until_done(), key=lambda r: r.id)
            rate = sum(len(r.generated_tokens) - 1 for r in done) / sched.decode_time_s
            best = rate if best is None else max(best, rate)
            tokens[mode] = [r.generated_tokens for r in done]
        out[f"{mode}_decode_tokens_per_s"] = round(best, 1)
    out["graph_tokens_equal_eager"] = tokens["graph"] == tokens["eager"]
    if not a.no_cpu_baseline:
        cross = [[(k.float().cpu(), v.float().cpu()) for k, v in kv] for kv in kvs]
        run = C.EagerDecode(C.Decoder(model.state_dict(), h, 64), cross)
        with torch.no_grad():
            cpu_toks, steps, busy = run.run(WHISPER_DEFAULT_PREFIX_TOKENS, n)
        out["cpu_tokens_equal_gpu"] = cpu_toks == tokens["eager"]
        out["cpu_baseline"] = baseline_record(round(b * steps / busy, 2), "tokens/s",
                                              f"{steps} decode steps of the {b} requests (all {n} tokens)")
    del model, kvs
    torch.cuda.empty_cache()
    return out


def main():
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU only; multi-GPU runs are not part of it",
                          "n_gpus": a.gpus}))
        sys.exit(2)
    import torch

    from speech_serving import native

    if not torch.cuda.is_available():
        raise RuntimeError("bench.py needs a HIP GPU")
    if a.mode == "copy":
        copy_calibration(a)
        return
    dev = torch.device("cuda", 0)
    if a.mode == "decode":  # the large-v3-shaped greedy decode alone (for kernel traces of the decode step)
        native.lib()
        print(json.dumps({"large_v3_decode": large_v3_decode(torch, dev, a)}))
        return
    if a.mode == "decode-eager":  # the same decode in the scheduler's eager mode
        native.lib()
        print(json.dumps({"large_v3_decode_eager": large_v3_decode(torch, dev, a, graph=False)}))
        return
    if a.mode == "serving":  # the large-v3 serving burst alone
        native.lib()
        print(json.dumps({"large_v3_serving": large_v3_serving(torch, dev, a)}))
        return
    if a.mode == "tts":  # the streaming TTS engine alone
        native.lib()
        print(json.dumps({"tts_decode": tts_decode(torch, dev, a)}))
        return
    if a.mode == "prefill":  # the prompt prefill's cross-attention alone
        native.lib()
        print(json.dumps({"large_v3_prefill_cross_attention": large_v3_prefill_cross(torch, native, dev, a),
                          "large_v3_encoder_attention": large_v3_encoder_attention(torch, native, dev, a)}))
        return
    if a.mode == "copies":  # the large-v3 append, gather, slot handoff copy and argmax alone
        native.lib()
        res = large_v3_append_gather(torch, native, dev, a)
        res["large_v3_cross_copy"] = large_v3_cross_copy(torch, native, dev, a)
        res["large_v3_argmax"] = large_v3_argmax(torch, native, dev, a)
        print(json.dumps(res))
        return
    if a.mode == "config1":  # the Whisper-tiny config-1 decode alone
        native.lib()
        print(json.dumps({"config1_decode": config1_decode(torch, dev, a)}))
        return
    dtype = torch.float16
    scale = 1.0 / math.sqrt(a.head_dim)
    native.lib()
    # The large-v3 kernel legs run first, while the process holds only their own allocations: the
    # same large-v3 paged launch measured up to 4% slower after the engine runs (models, pools and
    # captured graphs that come and go) and ~1% slower after the fp16 microbench sets.
    legs = {}
    if not a.no_large_v3:
        legs.update(large_v3_kernels(torch, native, dev, a))
        legs.update(large_v3_append_gather(torch, native, dev, a))
        legs["large_v3_prefill_cross_attention"] = large_v3_prefill_cross(torch, native, dev, a)
        legs["large_v3_encoder_attention"] = large_v3_encoder_attention(torch, native, dev, a)
        legs["large_v3_argmax"] = large_v3_argmax(torch, native, dev, a)
        legs["large_v3_cross_copy"] = large_v3_cross_copy(torch, native, dev, a)

    sets = paged_sets(torch, native, dev, dtype, a.batch, a.heads, a.head_dim, a.block_size, a.pool_blocks,
                      a.max_ctx, a.seed, a.chunk)
    nsets = len(sets)

    def step(s, longest_first=True):
        native.paged_attention(s.q, s.k_pool, s.v_pool, s.tables, s.ctx_dev, a.max_ctx, scale, out=s.out,
                               chunk_tokens=a.chunk, k_new=s.k_new, v_new=s.v_new, rows_longest_first=longest_first)

    # Steps run as captured graphs of back-to-back launches, as the decode runs them: its graph of one
    # token step holds one attention launch per decoder layer (32 at large-v3). graphs[n] holds n steps
    # cycling through the sets (step j on set j mod nsets), so K steps are K // GRAPH_STEPS replays of
    # graphs[GRAPH_STEPS] plus one replay of graphs[K mod GRAPH_STEPS].
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for s in sets:
            step(s)
    torch.cuda.current_stream().wait_stream(stream)
    graphs = {}
    for n in sorted({GRAPH_STEPS, a.steps % GRAPH_STEPS, a.warmup % GRAPH_STEPS} - {0}):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for j in range(n):
                step(sets[j % nsets])
        graphs[n] = g
    torch.cuda.synchronize()

    def run_steps(k):
        """Replays k steps; returns the algorithmic bytes they move."""
        for _ in range(k // GRAPH_STEPS):
            graphs[GRAPH_STEPS].replay()
        if k % GRAPH_STEPS:
            graphs[k % GRAPH_STEPS].replay()
        per_graph = [sum(sets[j % nsets].bytes for j in range(n)) for n in (GRAPH_STEPS, k % GRAPH_STEPS)]
        return (k // GRAPH_STEPS) * per_graph[0] + per_graph[1]

    run_steps(a.warmup)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    moved = run_steps(a.steps)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall / a.steps * 1e3
    value = moved / wall / 1e9

    # Roofline of the dominant (and only) kernel: HIP events around replays of a graph of
    # back-to-back launches on the replay stream.
    avg_us = graph_launch_us(torch, [lambda s=s: step(s) for s in sets])
    avg_bytes = sum(s.bytes for s in sets) / nsets
    achieved = avg_bytes / (avg_us * 1e-6) / 1e9
    # The same longest-first rows without the flag: the launch checks their order itself.
    unflagged_us = graph_launch_us(torch, [lambda s=s: step(s, False) for s in sets])

    # Correctness guard on the measured data: one set against the oracle.
    import numpy as np

    from oracle import paged_kv as O

    s = sets[0]
    step(s)  # appends the same rows again: the pool is unchanged
    torch.cuda.synchronize()
    want = O.paged_attention(s.q.double().cpu().numpy()[:, None], s.k_pool.double().cpu().numpy(),
                             s.v_pool.double().cpu().numpy(), s.tables_cpu.numpy(), s.ctx.tolist(), scale)[:, 0]
    max_err = float(np.abs(s.out.double().cpu().numpy() - want).max())

    result = {
        "metric": "decode tokens/sec + paged-attn achieved HBM GB/s (% of peak), 1 GPU",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic N(0,1) q/k/v, seeded",
        "config": {
            "workload": "paged decode attention microbench: fused append + paged attention, fp16, "
                        f"{a.heads} heads x {a.head_dim}, 1 layer, block size {a.block_size}, batch {a.batch}, "
                        f"ctx U[1,{a.max_ctx}], {a.pool_blocks}-block pool with seeded permuted tables",
            "batch": a.batch,
            "heads": a.heads,
            "head_dim": a.head_dim,
            "block_size": a.block_size,
            "pool_blocks": a.pool_blocks,
            "max_ctx": a.max_ctx,
            "rotating_sets": nsets,
            "step_launch": f"captured graphs of {GRAPH_STEPS} back-to-back steps cycling the {nsets} sets, as the "
                           "decode replays one attention launch per layer in its graph of a token step",
            "rows": "longest-first, flagged SKV_ATTN_ROWS_LONGEST_FIRST (the graph decode's batch layout)",
            "chunk_tokens": a.chunk or native.default_chunk_tokens(a.batch, a.heads, a.head_dim, a.max_ctx, dtype),
            "library": native.version(),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(a, native.library_digest(native.lib())),
            "traffic_source": "rocprofv3 FETCH_SIZE+WRITE_SIZE per launch, scaled by a known-size copy "
                              "(profiles/paged_attention_config2.md), used only when measured with a library "
                              "of the same source digest (else null)",
            "kernel": "attention_kernel<fp16, D=64, paged> with fused append",
            "avg_launch_us": round(avg_us, 3),
            "algorithmic_bytes_per_launch": int(avg_bytes),
        },
        "max_abs_err_vs_oracle": max_err,
    }
    if not a.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(sets[0], a, scale, a.cpu_seconds)
    del sets, graphs
    torch.cuda.empty_cache()
    # The same workload with the rows in drawn order, for comparison.
    sets = paged_sets(torch, native, dev, dtype, a.batch, a.heads, a.head_dim, a.block_size, a.pool_blocks,
                      a.max_ctx, a.seed, a.chunk, sorted_rows=False)
    un_us = graph_launch_us(torch, [lambda s=s: step(s, False) for s in sets])
    result["roofline"]["longest_first_unflagged_avg_launch_us"] = round(unflagged_us, 3)
    result["roofline"]["longest_first_unflagged_frac"] = round(avg_bytes / (unflagged_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
                                                               4)
    result["roofline"]["unsorted_rows_avg_launch_us"] = round(un_us, 3)
    result["roofline"]["unsorted_rows_frac"] = round(sum(s.bytes for s in sets) / len(sets) / (un_us * 1e-6) / 1e9
                                                     / HBM_PEAK_GBS, 4)
    del sets
    torch.cuda.empty_cache()
    result.update(legs)
    # The host-bound TTS step runs before the large-v3 decode, whose CPU baseline leaves the host busy
    # freeing several GB of float64 weights.
    if not a.no_tts:
        result["tts_decode"] = tts_decode(torch, dev, a)
    if not a.no_config1:
        result["config1_decode"] = config1_decode(torch, dev, a)
    if not a.no_large_v3:
        if not a.no_decode:
            result["large_v3_decode"] = large_v3_decode(torch, dev, a)
            result["large_v3_decode_eager"] = large_v3_decode(torch, dev, a, graph=False)
        if not a.no_serving:
            result["large_v3_serving"] = large_v3_serving(torch, dev, a)
    # Free the legs' host and device memory before the line is printed, so the process ends promptly.
    import gc

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
