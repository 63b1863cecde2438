"""Host logic behind bench.py's JSON line and the documented binding (no GPU):

- roofline.traffic comes from the committed rocprofv3 summary only for the same workload and a library built from
  the same sources (the source digest); any other digest, workload or a forced chunk gives null;
- the algorithmic bytes of a paged attention launch (K/V of every context, q, out, table entries, lengths);
- the ctypes binding shown in the integration guide passes as many arguments as include/speech_kv.h declares."""
import argparse
import math
import os
import re

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def config2(**kw):
    a = dict(batch=64, heads=32, head_dim=64, block_size=16, pool_blocks=4096, max_ctx=448, seed=0, chunk=0)
    a.update(kw)
    return argparse.Namespace(**a)


def committed_line():
    text = open(os.path.join(ROOT, "profiles", "paged_attention_config2.md")).read()
    line = next(l for l in text.splitlines() if l.startswith("traffic_bytes_per_launch="))
    return dict(f.split("=", 1) for f in line.split())


def test_traffic_only_for_the_measured_sources_and_workload():
    fields = committed_line()
    digest = fields["src"]
    assert bench.measured_traffic(config2(), digest) == int(fields["traffic_bytes_per_launch"])
    assert bench.measured_traffic(config2(), "0" * 16) is None        # another build
    assert bench.measured_traffic(config2(batch=32), digest) is None  # another workload
    assert bench.measured_traffic(config2(chunk=256), digest) is None  # a forced chunk launches differently


def test_committed_traffic_is_close_to_the_algorithmic_bytes():
    # The counters read the launch's real HBM traffic: within 1% of the algorithmic bytes (no re-reads).
    fields = committed_line()
    traffic = int(fields["traffic_bytes_per_launch"])
    algorithmic = 117332478  # config 2's realised contexts, as bench.py reports them
    assert abs(traffic / algorithmic - 1.0) < 0.01


def test_attention_bytes_formula():
    ctx, heads, d, elt, bs = [1, 16, 17, 448], 32, 64, 2, 16
    want = 0
    for c in ctx:
        want += 2 * c * heads * d * elt          # K and V rows
        want += 2 * heads * d * elt              # q read, out written
        want += 4 * math.ceil(c / bs) + 4        # table entries, length
    assert bench.attention_bytes(ctx, heads, d, elt, bs) == want


def test_integration_binding_matches_the_header():
    header = open(os.path.join(ROOT, "include", "speech_kv.h")).read()
    i = header.index("skv_paged_attention(")
    declared = header[i + len("skv_paged_attention("):header.index(");", i)].count(",") + 1
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    m = re.search(r"_lib\.skv_paged_attention\.argtypes = \[(.*?)\]\n", doc, re.S)
    assert m, "the integration guide no longer shows the skv_paged_attention binding"
    assert len([x for x in m.group(1).split(",") if x.strip()]) == declared
