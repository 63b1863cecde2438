"""Host-side bookkeeping on the CPU: block pools, release paths, admission.

Mirrors the reference's behaviour (speech_serving/block_manager.py:133-226,
encoder_block_manager.py:110-221, dual_cache_manager.py:31-90,
phase_aware_scheduler.py:224-329) and the reference tests
test_empty_pool_admission (test_speech_engine.py:222-235) and the zero-leak
assertions.
"""
import pytest
import torch

from paged_kv_cache.block_manager import BlockManager as ShimBlockManager
from speech_serving.block_manager import BlockManager
from speech_serving.dual_cache_manager import DualCacheManager
from speech_serving.encoder_block_manager import EncoderBlockManager
from speech_serving.memory_guard import MemoryGuard
from speech_serving.models import WhisperClassSpeechEncoderDecoderModel
from speech_serving.phase_aware_scheduler import PhaseAwareSpeechScheduler, WHISPER_DEFAULT_PREFIX_TOKENS


def bm(nb=8, **kw):
    return BlockManager(num_layers=2, num_kv_heads=4, head_dim=16, block_size=8, num_blocks=nb, dtype=torch.float32,
                        device="cpu", **kw)


def test_shim_import_path():
    assert ShimBlockManager is BlockManager


def test_pool_layout_zero_init_and_views():
    b = bm()
    assert len(b.key_pool) == 2 and b.key_pool[0].shape == (8, 8, 4, 16)
    assert all(t.is_contiguous() and not t.any() for t in b.key_pool + b.value_pool)
    b.key_pool[1][3, 2, 1, 5] = 7.0  # views share the one arena
    assert b.arena[1, 0, 3, 2, 1, 5] == 7.0


def test_lifo_allocation_and_exhaustion():
    b = bm(4)
    assert [b.allocate_block() for _ in range(4)] == [3, 2, 1, 0]
    with pytest.raises(RuntimeError, match="out of physical blocks"):
        b.allocate_block()
    b.free_blocks([1, 3])
    assert b.allocate_block() == 3  # last freed is reused first


def test_double_free_and_unknown_ids_are_ignored():
    b = bm(4)
    x = b.allocate_block()
    b.free_blocks([x, x, 99, -1])
    assert b.allocated_block_count == 0 and b.num_free_blocks == 4 and b.check_no_leaks()


def test_stats_keys_and_values():
    b = bm(10)
    for _ in range(3):
        b.allocate_block()
    s = b.get_stats()
    assert s["num_blocks"] == 10 and s["allocated_blocks"] == 3 and s["free_blocks"] == 7
    assert s["utilization_pct"] == 30.0
    assert s["pool_memory_mb"] == round(10 * 8 * 4 * 16 * 2 * 2 * 4 / 2 ** 20, 2)


@pytest.mark.parametrize("arg", ["num_layers", "num_kv_heads", "head_dim", "block_size", "num_blocks"])
def test_constructor_validation(arg):
    kw = dict(num_layers=1, num_kv_heads=1, head_dim=8, block_size=4, num_blocks=4, device="cpu")
    kw[arg] = 0
    with pytest.raises(ValueError):
        BlockManager(**kw)


def test_slot_mapping_helper():
    b = bm()
    assert b.slot([5, 2, 7], 0) == 40 and b.slot([5, 2, 7], 9) == 17 and b.blocks_for(17) == 3


def test_encoder_pool_refcount_and_prefix_sharing():
    e = EncoderBlockManager(num_layers=2, num_heads=4, head_dim=16, block_size=8, num_blocks=4, device="cpu",
                            dtype=torch.float32)
    b1, hit1 = e.allocate_block(content_hash="abc")
    b2, hit2 = e.allocate_block(content_hash="abc")
    assert (b1, hit1) == (0, False) and (b2, hit2) == (0, True) and e.ref_counts[0] == 2
    assert e.hit_rate > 0
    assert not e.release_block(b1) and e.release_block(b2)
    assert e.allocated_block_count == 0
    assert e.allocate_block()[0] == 1  # FIFO free list


def test_dual_cache_release_is_complete():
    e = EncoderBlockManager(2, 4, 16, 8, 8, device="cpu", dtype=torch.float32)
    d = bm(8)
    dc = DualCacheManager(e, d)
    table, hits = dc.allocate_encoder_blocks(20)
    dec = [dc.allocate_decoder_block() for _ in range(3)]
    assert len(table) == 3 and hits == 0
    r = dc.release_request_resources(table, dec)
    assert r == {"freed_encoder_blocks": 3, "freed_decoder_blocks": 3}
    assert e.allocated_block_count == 0 and d.allocated_block_count == 0


def test_dual_cache_encoder_allocation_is_all_or_nothing():
    e = EncoderBlockManager(2, 4, 16, 8, 2, device="cpu", dtype=torch.float32)
    dc = DualCacheManager(e, bm(4))
    with pytest.raises(RuntimeError):
        dc.allocate_encoder_blocks(30)  # needs 4 blocks, pool has 2
    assert e.allocated_block_count == 0


def _cpu_scheduler(enc_blocks=16, dec_blocks=16, hwm=75.0):
    enc = EncoderBlockManager(2, 4, 16, 8, enc_blocks, device="cpu", dtype=torch.float32)
    dec = BlockManager(2, 4, 16, 8, dec_blocks, dtype=torch.float32, device="cpu")
    model = WhisperClassSpeechEncoderDecoderModel(2, 2, 4, 64, 80, 256)
    return PhaseAwareSpeechScheduler(model, DualCacheManager(enc, dec), MemoryGuard(high_water_mark_pct=hwm),
                                     device="cpu"), enc, dec


def test_empty_pool_admission_is_never_rejected():
    sched, _, _ = _cpu_scheduler()
    assert sched.submit(torch.randn(80, 48), max_new_tokens=10) == 0


def test_high_water_mark_rejects_and_counts():
    sched, _, _ = _cpu_scheduler(enc_blocks=8, dec_blocks=8, hwm=50.0)
    # 48 mel frames -> 24 encoder positions -> 3 of 8 blocks (37.5%): admitted
    assert sched.submit(torch.randn(80, 48), max_new_tokens=8) == 0
    # the queued request's blocks count too: 6 of 8 projected -> rejected
    assert sched.submit(torch.randn(80, 48), max_new_tokens=8) is None
    assert sched.rejected_requests_count == 1


def test_default_prompt_and_eos_follow_vocab_size():
    sched, _, _ = _cpu_scheduler()
    sched.submit(torch.randn(80, 16), max_new_tokens=4)
    assert sched.queue[0].prompt_token_ids.tolist() == [[1]] and sched.queue[0].eos_token_id is None
    enc = EncoderBlockManager(2, 4, 16, 8, 16, device="cpu", dtype=torch.float32)
    dec = BlockManager(2, 4, 16, 8, 16, dtype=torch.float32, device="cpu")
    big = WhisperClassSpeechEncoderDecoderModel(1, 1, 4, 64, 80, 51865)
    s2 = PhaseAwareSpeechScheduler(big, DualCacheManager(enc, dec), device="cpu")
    s2.submit(torch.randn(80, 16), max_new_tokens=4)
    assert s2.queue[0].prompt_token_ids.tolist() == [WHISPER_DEFAULT_PREFIX_TOKENS]
    assert s2.queue[0].eos_token_id == 50257


def test_graph_direct_kv_requires_graph_decode():
    enc = EncoderBlockManager(2, 4, 16, 8, 16, device="cpu", dtype=torch.float32)
    dec = BlockManager(2, 4, 16, 8, 16, dtype=torch.float32, device="cpu")
    model = WhisperClassSpeechEncoderDecoderModel(2, 2, 4, 64, 80, 256)
    with pytest.raises(ValueError):
        PhaseAwareSpeechScheduler(model, DualCacheManager(enc, dec), device="cpu", graph_direct_encoder_kv=True)


def test_model_refuses_cpu_attention():
    model = WhisperClassSpeechEncoderDecoderModel(1, 1, 4, 64, 80, 100)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        model.decode_step(torch.tensor([[1, 2]]))


def test_state_dict_names_match_reference_layout():
    model = WhisperClassSpeechEncoderDecoderModel(1, 1, 4, 64, 80, 100)
    keys = set(model.state_dict())
    for k in ["conv1.weight", "conv2.bias", "encoder_layers.0.self_attn_q.weight", "encoder_norm.weight",
              "decoder_embed.weight", "decoder_layers.0.cross_attn_out.weight", "decoder_layers.0.norm3.bias",
              "decoder_layers.0.mlp.0.weight", "decoder_layers.0.mlp.2.bias", "decoder_norm.weight",
              "lm_head.weight"]:
        assert k in keys, k


def test_cross_arena_keeps_live_requests_in_the_leading_slots():
    """The eager encoder K/V arena: requests take slots 0, 1, 2, ...; a released slot is refilled by the
    last live request (its K/V moved, its cross_slot updated), so a batch in slot order is the views
    buf[0:n]; the T dimension grows with the live slots' contents kept."""
    from types import SimpleNamespace

    from speech_serving.phase_aware_scheduler import CrossArena, _slot_runs

    a = CrossArena(4, 2, 2, 8, torch.float32, torch.device("cpu"))
    reqs = [SimpleNamespace(id=i, cross_slot=None) for i in range(4)]
    kvs = []
    for i, r in enumerate(reqs[:3]):
        t = 5 + i
        kv = [(torch.full((1, 2, t, 8), 10.0 * i + l), torch.full((1, 2, t, 8), -10.0 * i - l)) for l in range(2)]
        kvs.append(kv)
        assert a.put(r, kv) == i and r.cross_slot == i
    a.release(reqs[0])  # the last live request moves into slot 0
    assert reqs[0].cross_slot is None and reqs[2].cross_slot == 0 and reqs[1].cross_slot == 1
    assert a.owner == [reqs[2], reqs[1]] and a.lens == [7, 6]
    views = a.views(0, 2, 7, 2)
    for l in range(2):
        assert torch.equal(views[l][0][0], kvs[2][l][0][0]) and torch.equal(views[l][1][0], kvs[2][l][1][0])
        assert torch.equal(views[l][0][1, :, :6], kvs[1][l][0][0])
    a.release(reqs[2])  # releasing the last slot moves nothing
    assert a.owner == [reqs[1]] and reqs[1].cross_slot == 0
    a.release(reqs[2])  # a second release is a no-op
    big = [(torch.ones(1, 2, 1600, 8), torch.ones(1, 2, 1600, 8)) for _ in range(2)]
    assert a.put(reqs[3], big) == 1 and a.max_len >= 1600  # grown, slot 0 kept
    assert torch.equal(a.views(0, 1, 6, 2)[1][0][0], kvs[1][1][0][0])
    with pytest.raises(RuntimeError, match="full"):
        for r in [SimpleNamespace(id=9, cross_slot=None) for _ in range(3)]:
            a.put(r, big)
    # batches split where the slots stop being consecutive
    rs = [SimpleNamespace(s=s) for s in (4, 0, 1, 3, 7, 2)]
    assert [[r.s for r in run] for run in _slot_runs(rs, lambda r: r.s)] == [[0, 1, 2, 3, 4], [7]]


def test_projection_helpers_call_modules_off_the_gpu():
    """On CPU tensors the decode step's projection, MLP and add+LayerNorm helpers run the modules and torch ops
    (the library's GEMM and LayerNorm launches are for GPU tensors only)."""
    import torch.nn as nn

    from speech_serving import models

    torch.manual_seed(0)
    lin = nn.Linear(16, 8)
    x = torch.randn(3, 16)
    assert torch.equal(models.proj(lin, x), lin(x))
    seq = nn.Sequential(nn.Linear(16, 32), nn.GELU(), nn.Linear(32, 16))
    assert torch.equal(models.mlp(seq, x), seq(x))
    norm = nn.LayerNorm(16)
    y = torch.randn(3, 16)
    s, n = models.add_norm(x, y, norm)
    assert torch.equal(s, x + y) and torch.equal(n, norm(x + y))
