"""MI355X-native decoder KV-cache hot path behind the reference engine's
`speech_serving` API (BlockManager, DualCacheManager, GraphDecodeBuffers,
PhaseAwareSpeechScheduler, WhisperClassSpeechEncoderDecoderModel).

Attention, paged append, block-table gather and greedy sampling run as
hand-written gfx950 HIP kernels (libspeechkv.so, bound in speech_serving.native).
"""
from .block_manager import BlockManager
from .dual_cache_manager import DualCacheManager
from .encoder_attention import EncoderAttentionBackend
from .encoder_block_manager import EncoderBlockManager
from .graph_decode_buffers import GraphDecodeBuffers
from .memory_guard import MemoryGuard
from .models import CrossKV, DecoderLayer, PagedKV, WhisperClassSpeechEncoderDecoderModel
from .phase_aware_scheduler import DualCacheRequest, PhaseAwareSpeechScheduler, RequestPhase

__all__ = [
    "BlockManager", "DualCacheManager", "EncoderAttentionBackend", "EncoderBlockManager", "GraphDecodeBuffers", "MemoryGuard",
    "CrossKV", "DecoderLayer", "PagedKV", "WhisperClassSpeechEncoderDecoderModel", "DualCacheRequest",
    "PhaseAwareSpeechScheduler", "RequestPhase",
]
