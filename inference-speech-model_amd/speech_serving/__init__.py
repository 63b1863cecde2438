"""MI355X-native decoder KV-cache hot path behind the reference engine's
`speech_serving` API (BlockManager, DualCacheManager, GraphDecodeBuffers,
PhaseAwareSpeechScheduler, WhisperClassSpeechEncoderDecoderModel,
StreamingMultiCodebookTTSModel, StreamingTTSEngine).

Attention, paged append, block-table gather and greedy sampling run as
hand-written gfx950 HIP kernels (libspeechkv.so, bound in speech_serving.native).
"""
from .block_manager import BlockManager
from .dual_cache_manager import DualCacheManager
from .encoder_attention import EncoderAttentionBackend
from .encoder_block_manager import EncoderBlockManager
from .graph_decode_buffers import GraphDecodeBuffers
from .memory_guard import MemoryGuard
from .models import (CrossKV, DecoderLayer, PagedKV, StreamingMultiCodebookTTSModel,
                     WhisperClassSpeechEncoderDecoderModel)
from .phase_aware_scheduler import DualCacheRequest, PhaseAwareSpeechScheduler, RequestPhase
from .tts_engine import StreamingTTSEngine, TTSRequest

__all__ = [
    "BlockManager", "DualCacheManager", "EncoderAttentionBackend", "EncoderBlockManager", "GraphDecodeBuffers", "MemoryGuard",
    "CrossKV", "DecoderLayer", "PagedKV", "StreamingMultiCodebookTTSModel", "WhisperClassSpeechEncoderDecoderModel",
    "DualCacheRequest", "PhaseAwareSpeechScheduler", "RequestPhase", "StreamingTTSEngine", "TTSRequest",
]
