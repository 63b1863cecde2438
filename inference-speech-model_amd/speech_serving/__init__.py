"""MI355X-native decoder KV-cache hot path behind the reference engine's
`speech_serving` API (BlockManager, DualCacheManager, GraphDecodeBuffers,
PhaseAwareSpeechScheduler, WhisperClassSpeechEncoderDecoderModel).

Attention, paged append and block-table gather run as hand-written gfx950 HIP
kernels (libspeechkv.so, bound in speech_serving.native).
"""
