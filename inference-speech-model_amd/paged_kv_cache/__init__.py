"""Import-path compatibility: `from paged_kv_cache.block_manager import BlockManager`
resolves to the decoder pool in speech_serving.block_manager (the reference
ships the same shim at paged_kv_cache/__init__.py:17-24)."""
from speech_serving.block_manager import BlockManager

__all__ = ["BlockManager"]
