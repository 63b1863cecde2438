"""Encoder KV pool with reference counting and content-hash block sharing.

Same public interface as the reference's EncoderBlockManager
(speech_serving/encoder_block_manager.py:17-221): FIFO free list,
allocate_block(content_hash) -> (block_id, hit), release_block(s),
store_encoder_kv(), ref_counts, hit_rate, get_stats(). The encoder phase is
not on the decoder KV-cache hot path; this pool exists so DualCacheManager and
the scheduler keep their API. Its writes and reads go through the same HIP
append / gather kernels as the decoder pool.
"""
from __future__ import annotations

import collections
from typing import Any, Dict, List, Optional, Tuple

import torch


class EncoderBlockManager:
    def __init__(
        self,
        num_layers: int,
        num_heads: int,
        head_dim: int,
        block_size: int = 16,
        num_blocks: Optional[int] = None,
        gpu_memory_utilization: float = 0.85,
        dtype: torch.dtype = torch.float16,
        device: str = "cuda",
    ):
        if isinstance(dtype, str):
            dtype = getattr(torch, dtype)
        self.num_layers = num_layers
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.dtype = dtype
        self.device = device
        self.gpu_memory_utilization = gpu_memory_utilization
        elt = torch.empty((), dtype=dtype).element_size()
        self.bytes_per_token = num_layers * 2 * num_heads * head_dim * elt
        self.bytes_per_block = self.bytes_per_token * block_size
        if num_blocks is None:
            if torch.cuda.is_available() and str(device) != "cpu":
                free, _ = torch.cuda.mem_get_info(torch.device(device))
                num_blocks = max(64, int(free * gpu_memory_utilization) // self.bytes_per_block)
            else:
                num_blocks = 512
        self.num_blocks = int(num_blocks)
        self.available_kv_memory_bytes = self.num_blocks * self.bytes_per_block
        self.arena = torch.zeros((num_layers, 2, self.num_blocks, block_size, num_heads, head_dim), dtype=dtype,
                                 device=device)
        self.key_pool: List[torch.Tensor] = [self.arena[l, 0] for l in range(num_layers)]
        self.value_pool: List[torch.Tensor] = [self.arena[l, 1] for l in range(num_layers)]
        self._free: collections.deque = collections.deque(range(self.num_blocks))
        self.ref_counts: Dict[int, int] = {i: 0 for i in range(self.num_blocks)}
        self.prefix_hash_table: Dict[str, int] = {}
        self.block_to_hash: Dict[int, str] = {}
        self.retained_caches: Dict[str, List[int]] = {}
        self.total_lookups = 0
        self.cache_hits = 0

    @property
    def free_block_list(self) -> List[int]:
        return list(self._free)

    def allocate_block(self, content_hash: Optional[str] = None) -> Tuple[int, bool]:
        """Reuse the block holding `content_hash` if still referenced, else take the oldest free block."""
        self.total_lookups += 1
        if content_hash is not None and content_hash in self.prefix_hash_table:
            blk = self.prefix_hash_table[content_hash]
            if self.ref_counts[blk] > 0:
                self.ref_counts[blk] += 1
                self.cache_hits += 1
                return blk, True
            del self.prefix_hash_table[content_hash]
        if not self._free:
            raise RuntimeError(
                f"encoder KV pool exhausted: no free block among {self.num_blocks} (all are held by "
                "requests or by cached encoder outputs)")
        blk = self._free.popleft()
        self.ref_counts[blk] = 1
        if content_hash is not None:
            self.prefix_hash_table[content_hash] = blk
            self.block_to_hash[blk] = content_hash
        return blk, False

    def release_block(self, blk: int) -> bool:
        """Drop one reference; returns True when the block went back to the free list."""
        if self.ref_counts.get(blk, 0) <= 0:
            return False
        self.ref_counts[blk] -= 1
        if self.ref_counts[blk]:
            return False
        h = self.block_to_hash.pop(blk, None)
        if h is not None:
            self.prefix_hash_table.pop(h, None)
        self._free.append(blk)
        return True

    def release_blocks(self, block_ids: List[int]) -> int:
        return sum(1 for b in block_ids if self.release_block(b))

    def store_encoder_kv(self, block_id: int, layer_idx: int, k_tensor: torch.Tensor, v_tensor: torch.Tensor):
        """Write [tok_count, H, D] rows at the start of `block_id` (HIP append kernel on GPU pools)."""
        from . import native

        n = k_tensor.shape[0]
        kp, vp = self.key_pool[layer_idx], self.value_pool[layer_idx]
        slots = torch.arange(n, dtype=torch.int64, device=kp.device) + block_id * self.block_size
        native.append(k_tensor, v_tensor, kp, vp, slots)

    @property
    def allocated_block_count(self) -> int:
        return self.num_blocks - len(self._free)

    @property
    def num_free_blocks(self) -> int:
        return len(self._free)

    @property
    def hit_rate(self) -> float:
        return round(self.cache_hits / self.total_lookups * 100, 2) if self.total_lookups else 0.0

    def get_stats(self) -> Dict[str, Any]:
        allocated = self.allocated_block_count
        return {
            "num_blocks": self.num_blocks,
            "block_size": self.block_size,
            "allocated_blocks": allocated,
            "free_blocks": self.num_free_blocks,
            "utilization_pct": round(allocated / self.num_blocks * 100, 2) if self.num_blocks else 0.0,
            "total_lookups": self.total_lookups,
            "cache_hits": self.cache_hits,
            "prefix_hit_rate_pct": self.hit_rate,
            "pool_memory_mb": round(self.num_blocks * self.bytes_per_block / (1024 ** 2), 2),
        }
