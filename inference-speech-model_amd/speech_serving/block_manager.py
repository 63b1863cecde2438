"""Decoder paged KV pool: physical blocks, LIFO free list, per-layer pools.

Public interface of the reference's BlockManager
(speech_serving/block_manager.py:33-236): constructor arguments, the
`key_pool[l]` / `value_pool[l]` tensors of shape
[num_blocks, block_size, num_kv_heads, head_dim] (zero-initialised),
allocate_block() (LIFO, RuntimeError when exhausted), free_blocks() (silently
ignores double frees), the counters, get_stats() keys and check_no_leaks().

MI355X layout: all layers' K and V pools are views into ONE zero-filled
allocation [num_layers, 2, num_blocks, block_size, num_kv_heads, head_dim], so
a token row of one layer (num_kv_heads * head_dim elements) is contiguous and
every block is block_size such rows back to back. The decode kernels read
these pools directly through per-request block tables.
"""
from __future__ import annotations

from typing import Any, Dict, List, Optional, Sequence

import torch


def _element_size(dtype: torch.dtype) -> int:
    return torch.empty((), dtype=dtype).element_size()


class BlockManager:
    """Fixed pool of decoder KV blocks (one block = block_size tokens of every layer)."""

    def __init__(
        self,
        num_layers: int,
        num_kv_heads: int,
        head_dim: int,
        block_size: int,
        num_blocks: Optional[int] = None,
        dtype: torch.dtype = torch.float16,
        device: str = "cuda",
    ):
        for name, val in (("num_layers", num_layers), ("num_kv_heads", num_kv_heads), ("head_dim", head_dim),
                          ("block_size", block_size)):
            if val <= 0:
                raise ValueError(f"{name} must be > 0, got {val}")
        if isinstance(dtype, str):
            dtype = getattr(torch, dtype)
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.dtype = dtype
        self.device = device

        if num_blocks is None:
            num_blocks = self._auto_num_blocks()
        if num_blocks <= 0:
            raise ValueError(f"num_blocks must be > 0, got {num_blocks}")
        self.num_blocks = num_blocks

        self.arena = torch.zeros((num_layers, 2, num_blocks, block_size, num_kv_heads, head_dim), dtype=dtype,
                                 device=device)
        self.key_pool: List[torch.Tensor] = [self.arena[l, 0] for l in range(num_layers)]
        self.value_pool: List[torch.Tensor] = [self.arena[l, 1] for l in range(num_layers)]

        # LIFO free list: allocate_block() pops the highest free id first.
        self._free_list: List[int] = list(range(num_blocks))
        self._allocated: set = set()

    # ------------------------------------------------------------------ sizing
    def block_bytes(self) -> int:
        """Bytes of one block across all layers, K and V."""
        return (self.num_layers * 2 * self.block_size * self.num_kv_heads * self.head_dim
                * _element_size(self.dtype))

    def _auto_num_blocks(self) -> int:
        """40% of the free device memory (at least 64 blocks); 512 blocks off-GPU."""
        if not torch.cuda.is_available() or str(self.device) == "cpu":
            return 512
        free, _total = torch.cuda.mem_get_info(torch.device(self.device))
        return int(max(64, int(free * 0.40) // self.block_bytes()))

    # ------------------------------------------------------------------ allocation
    def allocate_block(self) -> int:
        """Take one free block id (LIFO). Raises RuntimeError when none is left."""
        if not self._free_list:
            raise RuntimeError(
                f"BlockManager: out of physical blocks! All {self.num_blocks} blocks are allocated.")
        blk = self._free_list.pop()
        self._allocated.add(blk)
        return blk

    def free_blocks(self, block_ids: Sequence[int]) -> None:
        """Return blocks to the pool; ids that are not allocated are ignored."""
        for blk in block_ids:
            if blk in self._allocated:
                self._allocated.remove(blk)
                self._free_list.append(blk)

    @property
    def allocated_block_count(self) -> int:
        return len(self._allocated)

    @property
    def num_free_blocks(self) -> int:
        return len(self._free_list)

    # ------------------------------------------------------------------ paging helpers
    def slot(self, block_table: Sequence[int], position: int) -> int:
        """Pool slot of token `position` of a request: block * block_size + offset."""
        return int(block_table[position // self.block_size]) * self.block_size + position % self.block_size

    def blocks_for(self, num_tokens: int) -> int:
        return (num_tokens + self.block_size - 1) // self.block_size

    def gather(self, layer: int, block_tables: torch.Tensor, lens: torch.Tensor, max_len: int):
        """Contiguous zero-padded [B, H, max_len, D] K and V of `layer` (HIP gather kernel)."""
        from . import native

        return native.gather(self.key_pool[layer], self.value_pool[layer], block_tables, lens, max_len)

    # ------------------------------------------------------------------ telemetry
    def get_stats(self) -> Dict[str, Any]:
        allocated = self.allocated_block_count
        util = round(allocated / self.num_blocks * 100.0, 2) if self.num_blocks > 0 else 0.0
        return {
            "num_blocks": self.num_blocks,
            "allocated_blocks": allocated,
            "free_blocks": self.num_free_blocks,
            "utilization_pct": util,
            "pool_memory_mb": round(self.num_blocks * self.block_bytes() / (1024 ** 2), 2),
        }

    def check_no_leaks(self) -> bool:
        return self.allocated_block_count == 0

    def __repr__(self) -> str:
        s = self.get_stats()
        return (f"BlockManager(layers={self.num_layers}, heads={self.num_kv_heads}, head_dim={self.head_dim}, "
                f"block_size={self.block_size}, blocks={s['allocated_blocks']}/{self.num_blocks} "
                f"({s['utilization_pct']}% used), dtype={self.dtype}, device={self.device})")
