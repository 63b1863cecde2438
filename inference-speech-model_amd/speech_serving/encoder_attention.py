"""Non-causal attention over paged encoder K/V (the reference's EncoderAttentionBackend,
speech_serving/encoder_attention.py:22-71).

Every query of every batch row attends all `encoder_seq_len` positions held in
the blocks of one encoder block table. The reference gathers the blocks into a
contiguous copy and runs matmul/softmax/matmul; here the paged attention entry
point reads the blocks through the table itself (one table row shared by the
whole batch, every row's length = encoder_seq_len, no causal mask), so no copy is
made. In fp16/bf16 with head_dim 64 every 16 queries share one read of the blocks
and both products run on the matrix cores.
"""
import math
from typing import List

import torch

from . import native


class EncoderAttentionBackend:
    """Non-causal bidirectional attention over the blocks of an encoder block table."""

    @staticmethod
    def forward(
        query: torch.Tensor,
        encoder_block_table: List[int],
        key_pool_layer: torch.Tensor,
        value_pool_layer: torch.Tensor,
        encoder_seq_len: int,
        block_size: int = 16,
    ) -> torch.Tensor:
        """softmax(q K^T / sqrt(D)) V over the first encoder_seq_len positions of the table's blocks.

        query: [batch, heads, q_len, head_dim]; key/value_pool_layer: [num_blocks, BS, heads, head_dim]
        (the pool's own block size is used; `block_size` is kept for the reference's signature).
        Returns [batch, heads, q_len, head_dim]; zeros when the table is empty or the length is 0.
        """
        if not encoder_block_table or encoder_seq_len <= 0:
            return torch.zeros_like(query)
        if query.dim() != 4:
            raise RuntimeError(f"EncoderAttentionBackend: query must be [B, H, Q, D], got {tuple(query.shape)}")
        batch, _, _, head_dim = query.shape
        bs = key_pool_layer.shape[1]
        # As the reference's view(-1, H, D)[:encoder_seq_len]: at most the table's capacity.
        seq = min(int(encoder_seq_len), len(encoder_block_table) * bs)
        dev = query.device
        table = torch.tensor([list(encoder_block_table)], dtype=torch.int32, device=dev)
        rows = torch.zeros(batch, dtype=torch.int32, device=dev)
        lens = torch.full((batch,), seq, dtype=torch.int32, device=dev)
        out = native.paged_attention(query.transpose(1, 2), key_pool_layer, value_pool_layer, table, lens, seq,
                                     1.0 / math.sqrt(head_dim), causal=False, table_rows=rows)
        return out.transpose(1, 2).contiguous()
