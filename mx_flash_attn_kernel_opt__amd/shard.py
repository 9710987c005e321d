"""Sharding one batch's KV pages across devices for long-context decode.

A long sequence's pages can live on several GPUs: each holds a contiguous range of every
sequence's pages, runs ``paged_gqa_decode_partial`` over its own keys, the per-row (o, lse)
pairs are all-gathered, and ``lse_merge`` combines them into the exact single-device output
(the split/combine structure of the reference's split-KV decode, optimized_c500_flash_attn.cu:
537-551 and combine_splits at :666-728, with the splits placed on different devices).

``shard_pages`` computes that layout from one block table: per shard, a block table whose row b
starts at the shard's first page of sequence b, and the number of keys of sequence b the shard
holds.  Computed with device-side integer ops (no host synchronisation).
"""

from __future__ import annotations

import torch


def shard_pages(block_table: torch.Tensor, seq_lens: torch.Tensor, page_size: int,
                num_shards: int, seqlen_q: int = 1) -> list[tuple[torch.Tensor, torch.Tensor]]:
    """Cuts every sequence's pages into ``num_shards`` contiguous ranges.

    Returns ``[(block_table_s, seq_lens_s)]``: block_table_s [B, max_pages] int32 (entries past
    the shard's pages repeat the row's last entry and are never read), seq_lens_s [B] int32.
    Sequence b's keys [0, L_b) are split at page boundaries so that the last shard holds every
    key that a causal mask hides from some of the ``seqlen_q`` query tokens (keys
    >= L_b - seqlen_q + 1): calling the last shard with causal=1 and the others with causal=0
    then reproduces the end-aligned mask of the unsharded call.  The other pages are spread
    evenly; sequences shorter than ``num_shards`` pages leave some shards empty (length 0).
    """
    if num_shards < 1:
        raise ValueError("num_shards must be >= 1")
    if seqlen_q < 1:
        raise ValueError("seqlen_q must be >= 1")
    if block_table.dim() != 2 or seq_lens.shape != (block_table.shape[0],):
        raise ValueError("block_table must be [B, max_pages] and seq_lens [B]")
    P = int(page_size)
    width = block_table.shape[1]
    L = seq_lens.to(torch.int64).clamp(min=0, max=width * P)
    npg = (L + P - 1) // P
    # Pages [cut, npg) hold keys >= L - seqlen_q + 1 and all go to the last shard.
    cut = torch.minimum(npg, (L - seqlen_q + 1).clamp(min=0) // P)
    starts = [(s * cut) // num_shards for s in range(num_shards)] + [npg]
    cols = torch.arange(width, device=block_table.device, dtype=torch.int64)
    out = []
    for s in range(num_shards):
        first, end = starts[s], starts[s + 1]
        idx = (first.unsqueeze(1) + cols.unsqueeze(0)).clamp(max=width - 1)
        table_s = torch.gather(block_table, 1, idx).to(torch.int32).contiguous()
        lens_s = (torch.minimum(end * P, L) - first * P).clamp(min=0).to(torch.int32)
        out.append((table_s, lens_s))
    return out
