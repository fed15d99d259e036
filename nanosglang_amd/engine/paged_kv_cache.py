"""Paged KV cache: block pool, block tables and the slot bookkeeping of the
speculative verify step.

Keeps the reference's interface and layout (nano_sglang/engine/
paged_kv_cache.py:24-229):

* ``BlockTable(block_indices)`` (:24-32);
* ``BlockManager(num_blocks, block_size, num_layers, num_kv_heads, head_dim,
  dtype, device)`` owning ``k_cache`` / ``v_cache`` of shape
  ``(num_layers, num_blocks, block_size, num_kv_heads, head_dim)`` -- the
  NHD layout the verify-attention kernel reads (:60-69) -- with a LIFO free
  list, reference counts, ``allocate`` / ``free`` / ``allocate_blocks_for_tokens``
  raising ``RuntimeError`` when the pool runs out (:86-120), ``write_kv`` /
  ``read_kv`` (:122-162) and ``memory_bytes`` (:164-166);
* ``PagedKVCache(block_manager)`` with ``allocate_for_request``,
  ``append_block``, ``free_request``, ``get_kv_for_attention`` and
  ``write_kv_token`` (:174-229).

Additions for the speculative step (the reference's ``reset_draft_cache``
is a no-op, nano_sglang/decode/speculative.py:186-196):

* ``PagedKVCache.reserve(block_table, num_tokens)`` grows a table so that
  positions ``< num_tokens`` have a page -- the rule of
  ``Scheduler.ensure_decode_block`` (nano_sglang/engine/scheduler.py:221-232)
  applied to the k+1 verify positions, but raising instead of stopping
  silently when the pool is exhausted;
* ``PagedKVCache.truncate(block_table, num_tokens)`` is the rollback: after
  the acceptance step keeps ``num_tokens`` positions, pages wholly past them
  return to the pool;
* ``PagedKVCache.slots(block_table, start, count)`` -- flat slots
  ``block[pos // P] * P + pos % P`` (nano_sglang/engine/engine.py:437-443).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass
class BlockTable:
    """Physical block index of every logical block of one request (:24-32)."""
    block_indices: list[int] = field(default_factory=list)

    @property
    def num_blocks(self) -> int:
        return len(self.block_indices)


class BlockManager:
    """Pool of fixed-size KV blocks shared by all layers (:35-171)."""

    def __init__(self, num_blocks: int, block_size: int, num_layers: int, num_kv_heads: int,
                 head_dim: int, dtype: torch.dtype = torch.float16, device: str = "cuda"):
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = device
        shape = (num_layers, num_blocks, block_size, num_kv_heads, head_dim)
        self.k_cache = torch.zeros(shape, dtype=dtype, device=device)
        self.v_cache = torch.zeros(shape, dtype=dtype, device=device)
        self.free_blocks: list[int] = list(range(num_blocks))
        self.ref_counts: dict[int, int] = {}

    @property
    def num_free_blocks(self) -> int:
        return len(self.free_blocks)

    @property
    def num_used_blocks(self) -> int:
        return self.num_blocks - self.num_free_blocks

    def can_allocate(self, num_blocks: int) -> bool:
        return self.num_free_blocks >= num_blocks

    def allocate(self) -> int:
        if not self.free_blocks:
            raise RuntimeError("Out of KV cache blocks!")
        block_id = self.free_blocks.pop()
        self.ref_counts[block_id] = 1
        return block_id

    def free(self, block_id: int) -> None:
        if block_id not in self.ref_counts:
            return
        self.ref_counts[block_id] -= 1
        if self.ref_counts[block_id] <= 0:
            del self.ref_counts[block_id]
            self.free_blocks.append(block_id)

    def increment_ref(self, block_id: int) -> None:
        self.ref_counts[block_id] = self.ref_counts.get(block_id, 0) + 1

    def free_block_table(self, block_table: BlockTable) -> None:
        for block_id in block_table.block_indices:
            self.free(block_id)
        block_table.block_indices.clear()

    def allocate_blocks_for_tokens(self, num_tokens: int) -> list[int]:
        num_needed = (num_tokens + self.block_size - 1) // self.block_size
        if not self.can_allocate(num_needed):
            raise RuntimeError(f"Need {num_needed} blocks but only {self.num_free_blocks} free")
        return [self.allocate() for _ in range(num_needed)]

    def write_kv(self, block_id: int, layer_idx: int, slot_offset: int, k: torch.Tensor,
                 v: torch.Tensor) -> None:
        """k, v: (num_kv_heads, num_tokens, head_dim) -> NHD rows (:122-137)."""
        n = k.shape[1]
        self.k_cache[layer_idx, block_id, slot_offset:slot_offset + n] = k.transpose(0, 1)
        self.v_cache[layer_idx, block_id, slot_offset:slot_offset + n] = v.transpose(0, 1)

    def read_kv(self, block_ids: list[int], layer_idx: int, total_tokens: int):
        """(num_kv_heads, total_tokens, head_dim) K and V (:139-162)."""
        P = self.block_size
        need = (total_tokens + P - 1) // P
        idx = torch.as_tensor(block_ids[:need], device=self.k_cache.device)
        k = self.k_cache[layer_idx, idx].reshape(-1, self.num_kv_heads, self.head_dim)
        v = self.v_cache[layer_idx, idx].reshape(-1, self.num_kv_heads, self.head_dim)
        return k[:total_tokens].transpose(0, 1), v[:total_tokens].transpose(0, 1)

    @property
    def memory_bytes(self) -> int:
        return (self.k_cache.nelement() + self.v_cache.nelement()) * self.k_cache.element_size()

    def __repr__(self) -> str:
        used = self.num_blocks - self.num_free_blocks
        return (f"<BlockManager {used}/{self.num_blocks} pages in use, {self.block_size} "
                f"tokens per page, {self.memory_bytes / 2**30:.2f} GiB of K/V>")


class PagedKVCache:
    """Request-level view of a BlockManager (:174-229) plus the speculative
    step's reserve / truncate / slots."""

    def __init__(self, block_manager: BlockManager):
        self.block_manager = block_manager

    def allocate_for_request(self, num_tokens: int) -> BlockTable:
        return BlockTable(block_indices=self.block_manager.allocate_blocks_for_tokens(num_tokens))

    def append_block(self, block_table: BlockTable) -> int:
        block_id = self.block_manager.allocate()
        block_table.block_indices.append(block_id)
        return block_id

    def free_request(self, block_table: BlockTable) -> None:
        self.block_manager.free_block_table(block_table)

    def get_kv_for_attention(self, block_table: BlockTable, layer_idx: int, total_tokens: int):
        return self.block_manager.read_kv(block_table.block_indices, layer_idx, total_tokens)

    def write_kv_token(self, block_table: BlockTable, layer_idx: int, seq_position: int,
                       k: torch.Tensor, v: torch.Tensor) -> None:
        P = self.block_manager.block_size
        block_idx, slot = divmod(seq_position, P)
        while block_idx >= len(block_table.block_indices):
            self.append_block(block_table)
        self.block_manager.write_kv(block_table.block_indices[block_idx], layer_idx, slot, k, v)

    # ---- speculative-step bookkeeping ----
    def reserve(self, block_table: BlockTable, num_tokens: int) -> None:
        """Make positions < num_tokens addressable (all-or-nothing)."""
        P = self.block_manager.block_size
        need = (num_tokens + P - 1) // P - len(block_table.block_indices)
        if need <= 0:
            return
        if not self.block_manager.can_allocate(need):
            raise RuntimeError(f"Need {need} blocks but only "
                               f"{self.block_manager.num_free_blocks} free")
        for _ in range(need):
            self.append_block(block_table)

    def truncate(self, block_table: BlockTable, num_tokens: int) -> list[int]:
        """Rollback: free pages wholly past the first num_tokens positions."""
        P = self.block_manager.block_size
        keep = (num_tokens + P - 1) // P
        freed = block_table.block_indices[keep:]
        for b in freed:
            self.block_manager.free(b)
        del block_table.block_indices[keep:]
        return freed

    def slots(self, block_table: BlockTable, start: int, count: int) -> list[int]:
        P = self.block_manager.block_size
        bt = block_table.block_indices
        return [bt[(start + t) // P] * P + (start + t) % P for t in range(count)]
