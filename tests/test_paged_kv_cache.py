"""Host logic of the paged KV cache mirror (nano_sglang/engine/paged_kv_cache.py
semantics plus reserve / truncate / slots)."""
import pytest
import torch

from nanosglang_amd.engine.paged_kv_cache import BlockManager, BlockTable, PagedKVCache


def _kv(n=10, P=4):
    return PagedKVCache(BlockManager(n, P, num_layers=2, num_kv_heads=2, head_dim=8,
                                     dtype=torch.float32, device="cpu"))


def test_layout_and_lifo_allocation():
    kv = _kv()
    bm = kv.block_manager
    assert bm.k_cache.shape == (2, 10, 4, 2, 8)
    assert bm.memory_bytes == 2 * 2 * 10 * 4 * 2 * 8 * 4
    t = kv.allocate_for_request(9)                  # 3 blocks, popped from the end
    assert t.block_indices == [9, 8, 7] and bm.num_free_blocks == 7
    kv.free_request(t)
    assert t.block_indices == [] and bm.num_free_blocks == 10


def test_exhaustion_raises_runtime_error():
    kv = _kv(n=3)
    kv.allocate_for_request(8)
    with pytest.raises(RuntimeError, match="Need 1 blocks but only 1 free|Need"):
        kv.allocate_for_request(5)
    t = BlockTable()
    with pytest.raises(RuntimeError):
        kv.reserve(t, 9)                            # all-or-nothing
    assert t.block_indices == []


def test_reserve_truncate_slots():
    kv = _kv()
    t = kv.allocate_for_request(5)                  # positions 0..4 -> 2 blocks
    kv.reserve(t, 5 + 4 + 1)                        # verify window up to position 9
    assert t.num_blocks == 3
    assert kv.slots(t, 7, 3) == [t.block_indices[1] * 4 + 3, t.block_indices[2] * 4 + 0,
                                 t.block_indices[2] * 4 + 1]
    freed = kv.truncate(t, 6)                       # keep positions 0..5
    assert len(freed) == 1 and t.num_blocks == 2
    assert kv.block_manager.num_free_blocks == 8


def test_write_and_read_roundtrip():
    kv = _kv()
    t = BlockTable()
    k = torch.arange(2 * 6 * 8, dtype=torch.float32).view(2, 6, 8)
    for pos in range(6):
        kv.write_kv_token(t, 1, pos, k[:, pos:pos + 1], -k[:, pos:pos + 1])
    rk, rv = kv.get_kv_for_attention(t, 1, 6)
    assert torch.equal(rk, k) and torch.equal(rv, -k)


def test_refcounts():
    bm = _kv().block_manager
    b = bm.allocate()
    bm.increment_ref(b)
    bm.free(b)
    assert b not in bm.free_blocks
    bm.free(b)
    assert b in bm.free_blocks
