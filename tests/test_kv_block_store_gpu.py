"""KVBlockStore over the native store: the reference's tests/test_kv_block_store.py case by case.

Blocks use the reference layout [num_layers, batch, block_len, kv_heads, head_dim] on the GPU.
One difference is by design: a native session has one block length, so the many-moves
accounting case uses equal-sized blocks instead of the reference's 8 + block_id tokens.
"""
from __future__ import annotations

import logging

import pytest
import torch

pytestmark = pytest.mark.gpu


def make_block(*, num_layers=2, batch=1, tokens_per_block=16, kv_heads=2, head_dim=64, fill=0.0):
    shape = (num_layers, batch, tokens_per_block, kv_heads, head_dim)
    key = torch.full(shape, fill, dtype=torch.float16, device="cuda")
    value = torch.full(shape, fill + 0.5, dtype=torch.float16, device="cuda")
    return key, value


def test_offload_to_cpu_raises_when_ram_budget_would_be_exceeded():
    from pager_hf.kv_block_store import KVBlockStore

    store = KVBlockStore(tokens_per_block=16, ram_budget_bytes=1000)
    store.put_gpu(0, *make_block())
    with pytest.raises(RuntimeError, match="ram_budget exceeded"):
        store.ensure_cpu(0)
    assert store.has_gpu(0)
    assert not store.has_cpu(0)
    assert store.resident_cpu_bytes() == 0


def test_offload_to_cpu_succeeds_within_ram_budget():
    from pager_hf.kv_block_store import KVBlockStore

    store = KVBlockStore(tokens_per_block=16, ram_budget_bytes=1_000_000_000)
    store.put_gpu(0, *make_block())
    store.ensure_cpu(0)
    assert store.has_cpu(0)
    assert not store.has_gpu(0)


def test_offload_to_cpu_logs_error_when_ram_budget_exceeded(caplog):
    from pager_hf.kv_block_store import KVBlockStore

    store = KVBlockStore(tokens_per_block=16, ram_budget_bytes=1000)
    store.put_gpu(0, *make_block())
    with caplog.at_level(logging.ERROR, logger="pager_hf.kv_block_store"):
        with pytest.raises(RuntimeError, match="ram_budget exceeded"):
            store.ensure_cpu(0)
    assert any(r.levelno == logging.ERROR and "ram_budget exceeded" in r.message for r in caplog.records)


def test_offload_to_cpu_warns_when_approaching_ram_budget(caplog):
    from pager_hf.kv_block_store import KVBlockStore, kv_nbytes

    key, value = make_block()
    store = KVBlockStore(tokens_per_block=16, ram_budget_bytes=int(kv_nbytes(key, value) / 0.82))
    store.put_gpu(0, key, value)
    with caplog.at_level(logging.WARNING, logger="pager_hf.kv_block_store"):
        store.ensure_cpu(0)
    assert store.has_cpu(0)
    assert any(r.levelno == logging.WARNING and "ram_budget usage" in r.message for r in caplog.records)


def test_offload_to_cpu_ignores_ram_budget_when_unset():
    from pager_hf.kv_block_store import KVBlockStore

    store = KVBlockStore(tokens_per_block=16)
    store.put_gpu(0, *make_block())
    store.ensure_cpu(0)
    assert store.has_cpu(0)


def test_resident_bytes_stay_correct_across_many_moves():
    """Tracked totals match a from-scratch sum over both tiers, and data survives the moves."""
    from pager_hf.kv_block_store import KVBlockStore, kv_nbytes

    store = KVBlockStore(tokens_per_block=16)
    blocks = [make_block(fill=float(b)) for b in range(10)]
    for b, (k, v) in enumerate(blocks):
        store.put_gpu(b, k, v)
    for b in range(0, 10, 2):
        store.offload_to_cpu(b)
    for b in range(0, 10, 4):
        store.load_to_gpu(b, "cuda")
    gpu = sum(kv_nbytes(k, v) for k, v in store.gpu_blocks.values())
    cpu = sum(kv_nbytes(k, v) for k, v in store.cpu_blocks.values())
    assert store.resident_gpu_bytes() == gpu
    assert store.resident_cpu_bytes() == cpu
    assert store.gpu_block_ids() == [0, 1, 3, 4, 5, 7, 8, 9]
    assert store.cpu_block_ids() == [2, 6]
    for b, (k, v) in enumerate(blocks):
        gk, gv = store.get_any(b)
        assert torch.equal(gk, k) and torch.equal(gv, v)


def make_row_tagged_block(*, num_layers=2, batch=4, tokens_per_block=16, kv_heads=2, head_dim=32):
    """Every row filled with its own index (key) / index + 1000 (value)."""
    shape = (num_layers, batch, tokens_per_block, kv_heads, head_dim)
    key = torch.zeros(shape, dtype=torch.float16, device="cuda")
    value = torch.zeros(shape, dtype=torch.float16, device="cuda")
    for row in range(batch):
        key[:, row] = row
        value[:, row] = row + 1000
    return key, value


def test_reorder_batch_rows_reorders_duplicates_and_drops_on_both_tiers():
    from pager_hf.kv_block_store import KVBlockStore

    store = KVBlockStore(tokens_per_block=16)
    store.put_gpu(0, *make_row_tagged_block())
    store.put_gpu(1, *make_row_tagged_block())
    store.offload_to_cpu(1)
    new_row_indices = [2, 2, 1, 3]  # reorder, duplicate row 2, drop row 0
    store.reorder_batch_rows(new_row_indices)
    assert store.has_gpu(0) and store.has_cpu(1)  # tiers unchanged
    for block_id in (0, 1):
        key, value = store.get_any(block_id)
        for new_row, old_row in enumerate(new_row_indices):
            assert torch.all(key[:, new_row] == old_row)
            assert torch.all(value[:, new_row] == old_row + 1000)
    # A second reorder composes with the first, and moves keep the reordered data.
    store.reorder_batch_rows([3, 0, 0, 1])  # rows now hold old rows [3, 2, 2, 2]
    store.load_to_gpu(1, "cuda")
    store.offload_to_cpu(0)
    for block_id in (0, 1):
        key, value = store.get_any(block_id)
        for new_row, old_row in enumerate([3, 2, 2, 2]):
            assert torch.all(key[:, new_row] == old_row)
            assert torch.all(value[:, new_row] == old_row + 1000)


def test_reorder_batch_rows_rejects_a_different_batch_size():
    from pager_hf.kv_block_store import KVBlockStore

    store = KVBlockStore(tokens_per_block=16)
    store.put_gpu(0, *make_row_tagged_block())
    with pytest.raises(ValueError):
        store.reorder_batch_rows([0, 1])
    with pytest.raises(IndexError):
        store.reorder_batch_rows([0, 1, 2, 4])
