"""Block split/extract bookkeeping: the reference's own assertions (tests/test_kv_utils.py:41-131),
applied to both the product (pager_hf.kv_utils, torch) and the oracle (oracle.kv_layout, numpy)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_layout as ol
from pager_hf import kv_utils as pk


def make_fake_past(*, num_layers, batch, kv_heads, seq_len, head_dim, seed=0):
    g = torch.Generator().manual_seed(seed)
    return [
        (torch.randn(batch, kv_heads, seq_len, head_dim, generator=g),
         torch.randn(batch, kv_heads, seq_len, head_dim, generator=g))
        for _ in range(num_layers)
    ]


def as_np(past):
    return [(k.numpy(), v.numpy()) for k, v in past]


def test_split_at_block_boundary():
    past = make_fake_past(num_layers=2, batch=1, kv_heads=2, seq_len=35, head_dim=4)
    full, tail, full_tokens = pk.split_full_blocks_and_tail(past, tokens_per_block=16)
    assert full_tokens == 32 and full[0][0].shape[2] == 32 and tail[0][0].shape[2] == 3
    ofull, otail, ofull_tokens = ol.split_full_blocks_and_tail(as_np(past), 16)
    assert ofull_tokens == 32
    np.testing.assert_array_equal(tail[1][1].numpy(), otail[1][1])


def test_split_exact_multiple():
    past = make_fake_past(num_layers=1, batch=1, kv_heads=1, seq_len=32, head_dim=2)
    _, tail, full_tokens = pk.split_full_blocks_and_tail(past, tokens_per_block=16)
    assert full_tokens == 32 and tail[0][0].shape[2] == 0


@pytest.mark.parametrize("batch", [1, 3])
def test_blocks_round_trip(batch):
    num_layers, kv_heads, head_dim, tpb = 3, 2, 4, 16
    past = make_fake_past(num_layers=num_layers, batch=batch, kv_heads=kv_heads, seq_len=tpb * 4, head_dim=head_dim)
    blocks = pk.real_past_to_blocks(past, tokens_per_block=tpb)
    oblocks = ol.real_past_to_blocks(as_np(past), tpb)
    assert len(blocks) == 4
    for (key, value), (okey, ovalue) in zip(blocks, oblocks):
        assert key.shape == (num_layers, batch, tpb, kv_heads, head_dim)
        np.testing.assert_array_equal(key.numpy(), okey)
        np.testing.assert_array_equal(value.numpy(), ovalue)
    # Inverse: concatenating the blocks back along tokens restores every layer exactly.
    for layer in range(num_layers):
        rec_k = torch.cat([b[0][layer].transpose(1, 2) for b in blocks], dim=2)
        assert torch.equal(rec_k, past[layer][0])


def test_block_one_is_tokens_16_to_32():
    past = make_fake_past(num_layers=1, batch=1, kv_heads=1, seq_len=32, head_dim=2)
    key, _ = pk.extract_single_block_from_past(past, block_id=1, tokens_per_block=16)
    assert torch.equal(key[0], past[0][0][:, :, 16:32, :].permute(0, 2, 1, 3))


def test_legacy_past_key_values_forms():
    past = make_fake_past(num_layers=2, batch=1, kv_heads=1, seq_len=4, head_dim=2)

    class Out:
        pass

    o = Out()
    o.past_key_values = tuple(past)
    assert len(pk.get_legacy_past_key_values(o)) == 2

    class Cache:
        key_cache = [k for k, _ in past]
        value_cache = [v for _, v in past]

    o.past_key_values = Cache()
    got = pk.get_legacy_past_key_values(o)
    assert torch.equal(got[1][0], past[1][0])
    o.past_key_values = None
    with pytest.raises(RuntimeError):
        pk.get_legacy_past_key_values(o)
