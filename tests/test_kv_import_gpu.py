"""Prompt import, tier moves and row reordering of the native store, read back exactly.

Every record written by the import kernel (pool slots and the host mirror), every record
moved by the batched copy kernel (both directions) and every row copy of a reorder must
read back bit for bit as the K/V that went in.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

MIB16 = 16 * 2**20


def _decoder(layers, hkv, d, dtype, T=32, blocks=200):
    from pager_hf import PagedDecoder

    return PagedDecoder(num_layers=layers, num_query_heads=2 * hkv, num_kv_heads=hkv, head_dim=d, tokens_per_block=T,
                        dtype=dtype, device="cuda", pool_blocks=2 * blocks, host_blocks=2 * blocks + 8,
                        staging_blocks=16, staging_buffers=2)


def _check(dec, sid, ks, vs, n, row_src):
    for layer in range(len(ks)):
        for row, src in enumerate(row_src):
            k, v = dec.pool.export_tokens(sid, row, layer, n)
            assert torch.equal(k, ks[layer][src, :, :n]), f"layer {layer} row {row}"
            assert torch.equal(v, vs[layer][src, :, :n]), f"layer {layer} row {row}"


@pytest.mark.parametrize("d,dtype,place", [(64, torch.float16, True), (128, torch.bfloat16, True),
                                           (64, torch.float16, False), (16, torch.bfloat16, True),
                                           (256, torch.float16, True)])
def test_import_moves_and_reorder_read_back_exactly(d, dtype, place):
    layers, hkv, T, rows, n = 3, 2, 32, 3, 2000
    g = torch.Generator(device="cuda").manual_seed(d)
    n_src = n + 37  # the import reads a prefix of a longer buffer
    ks = [torch.randn(rows, hkv, n_src, d, device="cuda", generator=g).to(dtype) for _ in range(layers)]
    vs = [torch.randn(rows, hkv, n_src, d, device="cuda", generator=g).to(dtype) for _ in range(layers)]
    dec = _decoder(layers, hkv, d, dtype)
    sid = dec.add_session(capacity_tokens=n + 64, rows=rows, vram_budget=8 * MIB16, ram_budget=1 << 40,
                          recent_window=7, policy="recent_only")
    dec.prefill(sid, ks, vs, n, place=place)
    nb = n // T
    gpu_ids = dec.pool.block_ids(sid, True)
    if place:
        assert gpu_ids == list(range(nb - 8, nb))  # recent_only, 8 resident
    else:
        assert gpu_ids == list(range(nb))
    _check(dec, sid, ks, vs, n, list(range(rows)))
    # Moves in both directions in one call: even blocks to HBM, odd blocks to host.
    tiers = [0 if b % 2 == 0 else 1 for b in range(nb)]
    to_gpu, to_cpu, rc, _ = dec.pool.apply_tiers(sid, tiers)
    assert rc == 0 and (to_gpu or to_cpu)
    assert dec.pool.block_ids(sid, True) == [b for b in range(nb) if b % 2 == 0]
    _check(dec, sid, ks, vs, n, list(range(rows)))
    # And back, so blocks whose host copies already exist are evicted without a copy.
    to_gpu, to_cpu, rc, _ = dec.pool.apply_tiers(sid, [1 - t for t in tiers])
    assert rc == 0
    _check(dec, sid, ks, vs, n, list(range(rows)))
    # Beam reorder: row 0 <- 2, row 1 <- 2 (duplicate), row 2 <- 0; old row 1 dropped.
    dec.reorder_rows(sid, [2, 2, 0])
    _check(dec, sid, ks, vs, n, [2, 2, 0])
    dec.reorder_rows(sid, [1, 2, 1])  # now [2, 0, 2]
    to_gpu, to_cpu, rc, _ = dec.pool.apply_tiers(sid, tiers)
    assert rc == 0
    _check(dec, sid, ks, vs, n, [2, 0, 2])
    dec.pool.close()
