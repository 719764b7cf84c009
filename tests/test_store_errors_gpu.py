"""Failure handling of the native store on the GPU: every misuse raises the exception the
status code maps to (capacity -> MemoryError, unknown id -> KeyError, bad state ->
RuntimeError, bad argument -> ValueError) and leaves the store usable."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

MIB16 = 16 * 2**20


def _dec(pool_blocks=16, host_blocks=64, **kw):
    from pager_hf import PagedDecoder

    return PagedDecoder(num_layers=1, num_query_heads=4, num_kv_heads=2, head_dim=64, tokens_per_block=16,
                        dtype=torch.float16, device="cuda", pool_blocks=pool_blocks, host_blocks=host_blocks,
                        staging_blocks=16, **kw)


def _kv(n, rows=1, offset=0):
    """[rows, 2, n, 64] fp16 K and V; offset > 0 gives tensors that start `offset` elements
    into their storage (contiguous, but not 16-byte aligned for an odd offset)."""
    numel = rows * 2 * n * 64
    k = torch.randn(numel + offset, device="cuda").half()[offset:].view(rows, 2, n, 64)
    v = torch.randn(numel + offset, device="cuda").half()[offset:].view(rows, 2, n, 64)
    return [k], [v]


def _step(dec, sids):
    S = sum(dec.sessions[s].rows for s in sids)
    q = torch.randn(S, 4, 64, device="cuda").half()
    kn = torch.randn(S, 2, 64, device="cuda").half()
    dec.begin_step(sids)
    dec.decode_layer(0, q, kn, kn)
    return dec.end_step()


def test_hbm_pool_exhaustion_is_a_memory_error_and_the_store_stays_usable():
    """A prompt placed in HBM before its first placement needs no pool room (blocks past it
    keep their bytes on the host); a placement that loads more blocks than the pool holds
    raises MemoryError."""
    dec = _dec(pool_blocks=4)
    sid = dec.add_session(capacity_tokens=400, vram_budget=64 * MIB16, ram_budget=1 << 30, recent_window=63,
                          policy="recent_only")
    ks, vs = _kv(200)  # 12 full blocks, all wanted in HBM, 4 slots
    moves = dec.prefill(sid, ks, vs, 200, place=False)
    assert moves["to_gpu"] == list(range(12))
    assert dec.pool.session_info(sid)[2] == 12  # all 12 count as HBM-resident
    assert dec.pool.hbm_bytes()["pool"] == 4 * 2 * 2 * 16 * 64 * 2  # 4 slots of 8 KiB (K and V)
    with pytest.raises(MemoryError):  # the first placement loads all 12 into 4 slots
        _step(dec, [sid])
    dec.remove_session(sid)
    sid = dec.add_session(capacity_tokens=100, vram_budget=2 * MIB16, ram_budget=1 << 30, recent_window=1,
                          policy="recent_only")
    ks, vs = _kv(40)
    dec.prefill(sid, ks, vs, 40)
    _step(dec, [sid])


def test_session_capacity_and_host_mirror_limits():
    dec = _dec(host_blocks=8)
    with pytest.raises(MemoryError):  # the host range of one row does not fit
        dec.add_session(capacity_tokens=16 * 40, vram_budget=2 * MIB16, ram_budget=1 << 30, recent_window=1,
                        policy="recent_only")
    sid = dec.add_session(capacity_tokens=20, vram_budget=2 * MIB16, ram_budget=1 << 30, recent_window=1,
                          policy="recent_only")
    ks, vs = _kv(15)
    dec.prefill(sid, ks, vs, 15)
    with pytest.raises(MemoryError):
        for _ in range(40):  # grows past its declared capacity
            _step(dec, [sid])


def test_unknown_session_and_step_state_errors():
    dec = _dec()
    sid = dec.add_session(capacity_tokens=200, vram_budget=2 * MIB16, ram_budget=1 << 30, recent_window=1,
                          policy="recent_only")
    ks, vs = _kv(50)
    dec.prefill(sid, ks, vs, 50)
    with pytest.raises(KeyError):
        dec.pool.begin_step([sid + 7])
    with pytest.raises(ValueError):
        dec.pool.begin_step([sid, sid])  # a session listed twice
    dec.begin_step([sid])
    with pytest.raises(RuntimeError):
        dec.begin_step([sid])  # a step is already open
    with pytest.raises(RuntimeError):
        dec.pool.reorder_rows(sid, [0])  # not during a step
    with pytest.raises(ValueError):
        dec.decode_layer(0, torch.zeros(2, 4, 64, device="cuda").half(), torch.zeros(1, 2, 64, device="cuda").half(),
                         torch.zeros(1, 2, 64, device="cuda").half())  # wrong batch
    dec.end_step()
    _step(dec, [sid])  # the store is still usable
    with pytest.raises(KeyError):
        dec.pool.remove_session(sid + 9)


def test_misaligned_import_is_rejected():
    dec = _dec()
    sid = dec.add_session(capacity_tokens=200, vram_budget=2 * MIB16, ram_budget=1 << 30, recent_window=1,
                          policy="recent_only")
    ks, vs = _kv(50, offset=1)  # starts 2 bytes into its storage
    with pytest.raises(ValueError):
        dec.prefill(sid, ks, vs, 50)


def test_ram_budget_exceeded_during_placement(caplog):
    """The store's host-RAM budget (kv_block_store.py:86-99): placement that would offload
    past it raises, naming the budget."""
    dec = _dec(ram_budget_bytes=20_000)  # one 16-token block of this geometry is 8 KiB
    sid = dec.add_session(capacity_tokens=400, vram_budget=1 * MIB16, ram_budget=1 << 30, recent_window=0,
                          policy="recent_only")
    ks, vs = _kv(100)  # 6 full blocks: 5 wanted on the host, the budget holds 2
    with pytest.raises(RuntimeError, match="ram_budget exceeded while placing block 2"):
        dec.prefill(sid, ks, vs, 100)
    assert dec.pool.resident_bytes()[1] == 2 * 8192
    dec.remove_session(sid)
    assert dec.pool.resident_bytes() == (0, 0)
    sid = dec.add_session(capacity_tokens=400, vram_budget=4 * MIB16, ram_budget=1 << 30, recent_window=3,
                          policy="recent_only")
    ks, vs = _kv(100)  # 4 in HBM, 2 on the host: within the budget, above 80% of it
    with caplog.at_level("WARNING"):
        dec.prefill(sid, ks, vs, 100)
    assert dec.pool.resident_bytes()[1] == 2 * 8192
    assert "ram_budget usage at 82% after offloading block 1" in caplog.text
    _step(dec, [sid])
