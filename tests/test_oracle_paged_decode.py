"""Pins the paged decode oracle (oracle/paged_decode.py) against what the reference fixes.

- apply_tiers index lists: the closed form of pager_hf/kv_block_store.py:206-227 (ascending
  ids; tier 0 -> GPU, any other tier -> CPU; ids past len(tiers) -> CPU).
- Placement glue and gather indices (paged_model.py:792-799, 907-916, 1227-1231): a
  recent_only session worked by hand from core.rs:167-171, 209-214. With vram = 8 blocks and
  recent = 7, blocks N-8 .. N-1 stay resident and the block that leaves the window is evicted
  at the step that completes a new block.
- Scores handed to the pager (paged_model.py:1041-1048, 865-876): float64 brute force with
  scalar math.exp loops -- per layer the block mass of the full blocks known before the step,
  mean over rows and query heads, summed over layers, divided by num_layers, normalized.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle.paged_decode import PagedDecodeOracle, apply_tiers_moves

MIB16 = 16 * 1024 * 1024


def test_apply_tiers_closed_form():
    gpu, cpu = {0, 2, 5}, {1, 3, 4, 6}
    to_gpu, to_cpu = apply_tiers_moves(gpu, cpu, [1, 0, 0, 2, 1])  # ids 5, 6 past the tiers -> CPU
    assert to_gpu == [1]
    assert to_cpu == [0, 5]
    assert gpu == {1, 2}
    assert cpu == {0, 3, 4, 5, 6}
    assert apply_tiers_moves(gpu, cpu, [1, 0, 0]) == ([], [])  # idempotent


def _zeros(rows, hkv, n, d):
    return np.zeros((rows, hkv, n, d), np.float32)


def test_recent_only_window_gather_and_eviction():
    T, d, hkv, hq = 32, 8, 1, 1
    o = PagedDecodeOracle(num_layers=1, num_query_heads=hq, num_kv_heads=hkv, head_dim=d, tokens_per_block=T)
    o.add_session(0, vram_budget=8 * MIB16, ram_budget=1 << 40, recent_window=7, rebalance_interval=32,
                  policy="recent_only")
    to_gpu, to_cpu = o.prefill(0, [_zeros(1, hkv, 4096, d)], [_zeros(1, hkv, 4096, d)], 4096)
    assert to_gpu == list(range(120, 128))  # prefill starts every block on the host
    assert to_cpu == []
    zq = [np.zeros((1, hq, d), np.float32)]
    zk = [np.zeros((1, hkv, d), np.float32)]
    for step in range(1, 33):
        r = o.step([0], zq, zk, zk, compute=False)
        assert r["gather"] == [list(range(120))]  # host blocks read this step, ascending
        pl = r["placement"][0]
        if step < 32:
            assert pl["added"] == [] and pl["to_gpu"] == [] and pl["to_cpu"] == []
        else:  # token 4127 completes block 128: resident window moves to 121..128
            assert pl["added"] == [128]
            assert pl["to_cpu"] == [120]
            assert pl["to_gpu"] == []
            assert pl["scores"] == [1.0 / 129] * 129
    r = o.step([0], zq, zk, zk, compute=False)
    assert r["gather"] == [list(range(121))]
    assert sorted(o.sessions[0].gpu) == list(range(121, 129))


def _brute_force_layer(q, keys, vals, lo, n_rep, scale):
    """One sequence: q [Hq, D], keys/vals [Hkv, n, D]; valid positions >= lo. Float64."""
    hq, d = q.shape
    n = keys.shape[1]
    out = np.zeros((hq, d))
    weights = np.zeros((hq, n))
    for h in range(hq):
        kv = h // n_rep
        s = [sum(float(q[h, i]) * float(keys[kv, t, i]) for i in range(d)) * scale if t >= lo else -math.inf
             for t in range(n)]
        m = max(s)
        e = [math.exp(x - m) if x != -math.inf else 0.0 for x in s]
        z = sum(e)
        for t in range(n):
            weights[h, t] = e[t] / z
            out[h] += weights[h, t] * vals[kv, t].astype(np.float64)
    return out, weights


def test_scores_and_outputs_match_brute_force():
    rng = np.random.default_rng(7)
    L, hq, hkv, d, T, n0 = 2, 4, 2, 8, 16, 40
    n_rep = hq // hkv
    lo = [0, 5]
    o = PagedDecodeOracle(num_layers=L, num_query_heads=hq, num_kv_heads=hkv, head_dim=d, tokens_per_block=T)
    o.add_session(3, rows=2, vram_budget=1 * MIB16, ram_budget=1 << 40, recent_window=1, policy="sinks_heavy_hitter",
                  lo=lo)
    keys = [rng.standard_normal((2, hkv, n0, d)).astype(np.float32) for _ in range(L)]
    vals = [rng.standard_normal((2, hkv, n0, d)).astype(np.float32) for _ in range(L)]
    o.prefill(3, keys, vals, n0)
    q = [rng.standard_normal((2, hq, d)).astype(np.float32) for _ in range(L)]
    kn = [rng.standard_normal((2, hkv, d)).astype(np.float32) for _ in range(L)]
    vn = [rng.standard_normal((2, hkv, d)).astype(np.float32) for _ in range(L)]
    r = o.step([3], q, kn, vn)
    scale = 1.0 / math.sqrt(d)
    n_mass = n0 // T  # full blocks known before the step
    per_layer = []
    for layer in range(L):
        masses = []
        for row in range(2):
            k_all = np.concatenate([keys[layer][row], kn[layer][row][:, None]], axis=1)
            v_all = np.concatenate([vals[layer][row], vn[layer][row][:, None]], axis=1)
            out, w = _brute_force_layer(q[layer][row], k_all, v_all, lo[row], n_rep, scale)
            np.testing.assert_allclose(r["out"][layer][row], out, rtol=0, atol=2e-6)
            masses.append([[w[h, b * T:(b + 1) * T].sum() for b in range(n_mass)] for h in range(hq)])
        per_layer.append(np.mean(np.array(masses), axis=(0, 1)))  # mean over rows and heads
    averaged = np.sum(per_layer, axis=0) / L
    expected = averaged / averaged.sum()
    scores = r["placement"][3]["scores"]
    assert len(scores) == n0 // T  # on_step gets one entry per block known before the step
    np.testing.assert_allclose(scores, expected, rtol=0, atol=1e-6)
    # Row 1's padding (positions < 5) carries no weight; block 0 still gets row 0's mass.
    assert scores[0] > 0


def test_window_lo_skips_blocks_below_it():
    rng = np.random.default_rng(11)
    hq, hkv, d, T, n0 = 2, 1, 8, 16, 100
    o = PagedDecodeOracle(num_layers=1, num_query_heads=hq, num_kv_heads=hkv, head_dim=d, tokens_per_block=T)
    o.add_session(0, vram_budget=2 * MIB16, ram_budget=1 << 40, recent_window=1, policy="sinks_heavy_hitter",
                  lo=[40])
    keys = [rng.standard_normal((1, hkv, n0, d)).astype(np.float32)]
    vals = [rng.standard_normal((1, hkv, n0, d)).astype(np.float32)]
    o.prefill(0, keys, vals, n0)
    host_before = sorted(o.sessions[0].cpu)
    q = [rng.standard_normal((1, hq, d)).astype(np.float32)]
    kn = [rng.standard_normal((1, hkv, d)).astype(np.float32)]
    vn = [rng.standard_normal((1, hkv, d)).astype(np.float32)]
    r = o.step([0], q, kn, vn)
    # Gather starts at the block holding position lo (40 // 16 = 2).
    assert r["gather"] == [[b for b in host_before if b >= 2]]
    k_all = np.concatenate([keys[0][0], kn[0][0][:, None]], axis=1)
    v_all = np.concatenate([vals[0][0], vn[0][0][:, None]], axis=1)
    out, w = _brute_force_layer(q[0][0], k_all, v_all, 40, hq // hkv, 1.0 / math.sqrt(d))
    np.testing.assert_allclose(r["out"][0][0], out, rtol=0, atol=2e-6)
    scores = r["placement"][0]["scores"]
    assert scores[0] == 0.0 and scores[1] == 0.0  # blocks entirely below lo
    mass = np.array([w[:, b * T:(b + 1) * T].sum(axis=1).mean() for b in range(n0 // T)])
    np.testing.assert_allclose(scores, mass / mass.sum(), rtol=0, atol=1e-6)


def test_per_layer_window_against_brute_force():
    """A layer with its own sliding window (Gemma2's alternating layers) attends to the
    positions c > pos - W only (paged_model.py:977-982), on top of the row's first valid
    position; the other layer attends to everything. Outputs and scores against float64
    brute force, the valid set of each (row, layer) enumerated position by position."""
    rng = np.random.default_rng(13)
    L, hq, hkv, d, T, n0, W = 2, 4, 2, 8, 16, 70, 24
    n_rep = hq // hkv
    lo = [0, 5]
    o = PagedDecodeOracle(num_layers=L, num_query_heads=hq, num_kv_heads=hkv, head_dim=d, tokens_per_block=T)
    o.add_session(1, rows=2, vram_budget=1 * MIB16, ram_budget=1 << 40, recent_window=1, policy="sinks_heavy_hitter",
                  lo=lo)
    keys = [rng.standard_normal((2, hkv, n0, d)).astype(np.float32) for _ in range(L)]
    vals = [rng.standard_normal((2, hkv, n0, d)).astype(np.float32) for _ in range(L)]
    o.prefill(1, keys, vals, n0)
    q = [rng.standard_normal((2, hq, d)).astype(np.float32) for _ in range(L)]
    kn = [rng.standard_normal((2, hkv, d)).astype(np.float32) for _ in range(L)]
    vn = [rng.standard_normal((2, hkv, d)).astype(np.float32) for _ in range(L)]
    windows = [None, W]
    r = o.step([1], q, kn, vn, windows=windows)
    pos = n0  # the new token's position
    n_mass = n0 // T
    per_layer = []
    for layer in range(L):
        masses = []
        for row in range(2):
            valid = [c for c in range(pos + 1) if c >= lo[row] and (windows[layer] is None or c > pos - W)]
            first = min(valid)
            assert valid == list(range(first, pos + 1))  # one contiguous range
            k_all = np.concatenate([keys[layer][row], kn[layer][row][:, None]], axis=1)
            v_all = np.concatenate([vals[layer][row], vn[layer][row][:, None]], axis=1)
            out, w = _brute_force_layer(q[layer][row], k_all, v_all, first, n_rep, 1.0 / math.sqrt(d))
            np.testing.assert_allclose(r["out"][layer][row], out, rtol=0, atol=2e-6)
            masses.append([[w[h, b * T:(b + 1) * T].sum() for b in range(n_mass)] for h in range(hq)])
        per_layer.append(np.mean(np.array(masses), axis=(0, 1)))
    # The windowed layer gives no mass to blocks wholly at or before pos - W.
    assert per_layer[1][0] == 0.0 and per_layer[1][1] == 0.0 and per_layer[0][0] > 0
    averaged = np.sum(per_layer, axis=0) / L
    np.testing.assert_allclose(r["placement"][1]["scores"], averaged / averaged.sum(), rtol=0, atol=1e-6)


@pytest.mark.parametrize("policy", ["recent_only", "sinks_recent"])
def test_score_free_policies_pass_uniform_scores(policy):
    o = PagedDecodeOracle(num_layers=1, num_query_heads=1, num_kv_heads=1, head_dim=8, tokens_per_block=16)
    o.add_session(0, vram_budget=2 * MIB16, ram_budget=1 << 40, recent_window=1, policy=policy)
    o.prefill(0, [_zeros(1, 1, 50, 8)], [_zeros(1, 1, 50, 8)], 50)
    z = [np.zeros((1, 1, 8), np.float32)]
    r = o.step([0], z, z, z, compute=False)
    assert r["placement"][0]["scores"] == [1.0 / 3] * 3
