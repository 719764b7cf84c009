"""Pins the oracle's placement policy (oracle/pager_policy.py) against what the reference fixes.

Sources: the ten Rust unit tests of pager/src/core.rs:582-704 (restated as properties),
the published placement list of README.md:389 (bench/torch_kv_pager_integration_mvp.py),
bench/persistent_policy_compare_results.csv rows 2-3 (final blocks and copy counts of a
64-step run), and hand-derived micro cases for the tie and rounding rules.
"""
from __future__ import annotations

import json
import os
import struct

import numpy as np
import pytest

from oracle import pager_policy as op
from oracle.paged_decode import apply_tiers_moves

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
BLOCK = 16 * 1024 * 1024


def make_pager(vram_blocks, ram_blocks, recent_window, policy, cls=op.Pager):
    """core.rs:563-573."""
    return cls(vram_blocks * BLOCK, ram_blocks * BLOCK, recent_window, 4, 0.05, 0.20, policy)


def drive_blocks(pager, count):
    """core.rs:575-580."""
    for i in range(count):
        pager.on_step(i, 0, [1.0] * (i + 1))
        pager.force_rebalance(i)


# -- core.rs unit tests ----------------------------------------------------------------


def test_unknown_policy_name_falls_back_to_heavy_hitter():
    assert op.policy_from_name("not_a_real_policy") == op.HEAVY_HITTER
    assert op.policy_from_name("recent_only") == op.RECENT_ONLY
    assert op.policy_from_name("sinks_recent") == op.SINKS_RECENT
    assert op.policy_from_name("heavy_hitter") == op.HEAVY_HITTER
    assert op.policy_from_name("sinks_heavy_hitter") == op.SINKS_HEAVY_HITTER


def test_recent_only_respects_vram_budget_and_keeps_most_recent():
    p = make_pager(2, 100, 1, "recent_only")
    drive_blocks(p, 5)
    assert p.vram_block_ids() == [3, 4]


def test_sinks_recent_keeps_a_sink_block():
    p = make_pager(3, 100, 1, "sinks_recent")
    drive_blocks(p, 10)
    assert any(i < 4 for i in p.vram_block_ids())


def test_recent_only_ignores_attention_scores():
    p = make_pager(2, 100, 1, "recent_only")
    p.on_step(0, 0, [1000.0])
    p.force_rebalance(0)
    drive_blocks(p, 6)
    assert 0 not in p.vram_block_ids()


def test_ensure_blocks_grows_to_attention_length():
    p = make_pager(10, 10, 4, "recent_only")
    p.on_step(0, 0, [1.0, 1.0, 1.0])
    assert len(p.tiers()) == 3


def test_metrics_tokens_counts_on_step_calls():
    p = make_pager(5, 100, 10, "recent_only")
    assert p.get_metrics().tokens == 0
    for i in range(3):
        p.on_step(i, 0, [1.0] * (i + 1))
    assert p.get_metrics().tokens == 3


def test_vram_peak_never_exceeds_budget():
    p = make_pager(2, 100, 1, "sinks_heavy_hitter")
    drive_blocks(p, 20)
    assert p.get_metrics().vram_peak <= 2 * BLOCK


@pytest.mark.parametrize("policy", ["recent_only", "sinks_recent", "heavy_hitter", "sinks_heavy_hitter"])
def test_tiers_never_exceed_vram_budget(policy):
    p = make_pager(3, 100, 2, policy)
    drive_blocks(p, 15)
    assert len(p.vram_block_ids()) <= 3


def test_force_rebalance_is_idempotent():
    p = make_pager(2, 100, 1, "recent_only")
    drive_blocks(p, 5)
    before = p.vram_block_ids()
    p.force_rebalance(4)
    assert p.vram_block_ids() == before


# -- published placement list (README.md:389) ------------------------------------------


def synthetic_trace(rng, query_block, num_blocks):
    """Trace generator of bench/torch_kv_pager_integration_mvp.py:40-68 (test input only)."""
    attn = [0.001 for _ in range(num_blocks)]
    for b in range(min(4, num_blocks)):
        attn[b] += 0.20
    for b in range(max(0, query_block - 8), min(num_blocks, query_block + 1)):
        attn[b] += 0.08
    for b in (20, 21, 55, 56, 90, 91):
        if b < num_blocks:
            attn[b] += 0.12
    for b in range(num_blocks):
        attn[b] += rng.random() * 0.002
    total = sum(attn)
    return [x / total for x in attn]


def run_integration_golden(cls):
    import random

    with open(os.path.join(GOLDEN, "pager_integration_golden.json")) as f:
        g = json.load(f)
    rng = random.Random(g["seed"])
    p = cls(g["vram"], g["ram"], g["recent"], g["rebalance_interval"], g["promote_margin"],
            g["ram_promote_margin"], g["policy"])
    for q in range(g["first_query_block"], g["num_blocks"], g["query_stride"]):
        p.on_step(q, 0, synthetic_trace(rng, q, q + 1))
    return p, g


def test_oracle_reproduces_published_placement_list():
    p, g = run_integration_golden(op.Pager)
    assert p.vram_block_ids() == g["expected_vram_block_ids"]


# -- bench/persistent_policy_compare_results.csv rows 2-5 ------------------------------


def run_reload_path(policy, cls=op.Pager):
    """The 64-step reload-path loop of bench/real_kv_persistent_policy_compare_mvp.py:204-278
    with the store reduced to its residency sets; returns final sets and copy counts."""
    with open(os.path.join(GOLDEN, "policy_compare_rows.json")) as f:
        g = json.load(f)
    cfg = g["config"]
    p = cls(cfg["vram"], cfg["ram"], cfg["recent"], cfg["rebalance_interval"], cfg["promote_margin"],
            cfg["ram_promote_margin"], policy)
    gpu, cpu = set(range(cfg["initial_blocks"])), set()
    num_blocks = cfg["initial_blocks"]
    to_gpu_copies = to_cpu_copies = 0
    for step in range(1, cfg["steps"] + 1):
        to_gpu_copies += len(cpu)  # reload_all_blocks_for_forward
        gpu |= cpu
        cpu = set()
        added = [num_blocks] if step in cfg["added_at_steps"] else []
        for b in added:
            gpu.add(b)
            num_blocks += 1
        p.on_step(num_blocks - 1, 0, [1.0 / num_blocks] * num_blocks)
        if added:
            p.force_rebalance(num_blocks - 1)
        _, moved = apply_tiers_moves(gpu, cpu, p.tiers())
        to_cpu_copies += len(moved)
    return g, sorted(gpu), sorted(cpu), to_gpu_copies, to_cpu_copies


@pytest.mark.parametrize("policy", ["recent_only", "sinks_recent", "heavy_hitter", "sinks_heavy_hitter"])
def test_reload_path_copy_counts_match_published_rows(policy):
    g, gpu, cpu, to_gpu, to_cpu = run_reload_path(policy)
    row = g["rows"][policy]
    assert to_cpu == row["total_gpu_to_cpu_copies"]
    assert to_gpu == row["total_cpu_to_gpu_copies"]
    block_bytes = g["config"]["block_bytes"]
    assert to_cpu * block_bytes / 1e6 == pytest.approx(row["total_gpu_to_cpu_mb"], abs=1e-9)
    assert to_gpu * block_bytes / 1e6 == pytest.approx(row["total_cpu_to_gpu_mb"], abs=1e-9)
    if policy in ("recent_only", "sinks_recent"):  # score-free: final placement is fixed too
        assert gpu == row["final_gpu_blocks"]
        assert cpu == row["final_cpu_blocks"]


# -- hand-derived micro cases -----------------------------------------------------------


def test_compare_scores_treats_nan_as_equal():
    nan = np.float32("nan")
    assert op.compare_scores(nan, np.float32(1)) == 0
    assert op.compare_scores(np.float32(1), nan) == 0
    assert op.compare_scores(np.float32(1), np.float32(2)) == -1


def test_min_by_keeps_first_and_max_by_keeps_last_of_ties():
    keys = [np.float32(x) for x in (2.0, 1.0, 3.0, 1.0, 3.0)]
    assert op._min_by_first(range(5), lambda i: keys[i]) == 1
    assert op._max_by_last(range(5), lambda i: keys[i]) == 4


def _f32(x):
    return struct.unpack("f", struct.pack("f", x))[0]


def test_score_ema_rounds_each_f32_operation():
    """score = f32(f32(score*0.9f) + f32(a*0.1f)); a wider accumulator gives other bits."""
    p = op.Pager(10 * BLOCK, 10 * BLOCK, 0, 1000, 0.05, 0.2, "heavy_hitter")
    seq = [0.1344, 0.8474, 0.7638, 0.2551, 0.4954, 0.4495]
    expected = 0.0
    wide = 0.0
    fused = 0.0
    for a in seq:
        p.on_step(0, 0, [a])
        expected = _f32(_f32(expected * _f32(0.9)) + _f32(_f32(a) * _f32(0.1)))
        wide = wide * 0.9 + a * 0.1
        fused = _f32(fused * _f32(0.9) + _f32(_f32(a) * _f32(0.1)))  # one rounding: a fused multiply-add
    got = float(p.blocks[0].score)
    assert got == expected
    # These inputs tell the three roundings apart, so the check above has teeth.
    assert _f32(wide) != expected and fused != expected


def test_sinks_heavy_hitter_selection_by_hand():
    """12 blocks, 9 VRAM: 4 sinks, recent budget min(2, 9//2, 5) = 2 -> {10, 11}, then the 3
    best scores among 4..9; equal scores fall back to id order (stable sort)."""
    p = op.Pager(9 * BLOCK, 100 * BLOCK, 2, 1000, 0.05, 0.2, "sinks_heavy_hitter")
    p.on_step(11, 0, [0.5] * 12)
    assert p.vram_block_ids() == [0, 1, 2, 3, 4, 5, 6, 10, 11]
    q = op.Pager(9 * BLOCK, 100 * BLOCK, 2, 1000, 0.05, 0.2, "sinks_heavy_hitter")
    q.on_step(11, 0, [0.5] * 8 + [0.9] + [0.5] * 3)
    assert q.vram_block_ids() == [0, 1, 2, 3, 4, 5, 8, 10, 11]


def test_heavy_hitter_enforce_vram_budget_keeps_best_pinned_by_hand():
    """heavy_hitter, 3 VRAM, recent_window 0, blocks 0..5 (0..3 sinks and 5 recent pinned).
    First placement (no VRAM yet): pinned first -> {0,1,2} win by id order. A later
    rebalance puts every pinned block in VRAM, over the budget: {0,1,2,3,5} pinned ->
    enforce_vram_budget_keep_best keeps the 3 best by (pinned, score). No swap runs here
    (no unpinned VRAM block): the swaps are pinned in test_oracle_pager_hysteresis.py."""
    p = op.Pager(3 * BLOCK, 100 * BLOCK, 0, 1000, 0.05, 0.2, "heavy_hitter")
    p.on_step(5, 0, [0.1, 0.1, 0.1, 0.1, 0.9, 0.1])
    assert p.vram_block_ids() == [0, 1, 2]
    p.on_step(5, 0, [0.1, 0.1, 0.1, 0.5, 0.9, 0.8])
    p.force_rebalance(5)
    # scores: 0,1,2 -> 0.019; 3 -> 0.059; 4 -> 0.171; 5 -> 0.089; pinned = {0,1,2,3,5}
    assert p.vram_block_ids() == [0, 3, 5]


def test_fill_ram_by_score():
    """sinks_heavy_hitter with 4 VRAM and 2 RAM: the rest goes to the spill tier, RAM keeps
    the two best scores among the non-VRAM blocks (fill_ram; trim_ram is pinned in
    test_oracle_pager_hysteresis.py)."""
    p = op.Pager(4 * BLOCK, 2 * BLOCK, 0, 1000, 0.05, 0.2, "sinks_heavy_hitter")
    p.on_step(7, 0, [0.1, 0.1, 0.1, 0.1, 0.3, 0.7, 0.2, 0.1])
    # VRAM: 4 sinks (recent budget min(0, 2, 0) = 0); RAM: best of 4..7 = {5, 4}
    assert p.tiers() == [0, 0, 0, 0, 1, 1, 2, 2]
