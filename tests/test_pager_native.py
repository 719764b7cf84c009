"""The native placement core (pager.PyPager over libpgr.so) against the oracle, bit for bit.

Host code only: runs without a GPU. Covers the published goldens through the native path,
a seeded differential sweep over all four policies with deliberately tied and repeated
scores (ties are where stable sort, first-min and last-max decide the result), and the
Python surface of lib.rs (defaults, PyO3 argument conversion errors, Metrics getters).
"""
from __future__ import annotations

import random
import threading
import zlib

import numpy as np
import pytest

import pager
from oracle import pager_policy as op
from test_oracle_pager import BLOCK, drive_blocks, run_integration_golden, run_reload_path

POLICIES = ["recent_only", "sinks_recent", "heavy_hitter", "sinks_heavy_hitter"]


def metrics_tuple(m):
    return (m.tokens, m.vram_peak, m.ram_peak, m.swap_vram_ram, m.swap_ram_ssd, m.attention_mass_total,
            m.attention_mass_vram)


def test_native_reproduces_published_placement_list():
    p, g = run_integration_golden(pager.PyPager)
    assert p.vram_block_ids() == g["expected_vram_block_ids"]


@pytest.mark.parametrize("policy", POLICIES)
def test_native_reload_path_matches_published_rows(policy):
    g, gpu, cpu, to_gpu, to_cpu = run_reload_path(policy, cls=pager.PyPager)
    row = g["rows"][policy]
    assert (to_cpu, to_gpu) == (row["total_gpu_to_cpu_copies"], row["total_cpu_to_gpu_copies"])
    if policy in ("recent_only", "sinks_recent"):
        assert (gpu, cpu) == (row["final_gpu_blocks"], row["final_cpu_blocks"])


@pytest.mark.parametrize("policy", POLICIES)
def test_native_passes_core_rs_unit_properties(policy):
    p = pager.PyPager(3 * BLOCK, 100 * BLOCK, 2, 4, 0.05, 0.20, policy)
    drive_blocks(p, 15)
    assert len(p.vram_block_ids()) <= 3
    q = pager.PyPager(2 * BLOCK, 100 * BLOCK, 1, 4, 0.05, 0.20, "recent_only")
    drive_blocks(q, 5)
    before = q.vram_block_ids()
    q.force_rebalance(4)
    assert q.vram_block_ids() == before == [3, 4]


def _score_vector(rng, n, mode):
    if mode == "ties":
        levels = [0.0, 0.05, 0.05, 0.2, 0.5]
        return [rng.choice(levels) for _ in range(n)]
    if mode == "spiky":
        v = [rng.random() * 1e-3 for _ in range(n)]
        for _ in range(max(1, n // 7)):
            v[rng.randrange(n)] += rng.random()
        return v
    return [rng.random() for _ in range(n)]


@pytest.mark.parametrize("policy", POLICIES)
@pytest.mark.parametrize("mode", ["ties", "spiky", "uniform"])
def test_native_matches_oracle_on_random_traces(policy, mode):
    rng = random.Random(zlib.crc32(f"{policy}/{mode}".encode()))
    for trial in range(6):
        vram = rng.randint(0, 12) * BLOCK + rng.randint(0, BLOCK - 1)
        ram = rng.randint(0, 20) * BLOCK
        recent = rng.randint(0, 10)
        interval = rng.randint(1, 5)
        pm, rpm = rng.choice([0.0, 0.05, 0.1]), rng.choice([0.0, 0.2])
        a = pager.PyPager(vram, ram, recent, interval, pm, rpm, policy)
        b = op.Pager(vram, ram, recent, interval, pm, rpm, policy)
        n = rng.randint(1, 6)
        for step in range(40):
            if rng.random() < 0.3:
                n += 1
            scores = _score_vector(rng, n, mode)
            a.on_step(n - 1, 0, scores)
            b.on_step(n - 1, 0, scores)
            if rng.random() < 0.3:
                a.force_rebalance(n - 1)
                b.force_rebalance(n - 1)
            assert a.tiers() == b.tiers(), (trial, step)
        assert a.vram_block_ids() == b.vram_block_ids()
        assert metrics_tuple(a.metrics()) == metrics_tuple(b.get_metrics())


def test_scores_are_rounded_to_f32_like_pyo3():
    """A score that only differs from another below f32 resolution must tie with it."""
    x = 0.1
    y = float(np.nextafter(np.float64(0.1), 1.0))  # same f32 value, different f64
    for cls in (pager.PyPager, op.Pager):
        p = cls(1 * BLOCK, 10 * BLOCK, 0, 1000, 0.0, 0.0, "heavy_hitter")
        p.on_step(5, 0, [0.0, 0.0, 0.0, 0.0, x, y])
        # blocks 0..3 sinks and 5 pinned; one VRAM slot -> (pinned desc, score desc, stable)
        assert p.vram_block_ids() == [5]


def test_defaults_match_lib_rs():
    p = pager.PyPager(2 * BLOCK, 4 * BLOCK, 1)  # rebalance 32, margins 0.10 / 0.20, heavy_hitter
    q = op.Pager(2 * BLOCK, 4 * BLOCK, 1, 32, 0.10, 0.20, "heavy_hitter")
    for i in range(40):
        s = [((i * 7 + j * 3) % 11) / 10 for j in range(i + 1)]
        p.on_step(i, 0, s)
        q.on_step(i, 0, s)
        assert p.tiers() == q.tiers()


def test_pyo3_argument_conversion_errors():
    with pytest.raises(OverflowError):
        pager.PyPager(-1, 0, 0)
    with pytest.raises(TypeError):
        pager.PyPager(1.5, 0, 0)
    with pytest.raises(TypeError):
        pager.PyPager(1, 1, 1, policy=3)
    p = pager.PyPager(BLOCK, BLOCK, 1)
    with pytest.raises(OverflowError):
        p.on_step(-1, 0, [1.0])
    with pytest.raises(OverflowError):
        p.on_step(0, -1, [1.0])
    with pytest.raises(TypeError):
        p.on_step(0, 0, "abc")
    with pytest.raises(TypeError):
        p.on_step(0, 0, ["x"])
    with pytest.raises(OverflowError):
        p.force_rebalance(-3)


def test_metrics_object_is_read_only_snapshot():
    p = pager.PyPager(2 * BLOCK, 2 * BLOCK, 1, 4, 0.05, 0.2, "recent_only")
    p.on_step(0, 0, [1.0])
    m = p.metrics()
    assert m.tokens == 1 and m.vram_peak == BLOCK and m.attention_mass_total == 1.0
    with pytest.raises(AttributeError):
        m.tokens = 5
    p.on_step(1, 0, [0.5, 0.5])
    assert m.tokens == 1 and p.metrics().tokens == 2
    with pytest.raises(TypeError):
        pager.Metrics()


def test_zero_rebalance_interval_raises_on_second_step():
    """core.rs:95 computes tokens % rebalance_interval from the second call on."""
    p = pager.PyPager(BLOCK, BLOCK, 1, 0)
    p.on_step(0, 0, [1.0])  # tokens == 1 short-circuits
    with pytest.raises(ZeroDivisionError):
        p.on_step(1, 0, [1.0, 1.0])
    o = op.Pager(BLOCK, BLOCK, 1, 0)
    o.on_step(0, 0, [1.0])
    with pytest.raises(ZeroDivisionError):
        o.on_step(1, 0, [1.0, 1.0])


def test_concurrent_mutable_borrow_raises():
    p = pager.PyPager(BLOCK, BLOCK, 1)
    p._borrow.acquire()
    try:
        err = []

        def other():
            try:
                p.on_step(0, 0, [1.0])
            except RuntimeError as e:
                err.append(str(e))

        t = threading.Thread(target=other)
        t.start()
        t.join()
        assert err and "borrowed" in err[0]
    finally:
        p._borrow.release()


def test_empty_attention_vector():
    for cls in (pager.PyPager, op.Pager):
        p = cls(BLOCK, BLOCK, 1, 4, 0.05, 0.2, "heavy_hitter")
        p.on_step(2, 0, [])  # ensure_blocks(0); force_rebalance(2) grows to 3 blocks
        assert len(p.tiers()) == 3
