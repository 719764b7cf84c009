"""Hand-derived cases for heavy_hitter's hysteresis, run on the oracle and the native pager.

Each case is worked out by hand in its docstring from pager/src/core.rs, so the expected
tiers and swap counters do not come from either implementation:
  * promote_vram_with_hysteresis (core.rs:368-400): swaps out of SSD and out of RAM, a
    chain of two swaps, an improvement exactly equal to the margin (no swap: `<=` breaks),
    first-min among tied worst VRAM blocks and last-max among tied best candidates;
  * trim_ram (core.rs:429-448): RAM over budget after new blocks arrive (they start in
    RAM, core.rs:132-143), ties trimmed in ascending score order, stable by index;
  * promote_ram_with_hysteresis (core.rs:450-477): a swap whose best SSD block is the last
    of two tied maxima;
  * fill_ram (core.rs:402-427) with tied candidates (stable descending order);
  * the first-placement branch of place_heavy_hitter (core.rs:227-242) with tied scores.

Scores are set through on_step: a block's score starts at 0 and becomes
f32(f32(0 * 0.9f) + f32(a * 0.1f)). With a = 10 s for the small values s used here, the
product is s (1 + 1.5e-8), which rounds to s exactly in f32, so the exact-margin cases
compare exact values. A later on_step multiplies scores by 0.9f; those cases use values far
enough apart that rounding cannot reorder them. Counters are in bytes (16 MiB per block,
core.rs:6). count_tier_changes compares each block's tier before and after one placement
(core.rs:515-531), so a block that moves twice inside one placement counts once.
"""
from __future__ import annotations

import pytest

import pager
from oracle import pager_policy as op

BLOCK = 16 * 1024 * 1024
IMPLS = [pytest.param(op.Pager, id="oracle"), pytest.param(pager.PyPager, id="native")]


def metrics_of(p):
    m = p.get_metrics() if isinstance(p, op.Pager) else p.metrics()
    return (m.swap_vram_ram // BLOCK, m.swap_ram_ssd // BLOCK, m.vram_peak // BLOCK, m.ram_peak // BLOCK)


def new(cls, vram, ram, margin, ram_margin, policy="heavy_hitter", interval=1):
    return cls(vram * BLOCK, ram * BLOCK, 0, interval, margin, ram_margin, policy)


@pytest.mark.parametrize("cls", IMPLS)
def test_promote_vram_from_ssd_then_promote_ram(cls):
    """vram 7, ram 2, recent 0, interval 1, margins 0.05 / 0.2; 10 blocks, query block 9.
    Pinned: sinks 0-3 and recent block 9 (recent_start = 9 - 0).

    Step 1, a = [0,0,0,0,50,40,30,20,10,0]: scores [0,0,0,0,5,4,3,2,1,0]. No block is in
    VRAM yet, so the first-placement ranking applies: pinned first (0,1,2,3,9), then score
    descending (4,5,6,7,8). VRAM = ranks 0-6 = {0,1,2,3,9,4,5}, RAM = {6,7}, SSD = {8}.
    Every block started in RAM: 7 RAM->VRAM moves, 1 RAM->SSD.

    Step 2, a = [0,...,0,100 at 8,0]: scores 4: 4.5, 5: 3.6, 6: 2.7, 7: 1.8, 8: 0.9 + 10 =
    10.9, the rest 0. VRAM holds 7 = budget; promote_vram: worst unpinned VRAM of {4: 4.5,
    5: 3.6} is 5, best non-VRAM of {6: 2.7, 7: 1.8, 8: 10.9} is 8; 10.9 - 3.6 > 0.05, so
    8 -> VRAM and 5 -> SSD (8's tier before the swap). Next: worst {4: 4.5, 8: 10.9} = 4,
    best {5: 3.6, 6, 7} = 5, 3.6 - 4.5 <= 0.05: stop. fill_ram: RAM {6, 7} is at budget,
    trim_ram keeps both. promote_ram: worst RAM of {6: 2.7, 7: 1.8} = 7, best SSD {5: 3.6};
    3.6 - 1.8 > 0.2: 5 -> RAM, 7 -> SSD. Next: worst {5: 3.6, 6: 2.7} = 6, best SSD {7: 1.8}:
    stop. Tiers [0,0,0,0,0,1,1,2,0,0]. Against step 1: 5 VRAM->RAM, 7 RAM->SSD, 8 SSD->VRAM
    (counts in both): swap_vram_ram 7 + 2 = 9, swap_ram_ssd 1 + 2 = 3. Peaks 7 and 2."""
    p = new(cls, 7, 2, 0.05, 0.2)
    p.on_step(9, 0, [0, 0, 0, 0, 50, 40, 30, 20, 10, 0])
    assert p.tiers() == [0, 0, 0, 0, 0, 0, 1, 1, 2, 0]
    assert metrics_of(p) == (7, 1, 7, 2)
    p.on_step(9, 0, [0, 0, 0, 0, 0, 0, 0, 0, 100, 0])
    assert p.tiers() == [0, 0, 0, 0, 0, 1, 1, 2, 0, 0]
    assert metrics_of(p) == (9, 3, 7, 2)


@pytest.mark.parametrize("cls", IMPLS)
def test_chain_of_two_vram_swaps_from_ram(cls):
    """vram 7, ram 3, recent 0, interval 1; 11 blocks, query block 10: pinned {0,1,2,3,10}.

    Step 1, scores [0,0,0,0,6,5,4,3,2,1,0]: ranking pinned (0,1,2,3,10) then 4..9 by score.
    VRAM {0,1,2,3,10,4,5}, RAM {6,7,8}, SSD {9}: 7 RAM->VRAM, 1 RAM->SSD.

    Step 2, a = 100 at 6 and 90 at 7: scores 4: 5.4, 5: 4.5, 6: 3.6 + 10 = 13.6,
    7: 2.7 + 9 = 11.7, 8: 1.8, 9: 0.9. promote_vram: worst of {4: 5.4, 5: 4.5} = 5, best
    non-VRAM = 6 (13.6): swap, 5 takes 6's tier RAM. Then worst of {4: 5.4, 6: 13.6} = 4,
    best of {5: 4.5, 7: 11.7, 8, 9} = 7: swap, 4 -> RAM. Then worst of {6: 13.6, 7: 11.7} =
    7, best of {4: 5.4, 5, 8, 9} = 4: 5.4 - 11.7 <= 0.05, stop. RAM {4,5,8} is at its budget
    of 3 (trim keeps it); promote_ram: worst RAM 8 (1.8), best SSD 9 (0.9): stop.
    Tiers [0,0,0,0,1,1,0,0,1,2,0]: 4 swaps VRAM<->RAM, swap_vram_ram 7 + 4 = 11."""
    p = new(cls, 7, 3, 0.05, 0.2)
    p.on_step(10, 0, [0, 0, 0, 0, 60, 50, 40, 30, 20, 10, 0])
    assert p.tiers() == [0, 0, 0, 0, 0, 0, 1, 1, 1, 2, 0]
    p.on_step(10, 0, [0, 0, 0, 0, 0, 0, 100, 90, 0, 0, 0])
    assert p.tiers() == [0, 0, 0, 0, 1, 1, 0, 0, 1, 2, 0]
    assert metrics_of(p) == (11, 1, 7, 3)


@pytest.mark.parametrize("cls", IMPLS)
def test_tied_best_candidates_take_the_last_and_an_exact_margin_does_not_swap(cls):
    """vram 7, ram 10, recent 0, interval 1, promote margin 0.5; 10 blocks, pinned {0,1,2,3,9}.

    Step 1, all scores 0: the first-placement ranking is pinned (0,1,2,3,9), then the tied
    unpinned blocks in id order (stable sort): VRAM {0,1,2,3,9,4,5}, RAM {6,7,8}.

    Step 2, a = [.., 20, 25, 30, 30, 10, 0] on blocks 4..9: scores exactly 2, 2.5, 3, 3, 1, 0
    (0 * 0.9 = 0). Worst unpinned VRAM of {4: 2, 5: 2.5} = 4; best non-VRAM of {6: 3, 7: 3,
    8: 1}: 6 and 7 tie and max_by returns the last, 7. 3 - 2 = 1 > 0.5: 7 -> VRAM, 4 -> RAM.
    Next: worst of {5: 2.5, 7: 3} = 5, best of {4: 2, 6: 3, 8: 1} = 6; the improvement
    3 - 2.5 = 0.5 equals the margin exactly, and `improvement <= margin` stops the loop.
    RAM holds 3 of 10: fill_ram finds no SSD block, promote_ram stops (3 < 10).
    Tiers [0,0,0,0,1,0,1,0,1,0]: with first-max, 6 would be in VRAM instead of 7; with a
    strict comparison, 6 would also replace 5. swap_vram_ram 7 + 2 = 9."""
    p = new(cls, 7, 10, 0.5, 1.0)
    p.on_step(9, 0, [0.0] * 10)
    assert p.tiers() == [0, 0, 0, 0, 0, 0, 1, 1, 1, 0]
    p.on_step(9, 0, [0, 0, 0, 0, 20, 25, 30, 30, 10, 0])
    assert p.tiers() == [0, 0, 0, 0, 1, 0, 1, 0, 1, 0]
    assert metrics_of(p) == (9, 0, 7, 3)


@pytest.mark.parametrize("cls", IMPLS)
def test_tied_worst_vram_blocks_lose_the_first(cls):
    """As above (vram 7, ram 10, margin 0.5, step 1 all zeros: VRAM {0,1,2,3,9,4,5}), then
    scores 4: 2, 5: 2, 6: 3, 7: 0, 8: 0. Worst unpinned VRAM of {4: 2, 5: 2}: a tie, and
    min_by keeps the first, 4; best non-VRAM is 6 (3): 3 - 2 > 0.5, 6 -> VRAM, 4 -> RAM.
    Next: worst of {5: 2, 6: 3} = 5, best of {4: 2, 7: 0, 8: 0} = 4: 2 - 2 = 0, stop.
    Tiers [0,0,0,0,1,0,0,1,1,0] (with last-min, 5 would have left VRAM instead)."""
    p = new(cls, 7, 10, 0.5, 1.0)
    p.on_step(9, 0, [0.0] * 10)
    p.on_step(9, 0, [0, 0, 0, 0, 20, 20, 30, 0, 0, 0])
    assert p.tiers() == [0, 0, 0, 0, 1, 0, 0, 1, 1, 0]
    assert metrics_of(p) == (9, 0, 7, 3)


@pytest.mark.parametrize("cls", IMPLS)
def test_trim_ram_keeps_stable_ascending_order_then_promote_ram_takes_the_last_tie(cls):
    """vram 5, ram 2, recent 0, interval 1, margins 0.05 / 0.2.

    Step 1 (query 5, 6 blocks, a = 10 at block 4): pinned {0,1,2,3,5} fill the 5 VRAM
    slots in the first-placement ranking; RAM {4} (score 1). Tiers [0,0,0,0,1,0]: 5 moves
    RAM->VRAM. Peaks 5 and 1.

    Step 2 (query 9, 10 blocks, all a = 0): blocks 6-9 are created in RAM with score 0;
    block 4 decays to 0.9. Pinned {0,1,2,3,9}: block 5 is no longer pinned. Pinned blocks go
    to VRAM, so VRAM = {0,1,2,3,5,9}, one over budget; enforce_vram keeps pinned first, then
    score: block 5 -> RAM. promote_vram: no unpinned VRAM block, stop. fill_ram: RAM
    {4: 0.9, 5: 0, 6: 0, 7: 0, 8: 0} is over its budget of 2, so trim_ram sorts it by
    ascending score, ties in id order: [5, 6, 7, 8, 4], and sends the 3 first to SSD.
    RAM keeps {4, 8}. promote_ram: worst RAM of {4: 0.9, 8: 0} = 8, best SSD of {5, 6, 7}
    (all 0) = 7: 0 <= 0.2, stop. Tiers [0,0,0,0,1,2,2,2,1,0]. Against the tiers before this
    placement ([0,0,0,0,1,0] plus 6-9 in RAM): 5 VRAM->SSD (both counters), 6 and 7
    RAM->SSD, 9 RAM->VRAM: swap_vram_ram 5 + 2 = 7, swap_ram_ssd 0 + 3 = 3.

    Step 3 (a = 60 at 4, 50 at 6 and 7): scores 4: 0.81 + 6 = 6.81, 6: 5, 7: 5, the rest 0.
    VRAM holds only pinned blocks. RAM {4, 8} is at budget. promote_ram: worst RAM of
    {4: 6.81, 8: 0} = 8, best SSD of {5: 0, 6: 5, 7: 5}: tied, max_by takes the last, 7;
    5 > 0.2: 7 -> RAM, 8 -> SSD. Next: worst of {4: 6.81, 7: 5} = 7, best of {5, 6: 5, 8}
    = 6: 5 - 5 = 0, stop. Tiers [0,0,0,0,1,2,2,1,2,0]; swap_ram_ssd 3 + 2 = 5."""
    p = new(cls, 5, 2, 0.05, 0.2)
    p.on_step(5, 0, [0, 0, 0, 0, 10, 0])
    assert p.tiers() == [0, 0, 0, 0, 1, 0]
    assert metrics_of(p) == (5, 0, 5, 1)
    p.on_step(9, 0, [0.0] * 10)
    assert p.tiers() == [0, 0, 0, 0, 1, 2, 2, 2, 1, 0]
    assert metrics_of(p) == (7, 3, 5, 2)
    p.on_step(9, 0, [0, 0, 0, 0, 60, 0, 50, 50, 0, 0])
    assert p.tiers() == [0, 0, 0, 0, 1, 2, 2, 1, 2, 0]
    assert metrics_of(p) == (7, 5, 5, 2)


@pytest.mark.parametrize("cls", IMPLS)
def test_fill_ram_takes_tied_candidates_in_id_order(cls):
    """sinks_heavy_hitter, vram 4, ram 2, recent 0; 8 blocks, scores [0,0,0,0,2,3,3,3].
    VRAM: the 4 sinks fill the budget (recent budget min(0, 2, 0) = 0, no scored picks).
    fill_ram: RAM is empty, SSD candidates {4,5,6,7} sorted by descending score, ties in id
    order: [5, 6, 7, 4]; the first 2 go to RAM. Tiers [0,0,0,0,2,1,1,2]. From the initial
    RAM tier: 4 RAM->VRAM moves, blocks 4 and 7 RAM->SSD."""
    p = new(cls, 4, 2, 0.05, 0.2, policy="sinks_heavy_hitter", interval=1000)
    p.on_step(7, 0, [0, 0, 0, 0, 20, 30, 30, 30])
    assert p.tiers() == [0, 0, 0, 0, 2, 1, 1, 2]
    assert metrics_of(p) == (4, 2, 4, 2)
