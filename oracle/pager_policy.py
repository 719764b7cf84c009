"""CPU restatement of the reference's Rust placement policy, for use as a test oracle only.

TEST INFRASTRUCTURE. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only to check or time the product;
the product (``pager.PyPager`` over the native C++ core) never calls into it.

Follows ``pager/src/core.rs`` (the whole file), ``pager/src/lib.rs:17-25`` (defaults)
and ``pager/src/metrics.rs:4-27``. Every f32 operation is carried out in IEEE single
precision with ``numpy.float32`` scalars and no fused multiply-add, as Rust does.

Rust semantics reproduced exactly:
  * ``slice::sort_by`` is stable: :func:`_stable_sort` uses Python's stable sort.
  * ``Iterator::min_by`` keeps the FIRST of equal minima, ``max_by`` returns the
    LAST of equal maxima (core.rs:479-513).
  * ``compare_scores`` treats NaN as Equal (core.rs:553-555).
  * PyO3 turns Python floats into f32 by round-to-nearest (lib.rs:48).

Pinned by: tests/test_oracle_pager.py (the ten Rust unit tests of core.rs:582-704 as
properties, the README.md:389 placement list, bench/persistent_policy_compare_results.csv
rows 2-3, and hand-worked cases for each helper) and tests/test_oracle_pager_hysteresis.py
(hand-derived cases that run every swap of promote_vram_with_hysteresis and
promote_ram_with_hysteresis and every trim of trim_ram, with exact-margin and tie cases).
"""
from __future__ import annotations

import functools

import numpy as np

BLOCK_SIZE_BYTES = 16 * 1024 * 1024  # core.rs:6
SINK_BLOCKS = 4  # core.rs:7

VRAM, RAM, SSD = 0, 1, 2  # core.rs:10-14 and the u8 mapping of core.rs:113-122

RECENT_ONLY, SINKS_RECENT, HEAVY_HITTER, SINKS_HEAVY_HITTER = range(4)

_F32_090 = np.float32(0.90)
_F32_010 = np.float32(0.10)


def policy_from_name(name: str) -> int:
    """core.rs:24-33: unknown names fall back to heavy_hitter."""
    return {
        "recent_only": RECENT_ONLY,
        "sinks_recent": SINKS_RECENT,
        "heavy_hitter": HEAVY_HITTER,
        "sinks_heavy_hitter": SINKS_HEAVY_HITTER,
    }.get(name, HEAVY_HITTER)


def compare_scores(a: np.float32, b: np.float32) -> int:
    """core.rs:553-555: partial_cmp, NaN -> Equal. Returns -1/0/1."""
    if a < b:
        return -1
    if a > b:
        return 1
    return 0


def _stable_sort(items: list, cmp) -> list:
    return sorted(items, key=functools.cmp_to_key(cmp))


def _min_by_first(indices, key_of):
    """Iterator::min_by: running x vs next y -> keep x unless compare(x, y) == Greater."""
    best = None
    for idx in indices:
        if best is None or compare_scores(key_of(best), key_of(idx)) > 0:
            best = idx
    return best


def _max_by_last(indices, key_of):
    """Iterator::max_by: running x vs next y -> take y unless compare(x, y) == Greater."""
    best = None
    for idx in indices:
        if best is None or compare_scores(key_of(best), key_of(idx)) <= 0:
            best = idx
    return best


class Metrics:
    """metrics.rs:4-27."""

    __slots__ = (
        "tokens",
        "vram_peak",
        "ram_peak",
        "swap_vram_ram",
        "swap_ram_ssd",
        "attention_mass_total",
        "attention_mass_vram",
    )

    def __init__(self):
        self.tokens = 0
        self.vram_peak = 0
        self.ram_peak = 0
        self.swap_vram_ram = 0
        self.swap_ram_ssd = 0
        self.attention_mass_total = 0.0
        self.attention_mass_vram = 0.0

    def snapshot(self) -> "Metrics":
        out = Metrics()
        for name in self.__slots__:
            setattr(out, name, getattr(self, name))
        return out


class Block:
    __slots__ = ("id", "size", "score", "tier", "pinned")

    def __init__(self, block_id: int):
        self.id = block_id
        self.size = BLOCK_SIZE_BYTES
        self.score = np.float32(0.0)
        self.tier = RAM  # core.rs:139: new blocks start in RAM
        self.pinned = False


class Pager:
    """core.rs:56-551, driven the way lib.rs:16-66 drives it."""

    def __init__(
        self,
        vram: int,
        ram: int,
        recent: int,
        rebalance_interval: int = 32,
        promote_margin: float = 0.10,
        ram_promote_margin: float = 0.20,
        policy: str = "heavy_hitter",
    ):
        for name, value in (("vram", vram), ("ram", ram), ("recent", recent), ("rebalance_interval", rebalance_interval)):
            if value < 0:
                raise OverflowError(f"{name} must be non-negative")
        self.vram = int(vram)
        self.ram = int(ram)
        self.recent_window = int(recent)
        self.rebalance_interval = int(rebalance_interval)
        self.promote_margin = np.float32(promote_margin)
        self.ram_promote_margin = np.float32(ram_promote_margin)
        self.policy = policy_from_name(policy)
        self.metrics = Metrics()
        self.blocks: list[Block] = []

    # -- public surface (lib.rs:48-66) ---------------------------------------------------
    def on_step(self, token_idx: int, layer: int, attention) -> None:
        """core.rs:87-98."""
        if token_idx < 0 or layer < 0:
            raise OverflowError("can't convert negative int to unsigned")
        attention = [np.float32(a) for a in attention]
        self.metrics.tokens += 1
        self._ensure_blocks(len(attention))
        self._update_scores(attention)
        self._update_attention_quality(attention)
        self._pin_blocks(token_idx)
        if self.metrics.tokens == 1:
            self.force_rebalance(token_idx)
            return
        if self.rebalance_interval == 0:
            raise ZeroDivisionError("attempt to calculate the remainder with a divisor of zero")
        if self.metrics.tokens % self.rebalance_interval == 0:
            self.force_rebalance(token_idx)

    def force_rebalance(self, token_idx: int) -> None:
        """core.rs:100-107."""
        if token_idx < 0:
            raise OverflowError("can't convert negative int to unsigned")
        self._ensure_blocks(token_idx + 1)
        self._pin_blocks(token_idx)
        self._place_blocks()
        self._update_memory_peaks()

    def tiers(self) -> list[int]:
        return [block.tier for block in self.blocks]

    def vram_block_ids(self) -> list[int]:
        return [block.id for block in self.blocks if block.tier == VRAM]

    def get_metrics(self) -> Metrics:
        return self.metrics.snapshot()

    # -- internals -----------------------------------------------------------------------
    def _ensure_blocks(self, count: int) -> None:
        while len(self.blocks) < count:
            self.blocks.append(Block(len(self.blocks)))

    def _update_scores(self, attention) -> None:
        """core.rs:145-149: score = score*0.90 + a*0.10 in f32, no FMA."""
        for block, a in zip(self.blocks, attention):
            block.score = np.float32(np.float32(block.score * _F32_090) + np.float32(a * _F32_010))

    def _update_attention_quality(self, attention) -> None:
        """core.rs:151-165 (f64 sums, tier as of before this step's placement)."""
        total = 0.0
        vram = 0.0
        for block, a in zip(self.blocks, attention):
            value = float(a)
            total += value
            if block.tier == VRAM:
                vram += value
        self.metrics.attention_mass_total += total
        self.metrics.attention_mass_vram += vram

    def _pin_blocks(self, token_idx: int) -> None:
        """core.rs:167-181."""
        recent_start = max(token_idx - self.recent_window, 0)
        for block in self.blocks:
            is_recent = block.id >= recent_start
            is_sink = block.id < SINK_BLOCKS
            if self.policy == RECENT_ONLY:
                block.pinned = is_recent
            else:
                block.pinned = is_recent or is_sink

    def _place_blocks(self) -> None:
        """core.rs:183-199."""
        old_tiers = [block.tier for block in self.blocks]
        max_vram = self.vram // BLOCK_SIZE_BYTES
        max_ram = self.ram // BLOCK_SIZE_BYTES
        if self.policy in (RECENT_ONLY, SINKS_RECENT):
            self._place_baseline(old_tiers, max_vram, max_ram)
        elif self.policy == HEAVY_HITTER:
            self._place_heavy_hitter(old_tiers, max_vram, max_ram)
        else:
            self._place_sinks_heavy_hitter(old_tiers, max_vram, max_ram)

    def _place_baseline(self, old_tiers, max_vram, max_ram) -> None:
        """core.rs:201-219: (pinned desc, id asc)."""
        blocks = self.blocks

        def cmp(a, b):
            by_pin = (blocks[b].pinned > blocks[a].pinned) - (blocks[b].pinned < blocks[a].pinned)
            if by_pin:
                return by_pin
            return (blocks[a].id > blocks[b].id) - (blocks[a].id < blocks[b].id)

        ranked = _stable_sort(list(range(len(blocks))), cmp)
        self._reset_tiers(SSD)
        self._assign_ranked(ranked, max_vram, max_ram)
        self._count_tier_changes(old_tiers)

    def _pinned_then_score_desc(self, a: int, b: int) -> int:
        blocks = self.blocks
        by_pin = (blocks[b].pinned > blocks[a].pinned) - (blocks[b].pinned < blocks[a].pinned)
        if by_pin:
            return by_pin
        return compare_scores(blocks[b].score, blocks[a].score)

    def _place_heavy_hitter(self, old_tiers, max_vram, max_ram) -> None:
        """core.rs:221-255."""
        if not any(block.tier == VRAM for block in self.blocks):
            ranked = _stable_sort(list(range(len(self.blocks))), self._pinned_then_score_desc)
            self._assign_ranked(ranked, max_vram, max_ram)
            self._count_tier_changes(old_tiers)
            return
        for block in self.blocks:
            if block.pinned:
                block.tier = VRAM
        self._enforce_vram_budget_keep_best(max_vram)
        self._promote_vram_with_hysteresis(max_vram)
        self._fill_ram(max_ram)
        self._promote_ram_with_hysteresis(max_ram)
        self._count_tier_changes(old_tiers)

    def _place_sinks_heavy_hitter(self, old_tiers, max_vram, max_ram) -> None:
        """core.rs:257-318."""
        self._reset_tiers(SSD)
        if max_vram == 0:
            self._count_tier_changes(old_tiers)
            return
        selected: set[int] = set()
        for block in self.blocks[:SINK_BLOCKS]:
            if len(selected) >= max_vram:
                break
            selected.add(block.id)
        remaining = max(max_vram - len(selected), 0)
        recent_budget = min(self.recent_window, max(max_vram // 2, 1), remaining)
        recent_start = max(len(self.blocks) - recent_budget, 0)
        for block in self.blocks[recent_start:]:
            if len(selected) >= max_vram:
                break
            selected.add(block.id)
        scored = [(block.id, block.score) for block in self.blocks if block.id not in selected]
        scored = _stable_sort(scored, lambda a, b: compare_scores(b[1], a[1]))
        for block_id, _ in scored:
            if len(selected) >= max_vram:
                break
            selected.add(block_id)
        for block in self.blocks:
            if block.id in selected:
                block.tier = VRAM
        self._fill_ram(max_ram)
        self._count_tier_changes(old_tiers)

    def _assign_ranked(self, ranked, max_vram, max_ram) -> None:
        """core.rs:320-335."""
        for rank, idx in enumerate(ranked):
            if rank < max_vram:
                self.blocks[idx].tier = VRAM
            elif rank < max_vram + max_ram:
                self.blocks[idx].tier = RAM
            else:
                self.blocks[idx].tier = SSD

    def _reset_tiers(self, tier: int) -> None:
        for block in self.blocks:
            block.tier = tier

    def _enforce_vram_budget_keep_best(self, max_vram: int) -> None:
        """core.rs:343-366."""
        vram_ids = [i for i, block in enumerate(self.blocks) if block.tier == VRAM]
        if len(vram_ids) <= max_vram:
            return
        vram_ids = _stable_sort(vram_ids, self._pinned_then_score_desc)
        for idx in vram_ids[max_vram:]:
            self.blocks[idx].tier = RAM

    def _promote_vram_with_hysteresis(self, max_vram: int) -> None:
        """core.rs:368-400."""
        blocks = self.blocks
        score_of = lambda i: blocks[i].score  # noqa: E731
        while True:
            vram_count = sum(1 for block in blocks if block.tier == VRAM)
            if vram_count < max_vram:
                best = _max_by_last((i for i, b in enumerate(blocks) if b.tier != VRAM), score_of)
                if best is not None:
                    blocks[best].tier = VRAM
                    continue
                break
            worst = _min_by_first((i for i, b in enumerate(blocks) if b.tier == VRAM and not b.pinned), score_of)
            if worst is None:
                break
            best = _max_by_last((i for i, b in enumerate(blocks) if b.tier != VRAM), score_of)
            if best is None:
                break
            improvement = np.float32(blocks[best].score - blocks[worst].score)
            if improvement <= self.promote_margin:
                break
            previous_best_tier = blocks[best].tier
            blocks[best].tier = VRAM
            blocks[worst].tier = previous_best_tier

    def _fill_ram(self, max_ram: int) -> None:
        """core.rs:402-427."""
        current = sum(1 for block in self.blocks if block.tier == RAM)
        if current >= max_ram:
            self._trim_ram(max_ram)
            return
        candidates = [i for i, block in enumerate(self.blocks) if block.tier == SSD]
        blocks = self.blocks
        candidates = _stable_sort(candidates, lambda a, b: compare_scores(blocks[b].score, blocks[a].score))
        for idx in candidates[: max_ram - current]:
            blocks[idx].tier = RAM

    def _trim_ram(self, max_ram: int) -> None:
        """core.rs:429-448."""
        ram_ids = [i for i, block in enumerate(self.blocks) if block.tier == RAM]
        if len(ram_ids) <= max_ram:
            return
        blocks = self.blocks
        ram_ids = _stable_sort(ram_ids, lambda a, b: compare_scores(blocks[a].score, blocks[b].score))
        for idx in ram_ids[: len(ram_ids) - max_ram]:
            blocks[idx].tier = SSD

    def _promote_ram_with_hysteresis(self, max_ram: int) -> None:
        """core.rs:450-477."""
        blocks = self.blocks
        score_of = lambda i: blocks[i].score  # noqa: E731
        while True:
            ram_count = sum(1 for block in blocks if block.tier == RAM)
            if ram_count < max_ram:
                break
            worst = _min_by_first((i for i, b in enumerate(blocks) if b.tier == RAM), score_of)
            if worst is None:
                break
            best = _max_by_last((i for i, b in enumerate(blocks) if b.tier == SSD), score_of)
            if best is None:
                break
            improvement = np.float32(blocks[best].score - blocks[worst].score)
            if improvement <= self.ram_promote_margin:
                break
            blocks[best].tier = RAM
            blocks[worst].tier = SSD

    def _count_tier_changes(self, old_tiers) -> None:
        """core.rs:515-531."""
        for block, old in zip(self.blocks, old_tiers):
            pair = (old, block.tier)
            if pair in ((VRAM, RAM), (RAM, VRAM)):
                self.metrics.swap_vram_ram += block.size
            elif pair in ((RAM, SSD), (SSD, RAM)):
                self.metrics.swap_ram_ssd += block.size
            elif pair in ((VRAM, SSD), (SSD, VRAM)):
                self.metrics.swap_vram_ram += block.size
                self.metrics.swap_ram_ssd += block.size

    def _update_memory_peaks(self) -> None:
        """core.rs:533-550."""
        vram_used = sum(block.size for block in self.blocks if block.tier == VRAM)
        ram_used = sum(block.size for block in self.blocks if block.tier == RAM)
        self.metrics.vram_peak = max(self.metrics.vram_peak, vram_used)
        self.metrics.ram_peak = max(self.metrics.ram_peak, ram_used)


def selection_margin(pager: Pager) -> dict:
    """How close the pager's last placement came to a different choice, for reporting.

    sinks_heavy_hitter (core.rs:257-318): after the sinks and the recent budget, the scored
    blocks are taken best first; returns the EMA score gap between the last block taken and
    the first block left out (``gap``), with their ids and the number taken by score.
    heavy_hitter (core.rs:368-400): ``gap`` = promote_margin - (best non-VRAM score - worst
    unpinned VRAM score), i.e. how far the last comparison was from a swap. Other policies
    ignore scores: gap None. Computed from the pager's current tiers and scores."""
    blocks = pager.blocks
    max_vram = pager.vram // BLOCK_SIZE_BYTES
    if pager.policy == SINKS_HEAVY_HITTER and max_vram > 0:
        fixed = set(b.id for b in blocks[:SINK_BLOCKS][:max_vram])
        remaining = max(max_vram - len(fixed), 0)
        recent_budget = min(pager.recent_window, max(max_vram // 2, 1), remaining)
        for b in blocks[max(len(blocks) - recent_budget, 0):]:
            if len(fixed) >= max_vram:
                break
            fixed.add(b.id)
        scored = _stable_sort([(b.id, b.score) for b in blocks if b.id not in fixed],
                              lambda a, b: compare_scores(b[1], a[1]))
        n_taken = min(max(max_vram - len(fixed), 0), len(scored))
        if 0 < n_taken < len(scored):
            last, first_out = scored[n_taken - 1], scored[n_taken]
            return {"gap": float(last[1]) - float(first_out[1]), "taken": n_taken, "last": last[0],
                    "first_out": first_out[0]}
        return {"gap": None, "taken": n_taken}
    if pager.policy == HEAVY_HITTER:
        vram = [b for b in blocks if b.tier == VRAM and not b.pinned]
        other = [b for b in blocks if b.tier != VRAM]
        if vram and other:
            worst = min(float(b.score) for b in vram)
            best = max(float(b.score) for b in other)
            return {"gap": float(pager.promote_margin) - (best - worst)}
    return {"gap": None}
