"""Fused streaming decode over many paged sessions: the hot path of the reference's
patched layer forward (paged_model.py:926-1086) plus its per-step placement glue
(paged_model.py:768-812), batched across sessions.

Per decode step::

    dec.begin_step(handles)                      # plan: which blocks are resident / streamed
    for layer in range(num_layers):
        out = dec.decode_layer(layer, q, k_new, v_new)   # append + attend + mass, one call
    step_stats = dec.end_step()                  # new blocks -> pager.on_step -> apply_tiers

``q`` is [S, Hq, D] (post-RoPE), ``k_new``/``v_new`` [S, Hkv, D], where the S sequences are
the rows of the stepped sessions in order. The current token attends to itself exactly as in
the reference (tail + current token, paged_model.py:955, :984-987): the merge kernel folds it
in from k_new/v_new, and the attention kernel writes it into the session's open block for
later steps. Blocks outside the valid range [lo, position] are neither read nor streamed
(the reference reads and masks them, paged_model.py:961).

Placement glue follows paged_model.py:768-812: with N full blocks after the step,
``on_step(N - 1, 0, scores)`` then ``force_rebalance(N - 1)`` if a block completed, then
``apply_tiers(tiers())``. Scores are uniform ``[1/N]*N`` for recent_only / sinks_recent
(:788-790); otherwise the per-block attention mass of this step, averaged over layers and
normalized to sum 1 (:865-876), with the reference's length rule (one entry per block known
before the step; uniform over N if the total is not positive).
"""
from __future__ import annotations

import logging
from dataclasses import dataclass, field

import torch

import pager as _pager

from .kv_pool import NativeKVPool

logger = logging.getLogger(__name__)

# Warn once host-resident bytes pass this share of ram_budget_bytes (kv_block_store.py:10-13).
_RAM_BUDGET_WARNING_THRESHOLD = 0.8

_POLICIES_WITHOUT_ATTENTION_SIGNAL = frozenset({"recent_only", "sinks_recent"})  # paged_model.py:40


@dataclass
class DecodeSession:
    sid: int
    rows: int
    pager: object
    policy: str
    needs_attention: bool
    lo: list[int]
    step_stats: list[dict] = field(default_factory=list)


class PagedDecoder:
    def __init__(
        self,
        *,
        num_layers: int,
        num_query_heads: int,
        num_kv_heads: int,
        head_dim: int,
        tokens_per_block: int,
        dtype: torch.dtype,
        device: torch.device | str = "cuda",
        pool_blocks: int,
        host_blocks: int,
        staging_blocks: int = 2048,
        staging_buffers: int = 2,
        ram_budget_bytes: int | None = None,
        blocks_per_workgroup: int = 32,
        target_workgroups: int = 0,
        scale: float | None = None,
        softcap: float | None = None,
        stream_mode: str = "direct",
    ):
        self.pool = NativeKVPool(
            num_layers=num_layers,
            num_query_heads=num_query_heads,
            num_kv_heads=num_kv_heads,
            head_dim=head_dim,
            tokens_per_block=tokens_per_block,
            dtype=dtype,
            device=device,
            pool_blocks=pool_blocks,
            host_blocks=host_blocks,
            staging_blocks=staging_blocks,
            staging_buffers=staging_buffers,
            blocks_per_workgroup=blocks_per_workgroup,
            target_workgroups=target_workgroups,
            stream_mode=stream_mode,
        )
        self.pool.set_ram_budget(ram_budget_bytes)
        self._ram_budget = ram_budget_bytes
        self.device = self.pool.device
        self.num_layers = num_layers
        self.num_query_heads = num_query_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.tokens_per_block = tokens_per_block
        self.dtype = dtype
        self.scale = scale
        self.softcap = softcap
        self.sessions: dict[int, DecodeSession] = {}
        self._tokens: dict[int, int] = {}  # session length, mirrored to avoid native round trips
        self._step: list[int] | None = None
        self._mass: torch.Tensor | None = None
        # Persistent per-step mass accumulator [sessions, blocks] with a fixed row stride, so
        # a decode step captured in a graph keeps pointing at valid memory; it is replaced
        # (new pointer) only when a step needs more rows or blocks.
        self._mass_buf: torch.Tensor | None = None
        self._n_mass: list[int] = []

    # -- sessions ------------------------------------------------------------------------
    def add_session(
        self,
        *,
        capacity_tokens: int,
        rows: int = 1,
        vram_budget: int,
        ram_budget: int,
        recent_window: int = 64,
        rebalance_interval: int = 4,
        promote_margin: float = 0.05,
        ram_promote_margin: float = 0.20,
        policy: str = "sinks_heavy_hitter",
        lo: list[int] | None = None,
    ) -> int:
        """A new session; the pager arguments and defaults are PagedModel's (paged_model.py:200-215)."""
        lo = list(lo) if lo is not None else [0] * rows
        sid = self.pool.add_session(rows, capacity_tokens, lo)
        pg = _pager.PyPager(vram_budget, ram_budget, recent_window, rebalance_interval, promote_margin,
                            ram_promote_margin, policy)
        needs = policy not in _POLICIES_WITHOUT_ATTENTION_SIGNAL
        self.sessions[sid] = DecodeSession(sid, rows, pg, policy, needs, lo)
        self.pool.attach_pager(sid, pg._handle, needs)
        self._tokens[sid] = 0
        return sid

    def remove_session(self, sid: int) -> None:
        self.pool.remove_session(sid)
        del self.sessions[sid]
        del self._tokens[sid]

    def set_lo(self, sid: int, lo: list[int]) -> None:
        """First valid position per row (left padding and/or a sliding window bound)."""
        self.pool.set_lo(sid, lo)
        self.sessions[sid].lo = list(lo)

    def reorder_rows(self, sid: int, src_rows: list[int]) -> None:
        """Beam search (kv_block_store.py:229-254): new row r takes old row src_rows[r]'s
        K/V history on either tier and its first valid position; one source per row."""
        sess = self.sessions[sid]
        if len(src_rows) != sess.rows:
            raise ValueError(f"reorder_rows needs {sess.rows} source rows, got {len(src_rows)}")
        self.pool.reorder_rows(sid, src_rows)
        sess.lo = [sess.lo[i] for i in src_rows]

    def prefill(self, sid: int, keys, values, n_tokens: int, *, place: bool = True) -> dict[str, list[int]]:
        """Install a prompt's KV: keys[layer], values[layer] are [rows, Hkv, n_src, D] on this device.

        With place=True the pager places the blocks right away (on_step over a uniform score
        then force_rebalance, as a first decode step would) so that host blocks are streamed
        from the first step; with place=False every full block starts in HBM, like the
        reference's initial store (paged_model.py:1183-1192): logically, that is. Only as many
        as the HBM pool has room for (keeping two slots per row free) get a slot, the most
        recent first; the others are written to their host records and read from there until
        the first placement loads or evicts them (pgr_kv_apply_tiers).
        """
        s = self.sessions[sid]
        self.pool.set_length(sid, n_tokens)
        self._tokens[sid] = n_tokens
        n_blocks = n_tokens // self.tokens_per_block
        moves = {"to_gpu": [], "to_cpu": []}
        if n_blocks:
            if place:
                s.pager.on_step(n_blocks - 1, 0, [1.0 / n_blocks] * n_blocks)
                s.pager.force_rebalance(n_blocks - 1)
                tiers = s.pager.tiers()
            else:
                tiers = [0] * n_blocks
            to_gpu, to_cpu, rc, fail_block = self.pool.apply_tiers(sid, tiers)
            if rc != 0:
                raise RuntimeError(f"ram_budget exceeded while placing block {fail_block}")
            moves = {"to_gpu": to_gpu, "to_cpu": to_cpu}
            host_ids = [b for b in range(n_blocks) if b >= len(tiers) or tiers[b] != 0]
            if host_ids:  # prompt blocks placed host-side count as offloaded (kv_block_store.py:101-108)
                self._warn_ram_usage(host_ids[-1])
        if n_tokens:
            for layer in range(self.num_layers):
                for row in range(s.rows):
                    self.pool.import_tokens(sid, row, layer, keys[layer][row], values[layer][row], n_tokens)
        return moves

    def _warn_ram_usage(self, block_id: int) -> None:
        """The reference's warning when an offload leaves host-resident bytes above 80% of the
        RAM budget (kv_block_store.py:101-108)."""
        if not self._ram_budget:
            return
        cpu = self.pool.resident_bytes()[1]
        if cpu > _RAM_BUDGET_WARNING_THRESHOLD * self._ram_budget:
            logger.warning("ram_budget usage at %.0f%% after offloading block %d (%.2f MB of %.2f MB budget).",
                           100.0 * cpu / self._ram_budget, block_id, cpu / 1_000_000, self._ram_budget / 1_000_000)

    def num_blocks(self, sid: int) -> int:
        return self.pool.session_info(sid)[1]

    def num_tokens(self, sid: int) -> int:
        return self.pool.session_info(sid)[0]

    # -- decode --------------------------------------------------------------------------
    def begin_step(self, sids: list[int]) -> None:
        if self._step is not None:
            raise RuntimeError("begin_step called while a step is open")
        self.pool.begin_step(list(sids))
        self._step = list(sids)
        self._n_mass = [self._tokens[sid] // self.tokens_per_block for sid in sids]
        for sid in sids:
            self._tokens[sid] += 1
        if any(self.sessions[sid].needs_attention for sid in sids):
            rows, width = len(sids), max(self._n_mass) + 1
            buf = self._mass_buf
            if buf is None or buf.shape[0] < rows or buf.shape[1] < width:
                r = max(rows, 0 if buf is None else buf.shape[0])
                w = max(2 * width, 0 if buf is None else buf.shape[1])
                buf = self._mass_buf = torch.empty((r, w), dtype=torch.float32, device=self.device)
            buf[:rows, :width].zero_()
            self._mass = buf
        else:
            self._mass = None

    def num_sequences(self) -> int:
        return sum(self.sessions[sid].rows for sid in (self._step or []))

    def decode_layer(self, layer: int, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                     out: torch.Tensor | None = None, *, scale: float | None = None,
                     softcap: float | None = None, window: int | None = None) -> torch.Tensor:
        """Append k_new/v_new, attend q over every valid stored token plus the new one, and
        accumulate this layer's block mass. scale/softcap override the decoder's defaults.
        window: this layer's own sliding window (models whose layers alternate between
        windowed and global attention): stored positions <= current - window are masked as
        well, by the rule col > pos - W of paged_model.py:977-982."""
        if self._step is None:
            raise RuntimeError("decode_layer outside begin_step/end_step")
        S = self.num_sequences()
        exp_q = (S, self.num_query_heads, self.head_dim)
        exp_kv = (S, self.num_kv_heads, self.head_dim)
        if tuple(q.shape) != exp_q or tuple(k_new.shape) != exp_kv or tuple(v_new.shape) != exp_kv:
            raise ValueError(f"expected q {exp_q}, k_new/v_new {exp_kv}")
        for t in (q, k_new, v_new):
            if t.dtype != self.dtype or t.device != self.device:
                raise TypeError(f"q/k_new/v_new must be {self.dtype} on {self.device}")
        q, k_new, v_new = q.contiguous(), k_new.contiguous(), v_new.contiguous()
        if out is None:
            out = torch.empty(exp_q, dtype=self.dtype, device=self.device)
        self.pool.decode_layer(layer, q, k_new, v_new, out, self._mass, self.scale if scale is None else scale,
                               self.softcap if softcap is None else softcap, window)
        return out

    def step_host_blocks(self, seq: int) -> list[int]:
        """Ascending host-resident block ids streamed for sequence `seq` in the open step."""
        return self.pool.step_host_blocks(seq)

    def end_step(self, *, collect: bool = True) -> dict[int, dict]:
        """Close the step and place blocks natively (one call for every session).

        With collect=True returns per-session step stats in the reference's terms
        (paged_model.py:801-812): new blocks, moves, the scores handed to the pager and the
        share of them that sits in HBM after placement; with collect=False returns {}.
        """
        if self._step is None:
            raise RuntimeError("end_step without begin_step")
        sids = self._step
        blocks_after = [n + 1 for n in self._n_mass]  # upper bound on full blocks after the step
        cap = sum(blocks_after)
        try:  # the native call closes the step even when placement then fails
            rc, completed, rows, moves, scores = self.pool.end_step_place(
                len(sids), self._mass, self.num_layers, cap, cap if collect else 0
            )
        finally:
            self._step = None
            self._mass = None
        if rc != 0:
            bad = next(r[3] for r in rows if r[3] >= 0)
            raise RuntimeError(f"ram_budget exceeded: moving block {bad} to CPU")
        mo, last_to_cpu = 0, None
        for _, ng, nc, _, _ in rows:
            if nc:
                last_to_cpu = moves[mo + ng + nc - 1]
            mo += ng + nc
        if last_to_cpu is not None:
            self._warn_ram_usage(last_to_cpu)
        if not collect:
            return {}
        results = {}
        mo = so = 0
        bb = None
        for sid, (added, ng, nc, _, ns) in zip(sids, rows):
            to_gpu = list(moves[mo: mo + ng])
            to_cpu = list(moves[mo + ng: mo + ng + nc])
            mo += ng + nc
            block_attention = list(scores[so: so + ns])
            so += ns
            gpu_ids = self.pool.block_ids(sid, True) if ns else []
            bb = self.pool.block_bytes(sid) if bb is None else bb
            st = {
                "new_blocks": int(added >= 0),
                "added_block_ids": [added] if added >= 0 else [],
                "to_gpu": to_gpu,
                "to_cpu": to_cpu,
                "gpu_to_cpu_mb": nc * bb / 1_000_000,
                "gpu_to_cpu_copies": nc,
                "attention_in_gpu": sum(block_attention[b] for b in gpu_ids if b < len(block_attention)),
                "block_attention": block_attention,
            }
            self.sessions[sid].step_stats.append(st)
            results[sid] = st
        return results
