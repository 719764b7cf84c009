"""CPU model of the paged streaming decode step, for use as a test oracle only.

TEST INFRASTRUCTURE. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module; the product never calls it.

Restates, per decode step and session (one session = rows sharing one placement):
  * the store: full blocks on GPU or CPU; ``apply_tiers`` moves blocks in ascending id
    order, tier 0 -> GPU, anything else -> CPU, ids >= len(tiers) -> CPU
    (pager_hf/kv_block_store.py:206-227);
  * the append: the new token joins the tail (paged_model.py:955); when the tail reaches
    tokens_per_block it becomes block ``num_blocks`` (paged_model.py:1210-1233);
  * attention: dense fp32 softmax over every valid token of the row including the new one
    (tests/test_streaming_attention.py:20-40 form; validity = position >= lo, which folds the
    left-padding mask and the sliding-window rule col > pos - W of paged_model.py:977-982;
    a layer with its own window W, as Gemma2's alternating layers have
    (paged_model.py:153-177), also requires position > pos - W);
  * mass: block mass of the full blocks known before the step, mean over (rows, query
    heads), summed over layers (paged_model.py:1041-1048), then averaged and normalized
    (paged_model.py:865-876); uniform when the policy ignores scores (:788-790);
  * placement glue: on_step(N-1, 0, scores), force_rebalance(N-1) when a block was added,
    apply_tiers(tiers()) (paged_model.py:792-799);
  * gather indices: per row, the ascending ids of CPU-resident blocks the step reads
    (paged_model.py:907-916), restricted to blocks holding at least one valid token.

Pinned by tests/test_oracle_paged_decode.py (the reload-path copy counts of
bench/persistent_policy_compare_results.csv rows 2-3 follow from the same store and pager
rules) and by the dense attention pins of tests/test_oracle_attention.py.
"""
from __future__ import annotations

import numpy as np

from .attention import dense_reference
from .pager_policy import Pager

NO_SCORE_POLICIES = frozenset({"recent_only", "sinks_recent"})


def apply_tiers_moves(gpu: set[int], cpu: set[int], tiers) -> tuple[list[int], list[int]]:
    """kv_block_store.py:206-227 index lists; mutates gpu/cpu."""
    to_gpu, to_cpu = [], []
    for block_id in sorted(gpu | cpu):
        desired = tiers[block_id] if block_id < len(tiers) else 2
        if desired == 0:
            if block_id not in gpu:
                cpu.discard(block_id)
                gpu.add(block_id)
                to_gpu.append(block_id)
        elif block_id not in cpu:
            gpu.discard(block_id)
            cpu.add(block_id)
            to_cpu.append(block_id)
    return to_gpu, to_cpu


class _Session:
    def __init__(self, rows, pager, policy, lo, num_layers):
        self.rows = rows
        self.pager = pager
        self.needs_attention = policy not in NO_SCORE_POLICIES
        self.lo = list(lo)
        self.n_tokens = 0
        self.gpu: set[int] = set()
        self.cpu: set[int] = set()
        # keys[layer][row] -> float32 [Hkv, n, D]
        self.keys = [[None] * rows for _ in range(num_layers)]
        self.values = [[None] * rows for _ in range(num_layers)]


class PagedDecodeOracle:
    def __init__(self, *, num_layers, num_query_heads, num_kv_heads, head_dim, tokens_per_block, scale=None,
                 softcap=None):
        self.num_layers = num_layers
        self.hq = num_query_heads
        self.hkv = num_kv_heads
        self.d = head_dim
        self.T = tokens_per_block
        self.n_rep = num_query_heads // num_kv_heads
        self.scale = scale
        self.softcap = softcap
        self.sessions: dict[int, _Session] = {}

    def add_session(self, sid, *, rows=1, vram_budget, ram_budget, recent_window=64, rebalance_interval=4,
                    promote_margin=0.05, ram_promote_margin=0.20, policy="sinks_heavy_hitter", lo=None):
        pg = Pager(vram_budget, ram_budget, recent_window, rebalance_interval, promote_margin, ram_promote_margin,
                   policy)
        self.sessions[sid] = _Session(rows, pg, policy, lo if lo is not None else [0] * rows, self.num_layers)

    def set_lo(self, sid, lo):
        self.sessions[sid].lo = list(lo)

    def prefill(self, sid, keys, values, n_tokens, *, place=True):
        """keys[layer] [rows, Hkv, n_src, D] arrays (any float dtype holding the stored values).
        keys = values = None registers the length only: such a session takes part in
        placement and gather lists (step with compute=False and no q/k/v), not in attention."""
        s = self.sessions[sid]
        for layer in range(self.num_layers if keys is not None else 0):
            for r in range(s.rows):
                for store, src in ((s.keys, keys), (s.values, values)):
                    buf = np.zeros((self.hkv, n_tokens + 256, self.d), np.float32)
                    buf[:, :n_tokens] = np.asarray(src[layer][r][:, :n_tokens], dtype=np.float32)
                    store[layer][r] = buf
        s.n_tokens = n_tokens
        n_blocks = n_tokens // self.T
        s.cpu = set(range(n_blocks))
        if not n_blocks:
            return [], []
        if place:
            s.pager.on_step(n_blocks - 1, 0, [1.0 / n_blocks] * n_blocks)
            s.pager.force_rebalance(n_blocks - 1)
            tiers = s.pager.tiers()
        else:
            tiers = [0] * n_blocks
        return apply_tiers_moves(s.gpu, s.cpu, tiers)

    def host_ids(self, sid, row) -> list[int]:
        s = self.sessions[sid]
        first = max(s.lo[row], 0) // self.T
        n_full = s.n_tokens // self.T
        return [b for b in range(first, n_full) if b in s.cpu]

    def _append(self, sid, r, layer, k1, v1):
        """Appends one token; storage grows by doubling so a step costs O(1) amortized."""
        s = self.sessions[sid]
        n = s.n_tokens
        buf_k, buf_v = s.keys[layer][r], s.values[layer][r]
        if buf_k.shape[1] <= n:
            cap = max(2 * buf_k.shape[1], n + 64)
            nk = np.zeros((self.hkv, cap, self.d), np.float32)
            nv = np.zeros((self.hkv, cap, self.d), np.float32)
            nk[:, :n], nv[:, :n] = buf_k[:, :n], buf_v[:, :n]
            s.keys[layer][r], s.values[layer][r] = buf_k, buf_v = nk, nv
        buf_k[:, n] = np.asarray(k1, np.float32)
        buf_v[:, n] = np.asarray(v1, np.float32)
        return buf_k[:, : n + 1], buf_v[:, : n + 1]

    def step(self, sids, q, k_new, v_new, compute=True, windows=None):
        """q[layer] [S, Hq, D]; k_new/v_new[layer] [S, Hkv, D] (float32 arrays of the stored values);
        with compute=False they may be None (placement and gather lists only). windows[layer]:
        that layer's own sliding window, or None (default: none for every layer).

        Returns a dict with per-layer outputs, per-sequence gather ids, per-session block
        scores handed to the pager and the moves of apply_tiers. With compute=False the
        attention itself is skipped (outputs None; scores then need a score-free policy).
        """
        seqs = [(sid, r) for sid in sids for r in range(self.sessions[sid].rows)]
        gather = [self.host_ids(sid, r) for sid, r in seqs]
        n_mass_old = {sid: self.sessions[sid].n_tokens // self.T for sid in sids}
        mass_accum = {sid: np.zeros(n_mass_old[sid], np.float64) for sid in sids}
        outs = []
        for layer in range(self.num_layers):
            out = np.zeros((len(seqs), self.hq, self.d), np.float32)
            per_session = {sid: [] for sid in sids}
            for i, (sid, r) in enumerate(seqs):
                s = self.sessions[sid]
                if not compute and (k_new is None or s.keys[layer][r] is None):
                    continue  # placement only
                k, v = self._append(sid, r, layer, k_new[layer][i], v_new[layer][i])
                if not compute:
                    continue
                total = k.shape[1]
                # Tokens before the first block holding a valid position carry zero weight:
                # compute over [start, total) and place the block masses at their ids.
                start = (max(s.lo[r], 0) // self.T) * self.T
                lo = s.lo[r]
                window = windows[layer] if windows is not None else None
                if window:  # col > pos - W with pos = total - 1
                    lo = max(lo, total - window)
                valid = (np.arange(start, total) >= lo).astype(np.int32)[None]
                o, mass = dense_reference(
                    np.asarray(q[layer][i], np.float32)[None], k[None, :, start:], v[None, :, start:],
                    n_rep=self.n_rep, tokens_per_block=self.T, valid=valid, scale=self.scale, softcap=self.softcap,
                )
                out[i] = o[0]
                full_mass = np.zeros((self.hq, n_mass_old[sid]), np.float32)
                first = start // self.T
                if n_mass_old[sid] > first:
                    full_mass[:, first:] = mass[0, :, : n_mass_old[sid] - first]
                per_session[sid].append(full_mass)  # [Hq, n_mass_old]
            for sid in sids:
                if n_mass_old[sid] and per_session[sid]:
                    stacked = np.stack(per_session[sid])  # [rows, Hq, n]
                    mass_accum[sid] += stacked.mean(axis=(0, 1))
            outs.append(out if compute else None)
        placement = {}
        for sid in sids:
            s = self.sessions[sid]
            old_blocks = s.n_tokens // self.T
            s.n_tokens += 1
            n_blocks = s.n_tokens // self.T
            added = list(range(old_blocks, n_blocks))
            for b in added:
                s.gpu.add(b)
            if n_blocks == 0:
                placement[sid] = {"added": added, "scores": [], "to_gpu": [], "to_cpu": []}
                continue
            if s.needs_attention:
                if not compute:
                    raise ValueError("attention-scored placement needs compute=True")
                averaged = (mass_accum[sid] / self.num_layers).astype(np.float32).tolist()
                total = sum(averaged)
                scores = [x / total for x in averaged] if total > 0 else [1.0 / n_blocks] * n_blocks
            else:
                scores = [1.0 / n_blocks] * n_blocks
            s.pager.on_step(n_blocks - 1, 0, scores)
            if added:
                s.pager.force_rebalance(n_blocks - 1)
            to_gpu, to_cpu = apply_tiers_moves(s.gpu, s.cpu, s.pager.tiers())
            placement[sid] = {"added": added, "scores": scores, "to_gpu": to_gpu, "to_cpu": to_cpu}
        return {"out": outs, "gather": gather, "placement": placement}
