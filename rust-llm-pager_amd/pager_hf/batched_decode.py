"""Cross-session batched decode over one shared native paged store.

Replaces the reference's batched_decode_step (pager_hf/batched_decode.py:32-236), which
advanced several single-row PagedModel sessions in one model.forward() but only when they
shared a tail length, padded every session to the longest history and rejected sliding-window
models. Here all sessions live in one PagedDecoder (one HBM pool, one pinned host mirror,
per-session block tables and pagers), so any set of sessions -- ragged lengths, any tail
length, per-row window bounds -- advances in one forward whose attention is one native launch
pair per layer.

    engine = BatchedPagedEngine(model, max_sessions=64, vram_budget_per_session=..., ...)
    h = engine.open(prompt_ids, prompt_mask, capacity_tokens)   # prefill all but the last token
    logits = engine.step([h1, h2, ...], [tok1, tok2, ...])        # one token per session
    engine.close(h)

Placement per session follows the reference's PagedModel exactly: a fresh session's blocks
all start in HBM (paged_model.py:1183-1192) and its pager places them after each step
(paged_model.py:768-812).
"""
from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass, field

import torch
from transformers.cache_utils import DynamicCache

from .paged_decode import PagedDecoder
from .paged_model import _ATTN_IMPL, _LayerContext, PagedModel

BLOCK_SIZE_BYTES = 16 * 1024 * 1024  # the pager's logical block size (core.rs:6)


@dataclass
class EngineSession:
    sid: int
    pads: int              # leading padding tokens of the row (never attended)
    columns: int           # tokens stored so far, padding included
    capacity: int
    steps: int = 0
    stats: list[dict] = field(default_factory=list)


class BatchedPagedEngine:
    def __init__(
        self,
        model,
        *,
        max_sessions: int,
        vram_budget_per_session: int,
        ram_budget_per_session: int,
        policy: str = "sinks_heavy_hitter",
        tokens_per_block: int = 16,
        recent_window: int = 64,
        rebalance_interval: int = 4,
        promote_margin: float = 0.05,
        ram_promote_margin: float = 0.20,
        max_context_tokens: int = 8192,
        host_token_capacity: int | None = None,
        prefill_chunk_tokens: int = 512,
        stream_mode: str = "direct",
        staging_blocks: int = 64,
        staging_buffers: int = 2,
        collect_stats: bool = False,
    ):
        """``max_context_tokens``: most tokens one session may hold (prompt + generated);
        ``host_token_capacity``: tokens the pinned host mirror holds over all sessions
        (default max_sessions * max_context_tokens); ``staging_blocks`` / ``staging_buffers``:
        the HBM staging ring of the staged stream mode (records per buffer, buffers)."""
        if max_sessions < 1:
            raise ValueError("max_sessions must be >= 1")
        self.model = model
        self._helper = PagedModel(model, vram_budget=vram_budget_per_session, ram_budget=ram_budget_per_session,
                                  tokens_per_block=tokens_per_block, prefill_chunk_tokens=prefill_chunk_tokens)
        layers, hq, hkv, d, window = self._helper._model_geometry()
        self.num_layers, self.window = layers, window
        self.tokens_per_block = T = tokens_per_block
        self.max_context_tokens = max_context_tokens
        self.collect_stats = collect_stats
        dtype = next(model.parameters()).dtype
        device = next(model.parameters()).device
        self.device = device
        vram_blocks = max(1, vram_budget_per_session // BLOCK_SIZE_BYTES)
        # HBM: every session's budget plus its open block and a block completed in a step before
        # its placement. A fresh session's prompt needs no room of its own: its blocks count as
        # HBM-resident until the first placement, but only those the pool has room for get a
        # slot (the others are read from their host records until then).
        pool = max_sessions * (vram_blocks + 2) + 16
        host_tokens = host_token_capacity if host_token_capacity is not None else max_sessions * max_context_tokens
        host = -(-host_tokens // T) + max_sessions * 2
        self.decoder = PagedDecoder(
            num_layers=layers, num_query_heads=hq, num_kv_heads=hkv, head_dim=d, tokens_per_block=T, dtype=dtype,
            device=device, pool_blocks=pool, host_blocks=host, staging_blocks=staging_blocks,
            staging_buffers=staging_buffers, stream_mode=stream_mode,
        )
        self._pager_kwargs = dict(vram_budget=vram_budget_per_session, ram_budget=ram_budget_per_session,
                                  recent_window=recent_window, rebalance_interval=rebalance_interval,
                                  promote_margin=promote_margin, ram_promote_margin=ram_promote_margin, policy=policy)
        self.sessions: dict[int, EngineSession] = {}

    # -- sessions --------------------------------------------------------------------------
    @torch.inference_mode()
    def open(self, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None,
             capacity_tokens: int | None = None) -> EngineSession:
        """Prefill all but the last token of one row ([1, n]); the caller feeds the last token
        with the session's first step."""
        if input_ids.dim() != 2 or input_ids.shape[0] != 1:
            raise ValueError("open() takes one row: input_ids [1, n]")
        n = input_ids.shape[1]
        if attention_mask is None:
            attention_mask = torch.ones_like(input_ids)
        PagedModel._validate_left_padded(attention_mask)
        capacity = capacity_tokens if capacity_tokens is not None else self.max_context_tokens
        if capacity > self.max_context_tokens or capacity < n + 1:
            raise ValueError(f"capacity_tokens must be in [{n + 1}, {self.max_context_tokens}]")
        pads = int(attention_mask.shape[1] - attention_mask.long().sum().item())
        sid = self.decoder.add_session(capacity_tokens=capacity + self.tokens_per_block, rows=1, lo=[pads],
                                       **self._pager_kwargs)
        try:
            if n > 1:
                past = self._helper._chunked_prefill(input_ids[:, :-1], attention_mask[:, :-1])
                keys = [past.layers[i].keys for i in range(self.num_layers)]
                values = [past.layers[i].values for i in range(self.num_layers)]
                self.decoder.prefill(sid, keys, values, n - 1, place=False)
                del past, keys, values
        except BaseException:
            self.decoder.remove_session(sid)
            raise
        s = EngineSession(sid=sid, pads=pads, columns=n - 1, capacity=capacity)
        self.sessions[sid] = s
        return s

    def close(self, s: EngineSession) -> None:
        if self.sessions.pop(s.sid, None) is not None:
            self.decoder.remove_session(s.sid)

    # -- decode ----------------------------------------------------------------------------
    @contextmanager
    def _paged_attention(self):
        cfg = self.model.config
        previous = cfg._attn_implementation
        ctx = _LayerContext(self.decoder, None)
        modules = [layer.self_attn for layer in self.model.model.layers]
        for m in modules:
            m._pgr_ctx = ctx
        cfg._attn_implementation = _ATTN_IMPL
        try:
            yield
        finally:
            cfg._attn_implementation = previous
            for m in modules:
                m._pgr_ctx = None

    @torch.inference_mode()
    def step(self, sessions: list[EngineSession], input_tokens: list[int]) -> torch.Tensor:
        """Feed one token to each session in one forward; returns their next-token logits [S, V]."""
        if len(sessions) != len(input_tokens):
            raise ValueError("one input token per session")
        if not sessions:
            return torch.empty(0, device=self.device)
        if len({s.sid for s in sessions}) != len(sessions):
            raise ValueError("a session appears twice in one step")
        for s in sessions:
            if s.columns + 1 > s.capacity:
                raise ValueError(f"session {s.sid} reached its capacity of {s.capacity} tokens")
            if self.window is not None:
                self.decoder.set_lo(s.sid, [max(s.pads, s.columns - self.window + 1)])
        dec = self.decoder
        sids = [s.sid for s in sessions]
        ids = torch.tensor(input_tokens, dtype=torch.long, device=self.device).unsqueeze(1)
        pos = torch.tensor([s.columns - s.pads for s in sessions], dtype=torch.long, device=self.device).unsqueeze(1)
        dec.begin_step(sids)
        try:
            with self._paged_attention():
                out = self.model(input_ids=ids, position_ids=pos, use_cache=False, logits_to_keep=1)
        except BaseException:
            dec.end_step(collect=False)
            raise
        stats = dec.end_step(collect=self.collect_stats)
        for s in sessions:
            s.columns += 1
            s.steps += 1
            if self.collect_stats:
                s.stats.append(stats[s.sid])
        return out.logits[:, -1, :]

    def host_bytes_per_step(self) -> int:
        """K/V bytes the last step read over the host link (all layers)."""
        st = self.decoder.pool.step_stats()
        return st["host_tokens"] * 2 * self.decoder.num_kv_heads * self.decoder.head_dim * 2 * self.num_layers
