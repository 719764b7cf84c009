"""PagedModel: a HuggingFace causal LM whose KV cache is paged between HBM and host RAM.

Same public surface as the reference's ``pager_hf.PagedModel`` (paged_model.py:179-409):
the constructor arguments and defaults, ``generate(input_ids, attention_mask,
max_new_tokens, *, do_sample, temperature, top_k, top_p, generator)``, ``reset()``, the
session that persists across generate() calls, ``last_run_stats`` (GenerationStats) and the
one-call-at-a-time lock. What runs underneath is the native path:

* prefill: the model's own attention over the prompt (minus its last token) in chunks of
  ``prefill_chunk_tokens`` (paged_model.py:1121-1161); the resulting K/V is imported into the
  native store with every full block resident in HBM, as the reference's initial store is
  (paged_model.py:1183-1192);
* decode: one token per step. The model runs with the attention implementation registered
  here, which hands each layer's post-RoPE q / k_new / v_new to PagedDecoder.decode_layer:
  append, attention over HBM and host blocks, block mass -- in place of the reference's
  patched layer forward (paged_model.py:926-1086). After the step the native placement glue
  runs on_step / force_rebalance / apply_tiers (paged_model.py:768-812).

``generate_beam_search`` (paged_model.py:409-634) moves beam rows inside the native store.

Differences: ``use_streaming_attention=False`` (the reference's reload-everything mode)
runs the same native path, since it computes the same attention. Supported model types: the
reference's (paged_model.py:82-86: qwen2, qwen2_moe, starcoder2, llama, mistral, gemma, phi3,
gemma2) and qwen3, all of which call transformers 5.x's attention interface with post-RoPE
q/k/v. Head dims 16, 32, 64, 128 and 256. Mistral's and Starcoder2's sliding window is applied
per step through the sequences' first valid position; a layer that passes its own window
(Gemma2's alternating sliding layers) masks by it in the kernel, and its softcap and scale
(Gemma2's attn_logit_softcapping and query_pre_attn_scalar) come with each call
(paged_model.py:143-177).
"""
from __future__ import annotations

import logging
import threading
from collections import OrderedDict
from contextlib import contextmanager
from dataclasses import dataclass

import torch
from transformers import AttentionInterface
from transformers.cache_utils import DynamicCache

from .paged_decode import PagedDecoder

logger = logging.getLogger(__name__)

_ATTN_IMPL = "pgr_paged_decode"
_POLICIES_WITHOUT_ATTENTION_SIGNAL = frozenset({"recent_only", "sinks_recent"})  # paged_model.py:40
_PAGER_BLOCK_BYTES = 16 * 1024 * 1024  # the pager's logical block size (core.rs:6)
_SUPPORTED_MODEL_TYPES = frozenset({"llama", "mistral", "qwen2", "qwen2_moe", "qwen3", "starcoder2", "gemma", "gemma2",
                                    "phi3"})
# Model types whose every layer attends within config.sliding_window (when set): the blocks
# below the window are left out of the step altogether. Layers that pass their own window
# with each call (Gemma2's alternating layers) mask by it in the kernel.
_WINDOWED_MODEL_TYPES = frozenset({"mistral", "starcoder2", "phi3"})


def _paged_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """Attention interface of a decode step: query [B, Hq, 1, D], key/value [B, Hkv, 1, D]
    (post-RoPE, the current token only). The layer's scale, softcap (Gemma2) and sliding
    window (None for global layers) come as arguments of the call. Returns ([B, 1, Hq, D],
    None)."""
    ctx = getattr(module, "_pgr_ctx", None)
    if ctx is None:
        raise RuntimeError(f"attention implementation {_ATTN_IMPL!r} is only usable inside PagedModel.generate()")
    if query.shape[2] != 1:
        raise RuntimeError("paged decode attention takes exactly one new token per sequence")
    q = query[:, :, 0, :]
    k = key[:, :, 0, :]
    v = value[:, :, 0, :]
    softcap = kwargs.get("softcap")
    out = ctx.decoder.decode_layer(module.layer_idx, q, k, v, scale=scaling,
                                   softcap=ctx.softcap if softcap is None else softcap,
                                   window=kwargs.get("sliding_window"))
    return out.unsqueeze(1), None


AttentionInterface.register(_ATTN_IMPL, _paged_attention)


class _LayerContext:
    def __init__(self, decoder: PagedDecoder, softcap: float | None):
        self.decoder = decoder
        self.softcap = softcap


@dataclass
class GenerationStats:
    """paged_model.py:179-189."""

    total_new_blocks: int = 0
    final_num_blocks: int = 0
    total_gpu_to_cpu_mb: float = 0.0
    total_cpu_to_gpu_mb: float = 0.0
    total_gpu_to_cpu_copies: int = 0
    total_cpu_to_gpu_copies: int = 0
    mean_attention_in_gpu: float = 0.0
    min_attention_in_gpu: float = 0.0
    max_attention_in_gpu: float = 0.0


class PagedModel:
    def __init__(
        self,
        model,
        *,
        vram_budget: int,
        ram_budget: int,
        recent_window: int = 64,
        rebalance_interval: int = 4,
        promote_margin: float = 0.05,
        ram_promote_margin: float = 0.20,
        policy: str = "sinks_heavy_hitter",
        tokens_per_block: int = 16,
        prefill_chunk_tokens: int = 512,
        use_streaming_attention: bool = True,
        streaming_group_size_blocks: int = 64,
        max_context_tokens: int | None = None,
        stream_mode: str = "direct",
        use_hip_graphs: bool = False,
    ):
        """Arguments and defaults of paged_model.py:200-215. Added: ``max_context_tokens``
        (tokens per row the native store is sized for; default: the first session's prompt
        plus max_new_tokens) and ``stream_mode`` ("direct", "staged" or "mirror"; see
        NativeKVPool). The group size has no effect: the native kernel covers every block in
        one launch.
        ``use_hip_graphs=True`` replays decode steps from a captured HIP graph: the first
        decode step runs eagerly, a step whose launch signature differs from the captured one
        (a new block changes the grids about once per block) is captured and replayed, later
        steps with the same signature are replayed. In the staged stream mode the graph holds
        the staging copies on the store's copy stream too, each layer's under the layer
        before it. In the mirror mode the copies stay outside the graph: begin_step queues
        them on the store's copy stream, where they run beside the replay.
        ``use_streaming_attention=False`` selects the reference's reload mode, which copies
        every block back into one HBM cache per step and runs the model's own attention
        (paged_model.py:717-760). For the supported model types it computes the same
        attention as the paged path, so both settings run the native path."""
        if not use_streaming_attention:
            logger.info("use_streaming_attention=False: running the native paged path (same attention, no reload)")
        if tokens_per_block <= 0 or tokens_per_block % 16:
            raise ValueError("tokens_per_block must be a positive multiple of 16 for the native kernels")
        self.use_hip_graphs = use_hip_graphs
        self._graphs: OrderedDict = OrderedDict()  # launch signature -> (graph, (ids, pos, logits))
        self._graph_pool = None
        self._graph_warm = False
        self.model = model
        self.tokens_per_block = tokens_per_block
        self.prefill_chunk_tokens = prefill_chunk_tokens
        self.use_streaming_attention = use_streaming_attention
        self.streaming_group_size_blocks = streaming_group_size_blocks
        self.max_context_tokens = max_context_tokens
        self.stream_mode = stream_mode
        self._needs_attention = policy not in _POLICIES_WITHOUT_ATTENTION_SIGNAL
        self._ram_budget = ram_budget
        self._pager_kwargs = dict(
            vram_budget=vram_budget,
            ram_budget=ram_budget,
            recent_window=recent_window,
            rebalance_interval=rebalance_interval,
            promote_margin=promote_margin,
            ram_promote_margin=ram_promote_margin,
            policy=policy,
        )
        self.last_run_stats: GenerationStats | None = None
        self._decoder: PagedDecoder | None = None
        self._sid: int | None = None
        self._rows = 0
        self._capacity = 0
        self._num_layers: int | None = None
        self._primed_tokens = 0
        self._primed_prefix: torch.Tensor | None = None
        self._lock = threading.Lock()

    # -- lifetime ------------------------------------------------------------------------
    def _acquire_or_raise(self) -> None:
        """paged_model.py:270-282."""
        if not self._lock.acquire(blocking=False):
            raise RuntimeError(
                "Another generate() or reset() call is already running on this PagedModel instance. It holds one "
                "mutable session, so concurrent calls from another thread would corrupt its state rather than run "
                "as independent requests. Use a separate PagedModel per concurrent session, or synchronize calls "
                "to this one yourself."
            )

    def reset(self) -> None:
        """Drop the current session; the next generate() call starts fresh (paged_model.py:284-299)."""
        self._acquire_or_raise()
        try:
            self._close()
        finally:
            self._lock.release()

    def _close(self) -> None:
        # Releasing the last graph of a memory pool releases the pool: the next capture needs
        # a new pool handle (capturing into the released one fails inside the allocator).
        self._graphs.clear()
        self._graph_pool = None
        self._graph_warm = False
        if self._decoder is not None:
            self._decoder.pool.close()
        self._decoder = None
        self._sid = None
        self._num_layers = None
        self._primed_tokens = 0
        self._primed_prefix = None

    @property
    def decoder(self) -> PagedDecoder | None:
        return self._decoder

    # -- generation ------------------------------------------------------------------------
    @torch.inference_mode()
    def generate(
        self,
        input_ids: torch.Tensor,
        attention_mask: torch.Tensor,
        max_new_tokens: int,
        *,
        do_sample: bool = False,
        temperature: float = 1.0,
        top_k: int | None = None,
        top_p: float | None = None,
        generator: torch.Generator | None = None,
    ) -> list[int] | list[list[int]]:
        """paged_model.py:300-407: generate up to max_new_tokens, continuing any previous session."""
        self._acquire_or_raise()
        try:
            batch_size = input_ids.shape[0]
            self._validate_left_padded(attention_mask)
            if do_sample:
                if temperature <= 0:
                    raise ValueError(f"temperature must be > 0 for sampling, got {temperature}.")
                if top_k is not None and top_k < 1:
                    raise ValueError(f"top_k must be >= 1, got {top_k}.")
                if top_p is not None and not (0.0 < top_p <= 1.0):
                    raise ValueError(f"top_p must be in (0, 1], got {top_p}.")
            if self._decoder is None:
                self._start_session(input_ids, attention_mask, max_new_tokens)
            else:
                self._extend_session(input_ids, attention_mask, max_new_tokens)

            next_input_id = input_ids[:, -1:]
            # The mask only grows by a real column per generated token, so the current token's
            # position is the last one's plus 1 and each row's left padding stays the same
            # (paged_model.py:373-385 rebuilds both from the grown mask every step). Token ids
            # stay on the device until the loop ends: no host synchronization between steps
            # besides the placement's.
            _, _, _, _, window = self._model_geometry()
            position_ids = self._position_ids_from_mask(attention_mask)[:, -1:]
            n_cols = attention_mask.shape[1]
            pads = (n_cols - attention_mask.long().sum(dim=1)).tolist() if window is not None else None
            token_ids: list[torch.Tensor] = []
            stats = GenerationStats()
            in_gpu: list[float] = []
            for t in range(max_new_tokens):
                lo = None
                if window is not None:
                    col = n_cols - 1 + t
                    lo = [max(p, col - window + 1) for p in pads]
                logits, step = self._forward_step(next_input_id, None, position_ids=position_ids, lo=lo)
                if do_sample:
                    next_token_id = self._sample_next_token(logits, temperature=temperature, top_k=top_k, top_p=top_p,
                                                            generator=generator)
                else:
                    next_token_id = torch.argmax(logits, dim=-1, keepdim=True)
                token_ids.append(next_token_id)
                stats.total_new_blocks += step["new_blocks"]
                stats.total_gpu_to_cpu_mb += step["gpu_to_cpu_mb"]
                stats.total_cpu_to_gpu_mb += step["cpu_to_gpu_mb"]
                stats.total_gpu_to_cpu_copies += step["gpu_to_cpu_copies"]
                stats.total_cpu_to_gpu_copies += step["cpu_to_gpu_copies"]
                in_gpu.append(step["attention_in_gpu"])
                next_input_id = next_token_id
                position_ids = position_ids + 1
            if token_ids:
                generated_per_row: list[list[int]] = torch.cat(token_ids, dim=1).tolist()
            else:
                generated_per_row = [[] for _ in range(batch_size)]
            full_sequence = torch.cat(
                [input_ids, torch.tensor(generated_per_row, dtype=input_ids.dtype, device=input_ids.device)], dim=1
            )
            self._primed_prefix = full_sequence[:, :-1].detach().clone()
            self._primed_tokens = full_sequence.shape[-1] - 1
            stats.final_num_blocks = self._decoder.num_blocks(self._sid)
            if in_gpu:
                stats.mean_attention_in_gpu = sum(in_gpu) / len(in_gpu)
                stats.min_attention_in_gpu = min(in_gpu)
                stats.max_attention_in_gpu = max(in_gpu)
            self.last_run_stats = stats
            return generated_per_row[0] if batch_size == 1 else generated_per_row
        finally:
            self._lock.release()

    @torch.inference_mode()
    def generate_beam_search(
        self,
        input_ids: torch.Tensor,
        attention_mask: torch.Tensor,
        num_beams: int,
        max_new_tokens: int,
        *,
        eos_token_id: int | None = None,
        length_penalty: float = 1.0,
        num_return_sequences: int = 1,
        do_sample: bool = False,
        temperature: float = 1.0,
        top_k: int | None = None,
        top_p: float | None = None,
        generator: torch.Generator | None = None,
    ):
        """Beam search with the semantics of paged_model.py:409-634.

        Each prompt keeps num_beams rows; every step the num_beams best (or, with do_sample,
        sampled without replacement) continuations over all beams of the same prompt are
        kept, so one beam's history can go to several rows or to none. The rows are moved
        inside the native store (reorder_rows: the first child inherits its parent's
        records, further children get copies), so no K/V leaves the device. Beams start
        as copies of the prompt with only the first one live (score 0, the rest -inf); a
        beam that emitted eos_token_id only continues with eos at no score change. The
        final candidates are ranked by score / len**length_penalty. Every call starts a
        fresh session and closes it at the end (no continuation by generate()).

        Returns list[int] (one prompt, one sequence), list[list[int]] (one prompt and
        several sequences, or several prompts and one), or list[list[list[int]]]."""
        self._acquire_or_raise()
        try:
            batch_size = input_ids.shape[0]
            if num_beams < 1:
                raise ValueError(f"num_beams must be >= 1, got {num_beams}")
            if not 1 <= num_return_sequences <= num_beams:
                raise ValueError(
                    f"num_return_sequences must be between 1 and num_beams ({num_beams}), got {num_return_sequences}"
                )
            if do_sample:
                if temperature <= 0:
                    raise ValueError(f"temperature must be > 0 for sampling, got {temperature}.")
                if top_k is not None and top_k < 1:
                    raise ValueError(f"top_k must be >= 1, got {top_k}.")
                if top_p is not None and not (0.0 < top_p <= 1.0):
                    raise ValueError(f"top_p must be in (0, 1], got {top_p}.")
            self._validate_left_padded(attention_mask)
            device = input_ids.device
            rows = batch_size * num_beams
            ids = input_ids.repeat_interleave(num_beams, dim=0)
            mask = attention_mask.repeat_interleave(num_beams, dim=0)
            self._close()
            self._start_session(ids, mask, max_new_tokens)
            try:
                scores = torch.full((rows,), float("-inf"), dtype=torch.float32, device=device)
                scores[0::num_beams] = 0.0
                tokens: list[list[int]] = [[] for _ in range(rows)]
                finished = torch.zeros(rows, dtype=torch.bool, device=device)
                group_base = (torch.arange(batch_size, device=device) * num_beams).unsqueeze(1)
                nxt = ids[:, -1:]
                for _ in range(max_new_tokens):
                    logits, _ = self._forward_step(nxt, mask)
                    logp = torch.log_softmax(logits.float(), dim=-1)  # [rows, V]
                    vocab = logp.shape[-1]
                    if eos_token_id is not None and bool(finished.any()):
                        frozen = torch.full((vocab,), float("-inf"), device=device)
                        frozen[eos_token_id] = 0.0
                        logp[finished] = frozen
                    cand = self._filter_for_sampling(logp, temperature, top_k, top_p) if do_sample else logp
                    joint = (scores.unsqueeze(1) + cand).view(batch_size, num_beams * vocab)
                    if do_sample:
                        pick = torch.multinomial(torch.softmax(joint, dim=-1), num_beams, replacement=False,
                                                 generator=generator)
                        top = torch.gather(joint, 1, pick)
                    else:
                        top, pick = torch.topk(joint, num_beams, dim=-1)
                    parents = (pick // vocab + group_base).flatten()
                    chosen = (pick % vocab).flatten()
                    parent_list, chosen_list = parents.tolist(), chosen.tolist()
                    tokens = [tokens[p] + [t] for p, t in zip(parent_list, chosen_list)]
                    finished = finished[parents]
                    if eos_token_id is not None:
                        finished = finished | (chosen == eos_token_id)
                    scores = top.flatten()
                    self._decoder.reorder_rows(self._sid, parent_list)
                    nxt = chosen.to(ids.dtype).unsqueeze(1)
                    mask = torch.cat([mask[parents], mask.new_ones((rows, 1))], dim=1)
                    if bool(finished.all()):
                        break
                final_scores = scores.tolist()
            finally:
                self._close()
            results: list[list[list[int]]] = []
            for g in range(batch_size):
                ranked = []
                for r in range(g * num_beams, (g + 1) * num_beams):
                    seq = tokens[r]
                    if eos_token_id is not None and eos_token_id in seq:
                        seq = seq[: seq.index(eos_token_id) + 1]
                    ranked.append((final_scores[r] / (max(len(seq), 1) ** length_penalty), seq))
                ranked.sort(key=lambda x: x[0], reverse=True)
                results.append([seq for _, seq in ranked[:num_return_sequences]])
            if batch_size == 1:
                return results[0][0] if num_return_sequences == 1 else results[0]
            return [grp[0] for grp in results] if num_return_sequences == 1 else results
        finally:
            self._lock.release()

    @staticmethod
    def _filter_for_sampling(logp, temperature, top_k, top_p):
        """paged_model.py:530-546: temperature, top-k and nucleus filtering of log-probs,
        renormalized."""
        scaled = logp / temperature
        if top_k is not None:
            kth = torch.topk(scaled, min(top_k, scaled.shape[-1]), dim=-1).values[:, -1, None]
            scaled = scaled.masked_fill(scaled < kth, float("-inf"))
        if top_p is not None:
            srt, order = torch.sort(scaled, descending=True, dim=-1)
            probs = torch.softmax(srt, dim=-1)
            srt = srt.masked_fill(torch.cumsum(probs, dim=-1) - probs > top_p, float("-inf"))
            scaled = torch.full_like(scaled, float("-inf")).scatter(-1, order, srt)
        return torch.log_softmax(scaled, dim=-1)

    @staticmethod
    def _sample_next_token(logits, *, temperature, top_k, top_p, generator):
        """paged_model.py:643-670."""
        logits = logits / temperature
        if top_k is not None:
            kth_value = torch.topk(logits, min(top_k, logits.shape[-1]), dim=-1).values[:, -1, None]
            logits = logits.masked_fill(logits < kth_value, float("-inf"))
        if top_p is not None:
            sorted_logits, sorted_indices = torch.sort(logits, descending=True, dim=-1)
            sorted_probs = torch.softmax(sorted_logits, dim=-1)
            cumulative_probs = torch.cumsum(sorted_probs, dim=-1)
            sorted_logits = sorted_logits.masked_fill(cumulative_probs - sorted_probs > top_p, float("-inf"))
            logits = torch.full_like(logits, float("-inf")).scatter(-1, sorted_indices, sorted_logits)
        probs = torch.softmax(logits, dim=-1)
        return torch.multinomial(probs, num_samples=1, generator=generator)

    # -- session ---------------------------------------------------------------------------
    def _model_geometry(self):
        cfg = self.model.config
        model_type = getattr(cfg, "model_type", None)
        if model_type not in _SUPPORTED_MODEL_TYPES:
            raise NotImplementedError(
                f"PagedModel doesn't recognize model_type={model_type!r}; supported: {sorted(_SUPPORTED_MODEL_TYPES)}"
            )
        num_heads = cfg.num_attention_heads
        num_kv = getattr(cfg, "num_key_value_heads", None) or num_heads
        head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // num_heads
        window = getattr(cfg, "sliding_window", None) if model_type in _WINDOWED_MODEL_TYPES else None
        return cfg.num_hidden_layers, num_heads, num_kv, head_dim, window

    def _start_session(self, input_ids: torch.Tensor, attention_mask: torch.Tensor, max_new_tokens: int) -> None:
        """paged_model.py:672-689: prefill all but the last token; every full block counts as
        HBM-resident until the first placement, as in the reference's initial store.

        The HBM pool holds the placement budget (vram_budget / 16 MiB blocks per row, the
        pager's own bound, core.rs:185-186) plus the open block and a block completed in the
        step before its placement: the reference frees a block's GPU memory when it offloads
        it (kv_block_store.py:110-111), so its VRAM budget bounds its GPU memory. Prompt
        blocks beyond the pool's room are written to their host records and read from there
        until the first placement loads or evicts them."""
        layers, hq, hkv, d, _ = self._model_geometry()
        rows, total = input_ids.shape
        T = self.tokens_per_block
        n_prefix = total - 1
        capacity = max(self.max_context_tokens or 0, total + max_new_tokens + T)
        blocks = -(-capacity // T) + 2
        budget_blocks = int(self._pager_kwargs["vram_budget"]) // _PAGER_BLOCK_BYTES
        dtype = next(self.model.parameters()).dtype
        device = input_ids.device
        # Staged mode: each buffer holds a whole layer's host blocks, so every step streams
        # one chunk per layer and queues the next layer's copies under the current layer.
        # Mirror mode: three ring buffers, grown to a layer's host share by the first step.
        dec = PagedDecoder(
            num_layers=layers, num_query_heads=hq, num_kv_heads=hkv, head_dim=d, tokens_per_block=T, dtype=dtype,
            device=device, pool_blocks=rows * (budget_blocks + 2), host_blocks=rows * blocks,
            staging_blocks=rows * blocks if self.stream_mode == "staged" else 64,
            staging_buffers=3 if self.stream_mode == "mirror" else 2, ram_budget_bytes=self._ram_budget,
            stream_mode=self.stream_mode,
        )
        pads = (attention_mask.shape[1] - attention_mask.long().sum(dim=1)).tolist()
        sid = dec.add_session(capacity_tokens=capacity, rows=rows, lo=pads, **self._pager_kwargs)
        if n_prefix > 0:
            past = self._chunked_prefill(input_ids[:, :-1], attention_mask[:, :-1])
            keys = [past.layers[i].keys for i in range(layers)]
            values = [past.layers[i].values for i in range(layers)]
            dec.prefill(sid, keys, values, n_prefix, place=False)
            del past, keys, values
        self._decoder, self._sid, self._rows, self._capacity, self._num_layers = dec, sid, rows, capacity, layers
        logger.info("Started PagedModel session: batch_size=%d prompt_tokens=%d layers=%d blocks=%d policy=%r",
                    rows, total, layers, dec.num_blocks(sid), self._pager_kwargs["policy"])

    def _extend_session(self, input_ids: torch.Tensor, attention_mask: torch.Tensor, max_new_tokens: int) -> None:
        """paged_model.py:691-713: feed the tokens not yet primed before decoding new ones."""
        total_len = input_ids.shape[-1]
        if input_ids.shape[0] != self._rows:
            raise ValueError("batch size differs from the primed session; call reset() first")
        if total_len - 1 < self._primed_tokens:
            raise ValueError(
                "input_ids is shorter than the already-primed session "
                f"({total_len - 1} < {self._primed_tokens} tokens). "
                "Call reset() to start a new session instead of rewinding one."
            )
        if not torch.equal(input_ids[:, : self._primed_tokens].cpu(), self._primed_prefix.cpu()):
            raise ValueError(
                "input_ids diverges from the already-primed session prefix. generate() expects each call to extend "
                "the same growing sequence (previous input + previously generated tokens + any new tokens). Call "
                "reset() to start a different session."
            )
        if total_len + max_new_tokens > self._capacity:
            raise ValueError(
                f"the session would grow past the {self._capacity} tokens its store was sized for; pass a larger "
                "max_context_tokens to PagedModel"
            )
        pending = input_ids[:, self._primed_tokens : total_len - 1]
        for i in range(pending.shape[-1]):
            self._forward_step(pending[:, i : i + 1], attention_mask[:, : self._primed_tokens + i + 1])

    def _chunked_prefill(self, prefix_input_ids: torch.Tensor, prefix_attention_mask: torch.Tensor) -> DynamicCache:
        """paged_model.py:1121-1161 (absolute cache_position per chunk)."""
        seq_len = prefix_input_ids.shape[-1]
        position_ids = self._position_ids_from_mask(prefix_attention_mask)
        past = DynamicCache()
        for start in range(0, seq_len, self.prefill_chunk_tokens):
            end = min(start + self.prefill_chunk_tokens, seq_len)
            out = self.model(
                input_ids=prefix_input_ids[:, start:end],
                attention_mask=prefix_attention_mask[:, :end],
                position_ids=position_ids[:, start:end],
                cache_position=torch.arange(start, end, device=prefix_input_ids.device),
                past_key_values=past,
                use_cache=True,
                logits_to_keep=1,
            )
            past = out.past_key_values
        return past

    @contextmanager
    def _paged_attention(self):
        cfg = self.model.config
        previous = cfg._attn_implementation
        ctx = _LayerContext(self._decoder, None)
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

    def _forward_step(self, input_id_tensor: torch.Tensor, current_attention_mask: torch.Tensor | None, *,
                      position_ids: torch.Tensor | None = None, lo: list[int] | None = None):
        """One token per row through the model over the paged store, then the placement glue
        (paged_model.py:715-823). Returns (last-position logits [B, V], step stats).

        The current token's position ids [B, 1] and, for sliding-window models, each row's
        first valid column come from current_attention_mask, or from `position_ids` / `lo`
        when the caller tracks them (generate's loop, which then needs no mask). The step is
        opened before the position ids are computed: in the mirror stream mode begin_step
        starts the step's host-to-device copies."""
        dec, sid = self._decoder, self._sid
        _, _, _, _, window = self._model_geometry()
        if window is not None:
            if lo is None:
                # Valid columns c > current_column - window (the causal mask's sliding-window rule).
                col = current_attention_mask.shape[1] - 1
                pads = (current_attention_mask.shape[1] - current_attention_mask.long().sum(dim=1)).tolist()
                lo = [max(p, col - window + 1) for p in pads]
            dec.set_lo(sid, lo)
        dec.begin_step([sid])
        if position_ids is None:
            position_ids = self._position_ids_from_mask(current_attention_mask)[:, -1:]
        host_blocks = dec.pool.step_stats()["gather_blocks"]  # blocks gathered from the host tier
        try:
            if self.use_hip_graphs:
                logits = self._graph_forward(input_id_tensor, position_ids)
            else:
                with self._paged_attention():
                    out = self.model(input_ids=input_id_tensor, position_ids=position_ids, use_cache=False,
                                     logits_to_keep=1)
                logits = out.logits[:, -1, :]
        except BaseException:
            dec.end_step(collect=False)
            raise
        st = dec.end_step()[sid]
        block_bytes_layer = dec.pool.block_bytes(sid) // max(self._num_layers, 1) // max(self._rows, 1)
        step = {
            "new_blocks": st["new_blocks"],
            "gpu_to_cpu_mb": st["gpu_to_cpu_mb"],
            "gpu_to_cpu_copies": st["gpu_to_cpu_copies"],
            "cpu_to_gpu_mb": host_blocks * block_bytes_layer * self._num_layers / 1_000_000,
            "cpu_to_gpu_copies": host_blocks * self._num_layers,
            "attention_in_gpu": st["attention_in_gpu"],
        }
        return logits, step

    # Captured graphs kept at once: a step whose signature was seen recently (a sequence
    # returning to an earlier block count, beam rows) replays without a new capture.
    _MAX_GRAPHS = 4

    def _graph_forward(self, input_ids: torch.Tensor, position_ids: torch.Tensor) -> torch.Tensor:
        """The decode forward of an open step from a captured HIP graph. The native launches
        read the step's plan from the store's pinned plan buffer and workspace, written by
        begin_step, so a graph stays valid while the launch signature (plan buffer and
        workspace pointers, grids, mass buffer) and the input shapes are unchanged: one graph
        is kept per signature. Returns the last-position logits [B, V]; the tensor is reused
        by the next replay of the same graph."""
        dec = self._decoder
        mass = dec._mass
        sig = (dec.pool.step_signature(), None if mass is None else (mass.data_ptr(), mass.stride(0)),
               tuple(input_ids.shape))
        if not self._graph_warm:  # first decode step: eager, so libraries set up outside capture
            self._graph_warm = True
            with self._paged_attention():
                out = self.model(input_ids=input_ids, position_ids=position_ids, use_cache=False, logits_to_keep=1)
            return out.logits[:, -1, :]
        entry = self._graphs.get(sig)
        if entry is None:
            # Older graphs stay alive until the new one is captured: the memory pool is shared,
            # and releasing the last graph of a pool releases the pool.
            ids, pos = input_ids.clone(), position_ids.clone()
            graph = torch.cuda.CUDAGraph()
            if self._graph_pool is None:
                self._graph_pool = torch.cuda.graph_pool_handle()
            with self._paged_attention():
                with torch.cuda.graph(graph, pool=self._graph_pool):
                    out = self.model(input_ids=ids, position_ids=pos, use_cache=False, logits_to_keep=1)
            entry = (graph, (ids, pos, out.logits))
            self._graphs[sig] = entry
            while len(self._graphs) > self._MAX_GRAPHS:
                self._graphs.popitem(last=False)
        else:
            self._graphs.move_to_end(sig)
            ids, pos, _ = entry[1]
            ids.copy_(input_ids)
            pos.copy_(position_ids)
        entry[0].replay()
        # The replayed attention launch reads the step's plan buffer; the next begin_step must
        # not overwrite it before then (steps fed back to back, e.g. a continued prompt).
        dec.pool.step_replayed()
        return entry[1][2][:, -1, :]

    @staticmethod
    def _position_ids_from_mask(attention_mask: torch.Tensor) -> torch.Tensor:
        """paged_model.py:1163-1167."""
        position_ids = attention_mask.long().cumsum(-1) - 1
        return position_ids.masked_fill(attention_mask == 0, 0)

    @staticmethod
    def _validate_left_padded(attention_mask: torch.Tensor) -> None:
        """paged_model.py:1169-1181."""
        mask = attention_mask.bool()
        if not mask.any(dim=1).all():
            raise NotImplementedError("attention_mask has a row with no real (non-padding) tokens.")
        if not torch.all(mask[:, :-1] <= mask[:, 1:]):
            raise NotImplementedError(
                "PagedModel only supports left-padding (zero or more leading zeros, then all ones, per row); "
                "right-padding or interleaved masking is not supported."
            )
