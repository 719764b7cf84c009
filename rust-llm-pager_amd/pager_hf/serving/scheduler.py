"""Continuous-batching decode loop: the admission and round logic of the reference's
ContinuousBatchingScheduler (pager_hf/serving/scheduler.py:452-601) over one shared native
paged store.

Each request is one session of a shared BatchedPagedEngine with the per-session budgets the
reference gives each PagedModel (total / max_concurrent_sessions, scheduler.py:144-145). A
new request is admitted whenever an active one finishes.

A round (``_run_once``):
1. a fresh request is opened (prefill of its prompt minus the last token) and takes its first
   step alone, so its all-HBM initial placement is re-placed at once -- the reference's
   ``_step_single`` for fresh sessions (scheduler.py:465-528);
2. every started request then advances by one token in ONE forward over all of them,
   whatever their lengths -- the reference batched only sessions sharing a tail length
   (scheduler.py:480-493, batched_decode.py:87-108). The next tokens of the whole batch come
   from one argmax over its [S, V] logits and one device-to-host copy.

Decoding is greedy. The reference's HTTP-facing plumbing (multi-turn session registry,
Prometheus metrics, drain and health reporting, sampling) is not part of this decode path.
"""
from __future__ import annotations

import logging
import queue
import threading
import uuid
from collections import deque
from dataclasses import dataclass, field

import torch

from ..batched_decode import BatchedPagedEngine

logger = logging.getLogger(__name__)


class SchedulerAtCapacityError(RuntimeError):
    """submit() when active + queued requests reach the limit (scheduler.py:28-31)."""


@dataclass
class ServingRequest:
    """One request's state (scheduler.py:51-71): the prompt, the tokens generated so far and
    the stream they are published on (None marks the end)."""

    request_id: str
    input_ids: torch.Tensor
    attention_mask: torch.Tensor
    max_new_tokens: int
    eos_token_id: int | None
    generated_tokens: list[int] = field(default_factory=list)
    output_queue: "queue.Queue[int | None]" = field(default_factory=queue.Queue)
    done: threading.Event = field(default_factory=threading.Event)
    error: Exception | None = None
    engine_session: object | None = None
    next_token: int | None = None  # the token the request's next step feeds

    @property
    def context_tokens(self) -> int:
        return self.input_ids.shape[1] + len(self.generated_tokens)


class ContinuousBatchingScheduler:
    def __init__(
        self,
        model,
        tokenizer,
        *,
        max_concurrent_sessions: int,
        total_vram_budget: int,
        total_ram_budget: int,
        policy: str = "sinks_heavy_hitter",
        tokens_per_block: int = 16,
        max_queue_depth: int = 100,
        device: torch.device | str = "cpu",
        max_context_tokens: int = 8192,
        host_token_capacity: int | None = None,
        stream_mode: str = "direct",
        staging_blocks: int = 64,
        staging_buffers: int = 2,
        engine: BatchedPagedEngine | None = None,
    ):
        """Budget, policy and queue arguments of scheduler.py:118-133. Added:
        ``max_context_tokens`` (most tokens one request holds), ``host_token_capacity``
        (pinned host tokens over all sessions), ``stream_mode`` / ``staging_blocks`` /
        ``staging_buffers`` (host block streaming of the engine) and ``engine`` (an existing
        BatchedPagedEngine to serve from)."""
        if max_concurrent_sessions < 1:
            raise ValueError(f"max_concurrent_sessions must be >= 1, got {max_concurrent_sessions}")
        if max_queue_depth < 0:
            raise ValueError(f"max_queue_depth must be >= 0, got {max_queue_depth}")
        self._model = model
        self._tokenizer = tokenizer
        self._max_concurrent_sessions = max_concurrent_sessions
        self._max_queue_depth = max_queue_depth
        self._max_context_tokens = max_context_tokens
        self._engine_kwargs = dict(
            max_sessions=max_concurrent_sessions,
            vram_budget_per_session=total_vram_budget // max_concurrent_sessions,
            ram_budget_per_session=total_ram_budget // max_concurrent_sessions,
            policy=policy,
            tokens_per_block=tokens_per_block,
            max_context_tokens=max_context_tokens,
            host_token_capacity=host_token_capacity,
            stream_mode=stream_mode,
            staging_blocks=staging_blocks,
            staging_buffers=staging_buffers,
        )
        self._engine = engine
        self._device = torch.device(device)
        self._incoming: queue.Queue[ServingRequest] = queue.Queue()
        self._active: list[ServingRequest] = []
        self._stop = threading.Event()
        self._thread = threading.Thread(target=self._run, daemon=True)

    def engine(self) -> BatchedPagedEngine:
        if self._engine is None:
            self._engine = BatchedPagedEngine(self._model, **self._engine_kwargs)
        return self._engine

    # -- lifecycle -------------------------------------------------------------------------
    def start(self) -> None:
        """Runs rounds on a background thread until stop()."""
        self._thread.start()

    def stop(self) -> None:
        """Stops the round loop; requests not finished by then end with an error."""
        self._stop.set()
        if self._thread.ident is not None:
            self._thread.join()
        for req in list(self._active):
            req.error = RuntimeError("scheduler stopped before this request finished")
            self._retire(req)
        while True:
            try:
                req = self._incoming.get_nowait()
            except queue.Empty:
                break
            req.error = RuntimeError("scheduler stopped before this request was admitted")
            req.output_queue.put(None)
            req.done.set()

    def load(self) -> int:
        return len(self._active) + self._incoming.qsize()

    # -- submission (scheduler.py:320-360) ---------------------------------------------------
    def submit(self, input_ids: torch.Tensor, attention_mask: torch.Tensor, max_new_tokens: int) -> ServingRequest:
        """A request of one row ([1, n]); its session closes when it finishes."""
        depth, limit = self.load(), self._max_concurrent_sessions + self._max_queue_depth
        if depth >= limit:
            raise SchedulerAtCapacityError(f"scheduler is at capacity ({depth}/{limit} requests active or queued)")
        if input_ids.dim() != 2 or input_ids.shape[0] != 1:
            raise ValueError("submit() takes one row: input_ids [1, n]")
        if max_new_tokens < 1:
            raise ValueError("max_new_tokens must be >= 1")
        if input_ids.shape[1] + max_new_tokens > self._max_context_tokens:
            raise ValueError(f"prompt + max_new_tokens exceeds max_context_tokens={self._max_context_tokens}")
        req = ServingRequest(request_id=str(uuid.uuid4()), input_ids=input_ids.to(self._device),
                             attention_mask=attention_mask.to(self._device), max_new_tokens=max_new_tokens,
                             eos_token_id=getattr(self._tokenizer, "eos_token_id", None))
        self._incoming.put(req)
        return req

    # -- rounds (scheduler.py:452-601) -----------------------------------------------------
    def _run(self) -> None:
        while not self._stop.is_set():
            self._admit_new_requests()
            if not self._active:
                self._stop.wait(timeout=0.005)
                continue
            self._run_once()

    def _admit_new_requests(self) -> None:
        while len(self._active) < self._max_concurrent_sessions:
            try:
                req = self._incoming.get_nowait()
            except queue.Empty:
                return
            self._active.append(req)

    def _run_once(self) -> None:
        """One round: fresh requests are opened and take their first step alone; every other
        active request then advances one token in one batched step."""
        snapshot = list(self._active)
        fresh = [r for r in snapshot if r.engine_session is None]
        for req in fresh:
            self._open(req)
        started = [r for r in snapshot if r.engine_session is not None and not r.done.is_set() and r not in fresh]
        if started:
            self._step(started)

    def _open(self, req: ServingRequest) -> None:
        try:
            capacity = req.input_ids.shape[1] + req.max_new_tokens + 1
            req.engine_session = self.engine().open(req.input_ids, req.attention_mask, capacity)
            req.next_token = int(req.input_ids[0, -1])
        except Exception as exc:  # noqa: BLE001 -- surfaced to the caller via req.error
            logger.error("request %s failed to open: %s", req.request_id, exc)
            req.error = exc
            self._retire(req)
            return
        self._step([req])

    def _step(self, group: list[ServingRequest]) -> None:
        try:
            logits = self.engine().step([r.engine_session for r in group], [r.next_token for r in group])
            next_ids = torch.argmax(logits, dim=-1).tolist()
        except Exception as exc:  # noqa: BLE001
            logger.error("decode step failed for %d requests: %s", len(group), exc)
            for req in group:
                req.error = exc
                self._retire(req)
            return
        for req, token_id in zip(group, next_ids):
            self._finish_step(req, token_id)

    def _finish_step(self, req: ServingRequest, token_id: int) -> None:
        """scheduler.py:565-585: record and publish the token; retire on EOS or max_new_tokens."""
        req.generated_tokens.append(token_id)
        req.output_queue.put(token_id)
        is_eos = req.eos_token_id is not None and token_id == req.eos_token_id
        if is_eos or len(req.generated_tokens) >= req.max_new_tokens:
            self._retire(req)
        else:
            req.next_token = token_id

    def _retire(self, req: ServingRequest) -> None:
        """scheduler.py:587-601; the request's session is closed."""
        req.output_queue.put(None)
        req.done.set()
        if req in self._active:
            self._active.remove(req)
        if req.engine_session is not None and self._engine is not None:
            self._engine.close(req.engine_session)
