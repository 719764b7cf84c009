"""Continuous-batching decode scheduler: the reference's ContinuousBatchingScheduler
(pager_hf/serving/scheduler.py:74-601) over one shared native paged store.

Same public surface: ``ContinuousBatchingScheduler(model, tokenizer, *, max_concurrent_sessions,
total_vram_budget, total_ram_budget, policy, tokens_per_block, use_streaming_attention,
streaming_group_size_blocks, max_queue_depth, device, metrics_registry, device_label)``,
``submit``, ``create_session`` / ``submit_turn`` / ``delete_session``, ``start`` / ``stop`` /
``health`` / ``load``, ServingRequest with its token stream, the three error types, and the
Prometheus metrics. Each request is one session of a shared BatchedPagedEngine with the
per-session budgets the reference gives each PagedModel (total / max_concurrent_sessions).

A round (``_run_once``):
1. a fresh request is opened (prefill of its prompt minus the last token) and takes its first
   step alone, so its all-HBM initial placement is re-placed at once -- the reference's
   ``_step_single`` for fresh sessions (scheduler.py:465-528);
2. every started request then advances by one token in ONE forward over all of them,
   whatever their lengths -- the reference batched only sessions sharing a tail length
   (scheduler.py:480-493, batched_decode.py:87-108).

A request feeds a queue of tokens: the prompt's last token, or on a later turn of a
persistent session the previous turn's last token followed by the new turn's tokens; logits
are sampled only after the queue's last token (the reference's _extend_session feeds the
same tokens one decode step each, paged_model.py:691-713).
"""
from __future__ import annotations

import logging
import queue
import threading
import time
import uuid
from collections import deque
from dataclasses import dataclass, field

import torch
from prometheus_client import CollectorRegistry, Counter, Gauge, Histogram

from ..batched_decode import BatchedPagedEngine
from ..paged_model import PagedModel

logger = logging.getLogger(__name__)


class SessionCapacityError(RuntimeError):
    """create_session() when the persistent-session registry is full (scheduler.py:19-20)."""


class SessionBusyError(RuntimeError):
    """A session already has an in-flight turn (scheduler.py:23-25)."""


class SchedulerAtCapacityError(RuntimeError):
    """submit()/submit_turn() when active + queued reaches the limit (scheduler.py:28-31)."""


@dataclass
class SessionState:
    """A multi-turn conversation (scheduler.py:33-49): its engine session persists across turns."""

    session_id: str
    engine_session: object | None = None
    input_ids: torch.Tensor | None = None
    attention_mask: torch.Tensor | None = None
    last_token: int | None = None  # the previous turn's last generated token (not yet fed)


@dataclass
class ServingRequest:
    """One request's state (scheduler.py:51-71)."""

    request_id: str
    input_ids: torch.Tensor
    attention_mask: torch.Tensor
    max_new_tokens: int
    eos_token_id: int | None
    do_sample: bool = False
    temperature: float = 1.0
    top_k: int | None = None
    top_p: float | None = None
    session_id: str | None = None
    generated_tokens: list[int] = field(default_factory=list)
    output_queue: "queue.Queue[int | None]" = field(default_factory=queue.Queue)
    done: threading.Event = field(default_factory=threading.Event)
    error: Exception | None = None
    # engine state
    engine_session: object | None = None
    feed: deque = field(default_factory=deque)
    new_turn: torch.Tensor | None = None  # tokens of this turn (persistent sessions)


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
        use_streaming_attention: bool = True,
        streaming_group_size_blocks: int = 64,
        max_queue_depth: int = 100,
        device: torch.device | str = "cpu",
        metrics_registry: CollectorRegistry | None = None,
        device_label: str = "default",
        max_context_tokens: int = 8192,
        host_token_capacity: int | None = None,
        stream_mode: str = "direct",
        staging_blocks: int = 64,
        staging_buffers: int = 2,
        engine: BatchedPagedEngine | None = None,
    ):
        """Arguments of scheduler.py:118-133. Added: ``max_context_tokens`` (most tokens one
        request or session holds), ``host_token_capacity`` (pinned host tokens over all
        sessions), ``stream_mode`` / ``staging_blocks`` / ``staging_buffers`` (host block
        streaming of the engine) and ``engine`` (an existing BatchedPagedEngine to serve
        from). ``use_streaming_attention=False`` runs the same native path (see PagedModel);
        the group size has no effect."""
        if max_concurrent_sessions < 1:
            raise ValueError(f"max_concurrent_sessions must be >= 1, got {max_concurrent_sessions}")
        if max_queue_depth < 0:
            raise ValueError(f"max_queue_depth must be >= 0, got {max_queue_depth}")
        self._model = model
        self._tokenizer = tokenizer
        self._max_concurrent_sessions = max_concurrent_sessions
        self._max_queue_depth = max_queue_depth
        self._vram_budget_per_session = total_vram_budget // max_concurrent_sessions
        self._ram_budget_per_session = total_ram_budget // max_concurrent_sessions
        self._max_context_tokens = max_context_tokens
        self._engine_kwargs = dict(
            max_sessions=2 * max_concurrent_sessions,  # one-shot requests + persistent sessions
            vram_budget_per_session=self._vram_budget_per_session,
            ram_budget_per_session=self._ram_budget_per_session,
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
        self._device_label = device_label
        self._incoming: queue.Queue[ServingRequest] = queue.Queue()
        self._active: list[ServingRequest] = []
        self._stop = threading.Event()
        self._draining = threading.Event()
        self._thread = threading.Thread(target=self._run, daemon=True)
        self._sessions: dict[str, SessionState] = {}
        self._busy_sessions: set[str] = set()
        self._sessions_lock = threading.Lock()
        # Engine sessions of deleted persistent sessions, closed by the scheduler thread (the
        # native store is driven from that one thread only).
        self._pending_close: list = []

        self.metrics_registry = metrics_registry or CollectorRegistry()
        self._requests_total = Counter("pager_hf_requests_total", "Completions requests retired, by outcome",
                                       ["outcome", "device"], registry=self.metrics_registry)
        self._tokens_generated_total = Counter("pager_hf_tokens_generated_total", "Tokens generated across all requests",
                                               ["device"], registry=self.metrics_registry).labels(device=device_label)
        self._decode_round_seconds = Histogram("pager_hf_decode_round_seconds",
                                               "Wall time of one decode step call", ["device"],
                                               registry=self.metrics_registry).labels(device=device_label)
        self._step_calls_total = Counter("pager_hf_step_calls_total", "Decode-step calls, by mode", ["mode", "device"],
                                         registry=self.metrics_registry)
        Gauge("pager_hf_active_requests", "Requests currently admitted into the round-robin set", ["device"],
              registry=self.metrics_registry).labels(device=device_label).set_function(lambda: len(self._active))
        Gauge("pager_hf_queued_requests", "Requests submitted but not yet admitted", ["device"],
              registry=self.metrics_registry).labels(device=device_label).set_function(self._incoming.qsize)
        Gauge("pager_hf_active_sessions", "Persistent multi-turn sessions currently registered", ["device"],
              registry=self.metrics_registry).labels(device=device_label).set_function(lambda: len(self._sessions))

    # -- engine ----------------------------------------------------------------------------
    def engine(self) -> BatchedPagedEngine:
        if self._engine is None:
            self._engine = BatchedPagedEngine(self._model, **self._engine_kwargs)
        return self._engine

    # -- lifecycle (scheduler.py:237-310) ----------------------------------------------------
    def start(self) -> None:
        self._thread.start()
        logger.info("ContinuousBatchingScheduler started: max_concurrent_sessions=%d max_queue_depth=%d "
                    "vram_budget_per_session=%d ram_budget_per_session=%d", self._max_concurrent_sessions,
                    self._max_queue_depth, self._vram_budget_per_session, self._ram_budget_per_session)

    def health(self) -> dict:
        return {
            "status": "ok" if self._thread.is_alive() else "unhealthy",
            "thread_alive": self._thread.is_alive(),
            "active_requests": len(self._active),
            "queued_requests": self._incoming.qsize(),
            "active_sessions": len(self._sessions),
        }

    def stop(self, timeout: float | None = None) -> None:
        """Drain: admit nothing new, let active requests finish (up to timeout), then fail
        whatever is left (scheduler.py:262-293)."""
        self._draining.set()
        if self._thread.is_alive() or self._thread.ident is not None:
            self._thread.join(timeout)
            if self._thread.is_alive():
                self._stop.set()
                self._thread.join()
        for req in list(self._active):
            req.error = RuntimeError("scheduler shut down before this request finished (drain timeout exceeded)")
            self._retire(req)
        while True:
            try:
                req = self._incoming.get_nowait()
            except queue.Empty:
                break
            req.error = RuntimeError("scheduler shut down before this request could be admitted")
            req.done.set()
        self._close_pending()

    def load(self) -> int:
        return len(self._active) + self._incoming.qsize()

    def _check_capacity(self) -> None:
        depth = self.load()
        limit = self._max_concurrent_sessions + self._max_queue_depth
        if depth >= limit:
            raise SchedulerAtCapacityError(f"scheduler is at capacity ({depth}/{limit} requests active or queued)")

    # -- submission (scheduler.py:320-450) ---------------------------------------------------
    def _enqueue(self, input_ids, attention_mask, max_new_tokens, *, do_sample, temperature, top_k, top_p,
                 session_id, new_turn=None) -> ServingRequest:
        if max_new_tokens < 1:
            raise ValueError("max_new_tokens must be >= 1")
        req = ServingRequest(
            request_id=str(uuid.uuid4()), input_ids=input_ids, attention_mask=attention_mask,
            max_new_tokens=max_new_tokens, eos_token_id=getattr(self._tokenizer, "eos_token_id", None),
            do_sample=do_sample, temperature=temperature, top_k=top_k, top_p=top_p, session_id=session_id,
            new_turn=new_turn,
        )
        self._incoming.put(req)
        return req

    def submit(self, input_ids: torch.Tensor, attention_mask: torch.Tensor, max_new_tokens: int, *,
               do_sample: bool = False, temperature: float = 1.0, top_k: int | None = None,
               top_p: float | None = None) -> ServingRequest:
        """A one-shot request (its own session, closed when it finishes)."""
        self._check_capacity()
        if input_ids.shape[0] != 1:
            raise ValueError("submit() takes one row: input_ids [1, n]")
        if input_ids.shape[1] + max_new_tokens > self._max_context_tokens:
            raise ValueError(f"prompt + max_new_tokens exceeds max_context_tokens={self._max_context_tokens}")
        return self._enqueue(input_ids.to(self._device), attention_mask.to(self._device), max_new_tokens,
                             do_sample=do_sample, temperature=temperature, top_k=top_k, top_p=top_p, session_id=None)

    def create_session(self) -> str:
        with self._sessions_lock:
            if len(self._sessions) >= self._max_concurrent_sessions:
                raise SessionCapacityError(
                    f"session registry is full ({len(self._sessions)}/{self._max_concurrent_sessions} sessions)"
                )
            session_id = str(uuid.uuid4())
            self._sessions[session_id] = SessionState(session_id=session_id)
            return session_id

    def delete_session(self, session_id: str) -> None:
        with self._sessions_lock:
            if session_id not in self._sessions:
                raise KeyError(session_id)
            if session_id in self._busy_sessions:
                raise SessionBusyError(f"session {session_id!r} has an in-flight turn; wait for it to finish first")
            state = self._sessions.pop(session_id)
            if state.engine_session is not None:
                self._pending_close.append(state.engine_session)
        if not self._thread.is_alive():
            self._close_pending()

    def submit_turn(self, session_id: str, input_ids: torch.Tensor, attention_mask: torch.Tensor, max_new_tokens: int,
                    *, do_sample: bool = False, temperature: float = 1.0, top_k: int | None = None,
                    top_p: float | None = None) -> ServingRequest:
        """The next turn of a persistent session: input_ids are this turn's new tokens."""
        self._check_capacity()
        input_ids = input_ids.to(self._device)
        attention_mask = attention_mask.to(self._device)
        with self._sessions_lock:
            session = self._sessions.get(session_id)
            if session is None:
                raise KeyError(session_id)
            if session_id in self._busy_sessions:
                raise SessionBusyError(f"session {session_id!r} already has an in-flight turn")
            self._busy_sessions.add(session_id)
            if session.input_ids is None:
                combined_ids, combined_mask = input_ids, attention_mask
            else:
                combined_ids = torch.cat([session.input_ids, input_ids], dim=1)
                combined_mask = torch.cat([session.attention_mask, attention_mask], dim=1)
        return self._enqueue(combined_ids, combined_mask, max_new_tokens, do_sample=do_sample,
                             temperature=temperature, top_k=top_k, top_p=top_p, session_id=session_id,
                             new_turn=input_ids)

    # -- rounds (scheduler.py:452-601) ---------------------------------------------------------
    def _run(self) -> None:
        while not self._stop.is_set():
            if not self._draining.is_set():
                self._admit_new_requests()
            if not self._active:
                if self._draining.is_set():
                    return
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

    def _close_pending(self) -> None:
        with self._sessions_lock:
            pending, self._pending_close = self._pending_close, []
        for es in pending:
            if self._engine is not None:
                self._engine.close(es)

    def _run_once(self) -> None:
        """One round: fresh requests are opened and take their first step alone; every other
        active request then advances one token in one batched step."""
        self._close_pending()
        snapshot = list(self._active)
        fresh = [r for r in snapshot if r.engine_session is None]
        for req in fresh:
            self._open(req)
        started = [r for r in snapshot if r.engine_session is not None and not r.done.is_set() and r not in fresh]
        if started:
            self._step(started, mode="batched" if len(started) > 1 else "single")

    def _open(self, req: ServingRequest) -> None:
        eng = self.engine()
        try:
            if req.session_id is not None:
                with self._sessions_lock:
                    state = self._sessions.get(req.session_id)
                if state is not None and state.engine_session is not None:
                    # Later turn: feed the previous turn's last token, then the new turn.
                    req.engine_session = state.engine_session
                    req.feed.extend([state.last_token] + req.new_turn[0].tolist())
                else:
                    req.engine_session = eng.open(req.input_ids, req.attention_mask, self._max_context_tokens)
                    req.feed.append(int(req.input_ids[0, -1].item()))
                    if state is not None:
                        state.engine_session = req.engine_session
            else:
                capacity = req.input_ids.shape[1] + req.max_new_tokens + 1
                req.engine_session = eng.open(req.input_ids, req.attention_mask, capacity)
                req.feed.append(int(req.input_ids[0, -1].item()))
        except Exception as exc:  # noqa: BLE001 -- surfaced to the caller via req.error
            logger.error("request %s failed to open: %s", req.request_id, exc)
            req.error = exc
            self._retire(req)
            return
        self._step([req], mode="single")

    def _step(self, group: list[ServingRequest], mode: str) -> None:
        self._step_calls_total.labels(mode=mode, device=self._device_label).inc()
        started = time.monotonic()
        try:
            logits = self.engine().step([r.engine_session for r in group], [r.feed.popleft() for r in group])
        except Exception as exc:  # noqa: BLE001
            logger.error("decode step failed for %d requests: %s", len(group), exc)
            for req in group:
                req.error = exc
                self._retire(req)
            return
        finally:
            self._decode_round_seconds.observe(time.monotonic() - started)
        for req, lg in zip(group, logits):
            if req.feed:
                continue  # still feeding this turn's tokens: no output yet
            if req.do_sample:
                token_id = int(PagedModel._sample_next_token(lg.unsqueeze(0), temperature=req.temperature,
                                                             top_k=req.top_k, top_p=req.top_p,
                                                             generator=None).item())
            else:
                token_id = int(torch.argmax(lg).item())
            self._finish_step(req, token_id)

    def _finish_step(self, req: ServingRequest, token_id: int) -> None:
        """scheduler.py:565-585: record, grow input_ids, retire on EOS or max_new_tokens."""
        req.generated_tokens.append(token_id)
        req.output_queue.put(token_id)
        self._tokens_generated_total.inc()
        req.input_ids = torch.cat(
            [req.input_ids, torch.tensor([[token_id]], dtype=req.input_ids.dtype, device=req.input_ids.device)], dim=1
        )
        req.attention_mask = torch.cat([req.attention_mask, req.attention_mask.new_ones((1, 1))], dim=1)
        is_eos = req.eos_token_id is not None and token_id == req.eos_token_id
        if is_eos or len(req.generated_tokens) >= req.max_new_tokens:
            self._retire(req)
        else:
            req.feed.append(token_id)

    def _retire(self, req: ServingRequest) -> None:
        """scheduler.py:587-601; a one-shot request's session is closed."""
        req.output_queue.put(None)
        req.done.set()
        self._requests_total.labels(outcome="error" if req.error is not None else "success",
                                    device=self._device_label).inc()
        if req in self._active:
            self._active.remove(req)
        if req.session_id is not None:
            with self._sessions_lock:
                self._busy_sessions.discard(req.session_id)
                session = self._sessions.get(req.session_id)
                if session is not None:
                    session.input_ids = req.input_ids
                    session.attention_mask = req.attention_mask
                    session.last_token = req.generated_tokens[-1] if req.generated_tokens else session.last_token
                    if req.error is not None and session.engine_session is req.engine_session:
                        # The stored state is unknown after a failure: the next turn starts over.
                        session.engine_session = None
                        session.input_ids = session.attention_mask = None
                        if req.engine_session is not None and self._engine is not None:
                            self._engine.close(req.engine_session)
        elif req.engine_session is not None and self._engine is not None:
            self._engine.close(req.engine_session)
