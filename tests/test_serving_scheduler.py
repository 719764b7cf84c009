"""ContinuousBatchingScheduler host logic on the CPU, with a fake engine.

Follows the reference's tests/test_serving_scheduler.py:71-425 case by case where the
behaviour is shared (admission, EOS, the token stream, sessions and turns, capacity and
backpressure, drain and health); the batching cases check this build's rule instead
(fresh requests step alone, every started request joins one batched step per round).
Rounds are driven directly (_admit_new_requests / _run_once) except where the background
thread itself is under test.
"""
from __future__ import annotations

import threading
import time
from types import SimpleNamespace

import pytest
import torch

from pager_hf.serving.scheduler import (
    ContinuousBatchingScheduler,
    SchedulerAtCapacityError,
    SessionBusyError,
    SessionCapacityError,
)

EOS = 999
VOCAB = 1000


class FakeSession:
    def __init__(self, tokens):
        self.tokens = list(tokens)
        self.fed: list[int] = []
        self.closed = False


class FakeEngine:
    """open() hands out sessions that answer a prescribed token sequence, in submit order."""

    def __init__(self, sequences, never_ending=False):
        self.sequences = list(sequences)
        self.never_ending = never_ending
        self.opened: list[FakeSession] = []
        self.steps: list[list[FakeSession]] = []

    def open(self, input_ids, attention_mask, capacity):
        s = FakeSession(self.sequences[len(self.opened)] if self.sequences else [])
        s.prompt = input_ids[0].tolist()
        self.opened.append(s)
        return s

    def step(self, sessions, tokens):
        self.steps.append(list(sessions))
        logits = torch.zeros(len(sessions), VOCAB)
        for i, (s, t) in enumerate(zip(sessions, tokens)):
            s.fed.append(t)
            nxt = 7 if self.never_ending else (s.tokens.pop(0) if s.tokens else EOS)
            logits[i, nxt] = 1.0
        return logits

    def close(self, s):
        s.closed = True


def make(sequences=(), *, max_concurrent=2, max_queue_depth=100, never_ending=False):
    eng = FakeEngine(sequences, never_ending)
    sched = ContinuousBatchingScheduler(
        model=object(), tokenizer=SimpleNamespace(eos_token_id=EOS), max_concurrent_sessions=max_concurrent,
        total_vram_budget=2_000_000, total_ram_budget=4_000_000, max_queue_depth=max_queue_depth, engine=eng,
    )
    return sched, eng


def prompt(n=3, start=1):
    ids = torch.arange(start, start + n).unsqueeze(0)
    return ids, torch.ones_like(ids)


def drive(sched, rounds):
    for _ in range(rounds):
        sched._admit_new_requests()
        if sched._active:
            sched._run_once()


def test_rejects_invalid_arguments():
    with pytest.raises(ValueError):
        ContinuousBatchingScheduler(object(), None, max_concurrent_sessions=0, total_vram_budget=1, total_ram_budget=1)
    with pytest.raises(ValueError):
        ContinuousBatchingScheduler(object(), None, max_concurrent_sessions=1, total_vram_budget=1, total_ram_budget=1,
                                    max_queue_depth=-1)


def test_reload_mode_flag_is_accepted():
    eng = FakeEngine([[5]])
    sched = ContinuousBatchingScheduler(object(), SimpleNamespace(eos_token_id=EOS), max_concurrent_sessions=1,
                                        total_vram_budget=1, total_ram_budget=1, use_streaming_attention=False,
                                        engine=eng)
    req = sched.submit(*prompt(), max_new_tokens=1)
    drive(sched, 2)
    assert req.generated_tokens == [5]


def test_admission_respects_max_concurrent_sessions():
    sched, eng = make([[5, 6, 7]] * 3, max_concurrent=2)
    reqs = [sched.submit(*prompt(), max_new_tokens=3) for _ in range(3)]
    sched._admit_new_requests()
    assert len(sched._active) == 2 and sched._incoming.qsize() == 1
    drive(sched, 3)
    assert reqs[0].done.is_set() and reqs[1].done.is_set()
    drive(sched, 3)
    assert reqs[2].done.is_set()
    assert [r.generated_tokens for r in reqs] == [[5, 6, 7]] * 3


def test_fresh_requests_step_alone_then_join_one_batched_step():
    sched, eng = make([[5, 6, 7], [8, 9, 10]], max_concurrent=2)
    a = sched.submit(*prompt(), max_new_tokens=3)
    b = sched.submit(*prompt(start=10), max_new_tokens=3)
    drive(sched, 1)
    assert [len(s) for s in eng.steps] == [1, 1]  # each fresh request's first step alone
    drive(sched, 1)
    assert len(eng.steps[-1]) == 2  # started requests advance together
    drive(sched, 1)
    assert a.generated_tokens == [5, 6, 7] and b.generated_tokens == [8, 9, 10]
    # Each session was fed its prompt's last token, then its own generated tokens.
    assert eng.opened[0].fed == [3, 5, 6] and eng.opened[1].fed == [12, 8, 9]
    assert all(s.closed for s in eng.opened)


def test_eos_retires_request_before_max_new_tokens():
    sched, _ = make([[5, EOS, 6]])
    req = sched.submit(*prompt(), max_new_tokens=10)
    drive(sched, 5)
    assert req.done.is_set() and req.generated_tokens == [5, EOS]


def test_output_queue_drains_to_sentinel():
    sched, _ = make([[5, 6]])
    req = sched.submit(*prompt(), max_new_tokens=2)
    drive(sched, 3)
    got = []
    while True:
        t = req.output_queue.get_nowait()
        if t is None:
            break
        got.append(t)
    assert got == [5, 6]


def test_sessions_capacity_and_unique_ids():
    sched, _ = make(max_concurrent=2)
    a, b = sched.create_session(), sched.create_session()
    assert a != b
    with pytest.raises(SessionCapacityError):
        sched.create_session()


def test_submit_turn_unknown_session_raises_key_error():
    sched, _ = make()
    with pytest.raises(KeyError):
        sched.submit_turn("nope", *prompt(), max_new_tokens=1)


def test_turns_reuse_the_engine_session_and_feed_the_previous_output():
    # The fake answers every step; the two steps that only feed turn 2's tokens answer 0.
    sched, eng = make([[5, 6, 0, 0, 40, 41]])
    sid = sched.create_session()
    r1 = sched.submit_turn(sid, *prompt(), max_new_tokens=2)
    drive(sched, 3)
    assert r1.generated_tokens == [5, 6]
    r2 = sched.submit_turn(sid, torch.tensor([[20, 21]]), torch.ones(1, 2, dtype=torch.long), max_new_tokens=2)
    assert r2.input_ids[0].tolist() == [1, 2, 3, 5, 6, 20, 21]
    drive(sched, 5)
    assert r2.generated_tokens == [40, 41]
    assert len(eng.opened) == 1  # one engine session across turns
    # Turn 2 fed turn 1's last token and its own tokens; only the last one produced output.
    assert eng.opened[0].fed == [3, 5, 6, 20, 21, 40]
    assert not eng.opened[0].closed
    sched.delete_session(sid)
    assert eng.opened[0].closed


def test_concurrent_turn_rejected_and_delete_waits_for_it():
    sched, _ = make([[5, 6]])
    sid = sched.create_session()
    sched.submit_turn(sid, *prompt(), max_new_tokens=2)
    with pytest.raises(SessionBusyError):
        sched.submit_turn(sid, *prompt(), max_new_tokens=1)
    with pytest.raises(SessionBusyError):
        sched.delete_session(sid)
    drive(sched, 3)
    sched.delete_session(sid)
    with pytest.raises(KeyError):
        sched.delete_session(sid)


def test_submit_raises_at_capacity():
    sched, _ = make(max_concurrent=1, max_queue_depth=1)
    sched.submit(*prompt(), max_new_tokens=1)
    sched.submit(*prompt(), max_new_tokens=1)
    with pytest.raises(SchedulerAtCapacityError):
        sched.submit(*prompt(), max_new_tokens=1)


def test_submit_turn_at_capacity_does_not_mark_session_busy():
    sched, _ = make(max_concurrent=1, max_queue_depth=0)
    sid = sched.create_session()
    sched.submit(*prompt(), max_new_tokens=1)
    with pytest.raises(SchedulerAtCapacityError):
        sched.submit_turn(sid, *prompt(), max_new_tokens=1)
    assert sid not in sched._busy_sessions


def test_health_reports_thread_status():
    sched, _ = make([[5]])
    assert sched.health()["thread_alive"] is False
    sched.start()
    try:
        assert sched.health()["status"] == "ok"
    finally:
        sched.stop(timeout=5)
    assert sched.health()["thread_alive"] is False


def test_stop_drains_active_request_to_completion():
    sched, _ = make([[5, 6, 7]])
    sched.start()
    req = sched.submit(*prompt(), max_new_tokens=3)
    assert req.done.wait(5)
    sched.stop(timeout=5)
    assert req.error is None and req.generated_tokens == [5, 6, 7]


def test_stop_with_timeout_force_retires_a_request_that_never_finishes():
    sched, _ = make(never_ending=True)
    sched.start()
    req = sched.submit(*prompt(), max_new_tokens=8000)
    deadline = time.time() + 5
    while not req.generated_tokens and time.time() < deadline:
        time.sleep(0.01)
    sched.stop(timeout=0.2)
    assert req.done.is_set() and isinstance(req.error, RuntimeError)


def test_engine_failure_surfaces_on_the_request():
    sched, eng = make([[5, 6]])

    def boom(sessions, tokens):
        raise RuntimeError("device lost")

    eng.step = boom
    req = sched.submit(*prompt(), max_new_tokens=2)
    drive(sched, 1)
    assert req.done.is_set() and "device lost" in str(req.error)
    assert threading.active_count() >= 1
