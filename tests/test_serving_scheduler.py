"""ContinuousBatchingScheduler host logic on the CPU, with a fake engine.

Follows the reference's tests/test_serving_scheduler.py:71-425 where the admission and
round behaviour is shared (admission, EOS, the token stream, capacity and backpressure);
the batching cases check this build's rule instead (fresh requests step alone, every
started request joins one batched step per round). Rounds are driven directly
(_admit_new_requests / _run_once) except where the background thread itself is under test.
"""
from __future__ import annotations

import threading
import time
from types import SimpleNamespace

import pytest
import torch

from pager_hf.serving.scheduler import ContinuousBatchingScheduler, SchedulerAtCapacityError

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






def test_submit_raises_at_capacity():
    sched, _ = make(max_concurrent=1, max_queue_depth=1)
    sched.submit(*prompt(), max_new_tokens=1)
    sched.submit(*prompt(), max_new_tokens=1)
    with pytest.raises(SchedulerAtCapacityError):
        sched.submit(*prompt(), max_new_tokens=1)






def test_engine_failure_surfaces_on_the_request():
    sched, eng = make([[5, 6]])

    def boom(sessions, tokens):
        raise RuntimeError("device lost")

    eng.step = boom
    req = sched.submit(*prompt(), max_new_tokens=2)
    drive(sched, 1)
    assert req.done.is_set() and "device lost" in str(req.error)
    assert threading.active_count() >= 1


def test_background_thread_serves_requests_and_stop_fails_the_rest():
    sched, _ = make([[5, 6, 7]], never_ending=False)
    sched.start()
    req = sched.submit(*prompt(), max_new_tokens=3)
    assert req.done.wait(5)
    assert req.error is None and req.generated_tokens == [5, 6, 7]
    sched.stop()
    late = sched.submit(*prompt(), max_new_tokens=3)
    sched.stop()
    assert late.done.is_set() and isinstance(late.error, RuntimeError)


def test_one_argmax_per_round_over_the_batch():
    """The batched step reads all next tokens with one argmax over [S, V]."""
    sched, eng = make([[5, 6], [8, 9]], max_concurrent=2)
    calls = []
    real = torch.argmax

    def counting(t, *a, **k):
        calls.append(tuple(t.shape))
        return real(t, *a, **k)

    a = sched.submit(*prompt(), max_new_tokens=2)
    b = sched.submit(*prompt(start=10), max_new_tokens=2)
    drive(sched, 1)
    torch.argmax = counting
    try:
        drive(sched, 1)
    finally:
        torch.argmax = real
    assert calls == [(2, VOCAB)]
    assert a.generated_tokens == [5, 6] and b.generated_tokens == [8, 9]
