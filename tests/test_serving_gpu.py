"""Continuous batching on the GPU: every request's tokens against its own unpaged baseline.

The scheduler runs rounds directly (deterministic); requests of ragged prompt lengths and
output lengths share one native store and one forward per round. Parity is judged as in
test_paged_model_gpu.py (identical tokens up to the first baseline near-tie).
"""
from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from test_paged_model_gpu import MIB16, SMALL, _baseline, _check_free_running, _model

pytestmark = pytest.mark.gpu


def _run_all(sched, reqs, max_rounds=2000):
    for _ in range(max_rounds):
        sched._admit_new_requests()
        if not sched._active and sched._incoming.qsize() == 0:
            break
        sched._run_once()
    assert all(r.done.is_set() for r in reqs)
    for r in reqs:
        assert r.error is None, r.error


def test_continuous_batching_ragged_requests_match_unpaged():
    from pager_hf.serving.scheduler import ContinuousBatchingScheduler

    model = _model(SMALL, seed=21, init_std=0.05)
    g = torch.Generator().manual_seed(9)
    lens = [300, 450, 120, 600, 77, 500]
    news = [20, 35, 10, 25, 40, 15]
    prompts = [torch.randint(0, SMALL["vocab_size"], (1, n), generator=g).cuda() for n in lens]
    sched = ContinuousBatchingScheduler(
        model, SimpleNamespace(eos_token_id=None), max_concurrent_sessions=3, total_vram_budget=3 * 5 * MIB16,
        total_ram_budget=1 << 40, policy="sinks_heavy_hitter", tokens_per_block=16, max_context_tokens=1024,
        device="cuda",
    )
    reqs = [sched.submit(p, torch.ones_like(p), max_new_tokens=n) for p, n in zip(prompts, news)]
    _run_all(sched, reqs)
    for p, n, r in zip(prompts, news, reqs):
        want, _, gaps = _baseline(model, p, torch.ones_like(p), n)
        assert len(r.generated_tokens) == n
        _check_free_running([r.generated_tokens], want, gaps)
    assert len(sched.engine().sessions) == 0  # one-shot sessions are closed on retirement
    sched.stop()



def test_mistral_sliding_window_per_row():
    """Sliding window 64 with sessions at different positions in one batched step."""
    from transformers import MistralConfig, MistralForCausalLM

    from pager_hf import PagedModel
    from pager_hf.serving.scheduler import ContinuousBatchingScheduler

    cfg = MistralConfig(hidden_size=512, intermediate_size=1024, num_hidden_layers=3, num_attention_heads=8,
                        num_key_value_heads=2, vocab_size=2048, max_position_embeddings=4096, sliding_window=64,
                        initializer_range=0.05)
    torch.manual_seed(23)
    model = MistralForCausalLM(cfg).to(dtype=torch.float16, device="cuda").eval()
    g = torch.Generator().manual_seed(11)
    prompts = [torch.randint(0, 2048, (1, n), generator=g).cuda() for n in (180, 95, 260)]
    # Single session through PagedModel.
    pm = PagedModel(model, vram_budget=3 * MIB16, ram_budget=1 << 40, recent_window=2, tokens_per_block=16)
    want, _, gaps = _baseline(model, prompts[0], torch.ones_like(prompts[0]), 24)
    _check_free_running([pm.generate(prompts[0], torch.ones_like(prompts[0]), 24)], want, gaps)
    pm.reset()
    # Batched sessions at different positions.
    sched = ContinuousBatchingScheduler(
        model, SimpleNamespace(eos_token_id=None), max_concurrent_sessions=3, total_vram_budget=3 * 3 * MIB16,
        total_ram_budget=1 << 40, tokens_per_block=16, max_context_tokens=512, device="cuda",
    )
    reqs = [sched.submit(p, torch.ones_like(p), max_new_tokens=24) for p in prompts]
    _run_all(sched, reqs)
    for p, r in zip(prompts, reqs):
        want, _, gaps = _baseline(model, p, torch.ones_like(p), 24)
        _check_free_running([r.generated_tokens], want, gaps)
    sched.stop()
