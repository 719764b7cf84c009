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


# Configuration 5: Qwen2.5-1.5B architecture (public intermediate size 8960 and vocab 151936),
# bf16, random init from a seed.
QWEN15 = dict(hidden_size=1536, intermediate_size=8960, num_hidden_layers=28, num_attention_heads=12,
              num_key_value_heads=2, vocab_size=151936, max_position_embeddings=131072, rope_theta=1e6,
              tie_word_embeddings=True)


def test_config5_continuous_batching_rounds_against_the_oracle():
    """Configuration 5 through the scheduler: 64 concurrent requests, prompts lognormal
    (median 4096, sigma 1) clipped to [256, 65536], outputs U[64, 512] except the first 8,
    which get U[8, 32] so that they finish and queued requests are admitted within the run;
    4 GB of real HBM K/V bytes = 68 logical blocks per session, recent_only, 32-token blocks.
    For 72 rounds every session's host-block list, new block ids and tier moves equal the
    oracle's (placement-only sessions, uniform scores). Two watched sessions with host blocks
    have their layer 0 and layer 27 attention checked against the dense oracle on three rounds
    (their K/V: the prompt's K/V as the model's prefill produced it, taken before the store
    imports it, then each round's k_new / v_new)."""
    import numpy as np
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from oracle.attention import dense_reference
    from oracle.paged_decode import PagedDecodeOracle
    from pager_hf.batched_decode import BatchedPagedEngine
    from pager_hf.serving.scheduler import ContinuousBatchingScheduler

    conc, T, rounds = 64, 32, 72
    cfg = Qwen2Config(**QWEN15)
    torch.manual_seed(0)
    with torch.device("cuda"):
        model = Qwen2ForCausalLM(cfg)
    model = model.to(torch.bfloat16).eval()
    rng = np.random.default_rng(5)
    n_req = conc + 16
    lens = np.clip(np.exp(rng.normal(np.log(4096), 1.0, n_req)), 256, 65536).astype(int).tolist()
    outs = rng.integers(64, 513, n_req)
    outs[:8] = rng.integers(8, 33, 8)
    blocks = int(4e9 // (conc * (2 * 2 * 128 * 2 * T * 28)))
    assert blocks == 68
    kw = dict(vram_budget=blocks * MIB16, ram_budget=1 << 36, recent_window=64, rebalance_interval=4,
              policy="recent_only")
    engine = BatchedPagedEngine(model, max_sessions=conc, vram_budget_per_session=kw["vram_budget"],
                                ram_budget_per_session=kw["ram_budget"], policy="recent_only", tokens_per_block=T,
                                max_context_tokens=65536 + 1024, host_token_capacity=900_000, collect_stats=True)
    sched = ContinuousBatchingScheduler(model, SimpleNamespace(eos_token_id=None), max_concurrent_sessions=conc,
                                        total_vram_budget=conc * kw["vram_budget"], total_ram_budget=1 << 42,
                                        policy="recent_only", tokens_per_block=T, max_context_tokens=65536 + 1024,
                                        max_queue_depth=n_req, device="cuda", engine=engine)
    g = torch.Generator().manual_seed(6)
    reqs = [sched.submit(torch.randint(0, cfg.vocab_size, (1, n), generator=g), torch.ones(1, n, dtype=torch.long),
                         max_new_tokens=int(m)) for n, m in zip(lens, outs)]
    # Watched: two requests that keep host blocks (prompt > 68 blocks) and run all rounds.
    watched = [i for i in range(8, conc) if 4000 < lens[i] < 20000][:2]
    assert len(watched) == 2
    layers_checked = (0, 27)
    check_rounds = {5, 30, 60}

    dec = engine.decoder
    # The watched requests' prompt K/V at layers 0 and 27, from the model's prefill, before the
    # store imports it (sid -> {layer: (K, V)}, overwritten when a sid is reused).
    prefill_kv: dict[int, dict] = {}
    watched_prefix = {lens[i] - 1 for i in watched}
    orig_prefill = dec.prefill

    def prefill(sid, keys, values, n_tokens, **kwargs):
        if n_tokens in watched_prefix:
            prefill_kv[sid] = {layer: (keys[layer][0, :, :n_tokens].float().cpu().numpy(),
                                       values[layer][0, :, :n_tokens].float().cpu().numpy())
                               for layer in layers_checked}
        return orig_prefill(sid, keys, values, n_tokens, **kwargs)

    dec.prefill = prefill
    ora = PagedDecodeOracle(num_layers=28, num_query_heads=12, num_kv_heads=2, head_dim=128, tokens_per_block=T)
    seen: dict[int, object] = {}  # id(engine session) -> request (sids are reused after a close)
    failures: list[BaseException] = []  # the scheduler turns exceptions of a step into request errors
    kv: dict[tuple[int, int], list] = {}  # (watched request, layer) -> [K [2, n, 128], V] float32
    captured = {}
    orig_decode = dec.decode_layer

    def decode_layer(layer, q, k_new, v_new, out=None, **kwargs):
        o = orig_decode(layer, q, k_new, v_new, out, **kwargs)
        if layer == 0:
            captured["gather"] = [dec.step_host_blocks(i) for i in range(q.shape[0])]
        if layer in layers_checked:
            captured[layer] = tuple(x.float().cpu().numpy() for x in (q, k_new, v_new, o))
        return o

    dec.decode_layer = decode_layer
    orig_step = engine.step
    n_checked = {"placement": 0, "attention": 0, "admitted": 0}
    round_no = {"r": 0}

    def step(sessions, tokens):
        try:
            return checked_step(sessions, tokens)
        except BaseException as exc:
            failures.append(exc)
            raise

    def checked_step(sessions, tokens):
        for s in sessions:  # sessions opened since the last step join the oracle
            if id(s) not in seen:
                req = next(r for r in reqs if r.engine_session is s)
                seen[id(s)] = req
                n_prefix = req.input_ids.shape[1] - 1
                ora.add_session(s.sid, **kw)
                ora.prefill(s.sid, None, None, n_prefix, place=False)
                idx = reqs.index(req)
                if idx >= conc:
                    n_checked["admitted"] += 1
                if idx in watched:
                    for layer in layers_checked:
                        k, v = prefill_kv[s.sid][layer]
                        assert k.shape == (2, n_prefix, 128)
                        kv[(idx, layer)] = [k, v]
        logits = orig_step(sessions, tokens)
        sids = [s.sid for s in sessions]
        ref = ora.step(sids, None, None, None, compute=False)
        assert captured["gather"] == ref["gather"], f"round {round_no['r']}: gather lists differ"
        for s in sessions:
            got, want = s.stats[-1], ref["placement"][s.sid]
            assert got["added_block_ids"] == want["added"]
            assert (got["to_gpu"], got["to_cpu"]) == (want["to_gpu"], want["to_cpu"]), f"session {s.sid} moves"
        n_checked["placement"] += len(sessions)
        for i, s in enumerate(sessions):
            idx = reqs.index(seen[id(s)])
            if idx not in watched:
                continue
            for layer in layers_checked:
                q, kn, vn, o = captured[layer]
                K, V = kv[(idx, layer)]
                K = np.concatenate([K, kn[i][:, None]], axis=1)
                V = np.concatenate([V, vn[i][:, None]], axis=1)
                kv[(idx, layer)] = [K, V]
                if round_no["r"] in check_rounds and len(sessions) > 1:
                    ref_o, _ = dense_reference(q[i][None], K[None], V[None], n_rep=6, tokens_per_block=T)
                    err = float(np.abs(o[i] - ref_o[0]).max())
                    assert err < 2e-3, f"round {round_no['r']}, request {idx}, layer {layer}: error {err}"
                    n_checked["attention"] += 1
        return logits

    engine.step = step
    for r in range(rounds):
        round_no["r"] = r
        sched._admit_new_requests()
        sched._run_once()
        if failures:
            raise failures[0]
        if r == 0:
            print(f"config 5: opened {len(seen)} sessions, {sum(x.context_tokens for x in sched._active)} live "
                  "tokens", flush=True)
    assert all(r.error is None for r in reqs if r.done.is_set())  # before stop() fails the unfinished ones
    sched.stop()
    assert n_checked["attention"] == 2 * len(layers_checked) * len(check_rounds)
    assert n_checked["admitted"] >= 8  # the short requests finished and queued ones took their places
    print(f"config 5: {rounds} rounds, {n_checked['placement']} session-steps placed as the oracle, "
          f"{n_checked['admitted']} requests admitted after the first 64, {n_checked['attention']} attention checks")
