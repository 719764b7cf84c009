"""Decode-attention throughput of the fused paged path on one MI355X.

By default the line also carries configurations 1, 3, 4 and 5 as sub-records under
"configs" (each with its own step or token rate, HBM and host-link GB/s against their peaks,
and the reference's CPU path timed on its K/V); --configs "" leaves them out.

Workload (one "step" = one decode step of one layer over the whole batch): Qwen2.5-0.5B
attention geometry (14 query heads, 2 KV heads, head_dim 64, fp16, 32-token blocks), batch 8,
contexts drawn uniform in [1024, 32768] from a seed, each sequence keeping its 64 most recent
blocks in HBM and the rest in pinned host RAM (recent_only placement). Every step appends one
token per sequence, reads the host blocks over the host link (in place, or through a staging
ring with --stream-mode staged), attends, and evicts the block that leaves the resident
window. `value` is the (HBM + host) K/V bytes per step over the step time; `host_link` the
host part against PCIe Gen5 x16.

The HBM roofline is measured on the same batch with every block resident, over 24 layers
(1.45 GB of K/V per step, beyond the 256 MB MALL): `roofline` is paged_attn_kernel's K/V
bytes per launch over its launch time there, each step's launches run again back to back
between one pair of HIP events (and, beside it, each launch between its own pair of events,
which adds the time from each start marker to its dispatch). `roofline_by_launch_size` repeats that
measurement at batch 16, 32 and 64, at batch 8 with every context 32768 tokens, and for a
Mistral-7B layer, each row with its whole per-layer step as well (--no-launch-scale leaves it
out). `operator_api` times the six-function operator API at the shapes of the reference's
kernel probe (--no-operator leaves it out). Synthetic N(0,1)*0.5 data. Prints one JSON line.
"""
from __future__ import annotations

import argparse
import contextlib
import gc
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "rust-llm-pager_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
LINK_PEAK_GBS = 64.0  # PCIe Gen5 x16 per direction
MIB16 = 16 * 1024 * 1024

CFG = dict(batch=8, hq=14, hkv=2, d=64, tpb=32, ctx_lo=1024, ctx_hi=32768, resident_blocks=64, seed=2)


def draw_contexts(seed, batch, lo, hi):
    import torch

    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (batch,), generator=g).tolist()


def build(steps_total, staging_blocks=2048, staging_buffers=3, blocks_per_wg=32, resident_blocks=None,
          target_wg=0, layers=1, stream_mode="direct"):
    import torch

    from pager_hf import PagedDecoder

    c = dict(CFG)
    if resident_blocks is not None:
        c["resident_blocks"] = resident_blocks
    ctx = draw_contexts(c["seed"], c["batch"], c["ctx_lo"], c["ctx_hi"])
    dec = PagedDecoder(
        num_layers=layers, num_query_heads=c["hq"], num_kv_heads=c["hkv"], head_dim=c["d"], tokens_per_block=c["tpb"],
        dtype=torch.float16, device="cuda", pool_blocks=c["batch"] * (c["resident_blocks"] + 4),
        host_blocks=sum(n // c["tpb"] + steps_total // c["tpb"] + 8 for n in ctx), staging_blocks=staging_blocks,
        staging_buffers=staging_buffers, blocks_per_workgroup=blocks_per_wg, target_workgroups=target_wg,
        stream_mode=stream_mode,
    )
    gen = torch.Generator(device="cuda").manual_seed(c["seed"])
    sids = []
    for n in ctx:
        sid = dec.add_session(capacity_tokens=n + steps_total + 64, vram_budget=c["resident_blocks"] * MIB16,
                              ram_budget=1 << 40, recent_window=c["resident_blocks"] - 1, policy="recent_only")
        ks = [(torch.randn(1, c["hkv"], n, c["d"], device="cuda", generator=gen) * 0.5).half() for _ in range(layers)]
        vs = [(torch.randn(1, c["hkv"], n, c["d"], device="cuda", generator=gen) * 0.5).half() for _ in range(layers)]
        dec.prefill(sid, ks, vs, n)
        del ks, vs
        sids.append(sid)
    S = c["batch"]
    q = (torch.randn(steps_total, S, c["hq"], c["d"], device="cuda", generator=gen) * 0.5).half()
    kn = (torch.randn(steps_total, S, c["hkv"], c["d"], device="cuda", generator=gen) * 0.5).half()
    vn = (torch.randn(steps_total, S, c["hkv"], c["d"], device="cuda", generator=gen) * 0.5).half()
    out = torch.empty(S, c["hq"], c["d"], dtype=torch.float16, device="cuda")
    torch.cuda.synchronize()
    return dec, sids, ctx, q, kn, vn, out


# Spin-kernel cycles queued ahead of each step of a pass that stamps its launches with
# events: the GPU then reaches a launch's start event after the host has queued the launch,
# so the events hold the GPU's time only (without it, a host a little slower than the GPU
# adds its submission time to some launches' intervals).
TIMING_SPIN_CYCLES = 1_000_000


@contextlib.contextmanager
def gc_paused():
    """Python's cyclic garbage collector off over a wall-clock timed region, after one
    collection, as `timeit` does: a full collection pass (milliseconds with torch loaded) would
    otherwise land in some steps and not others."""
    was = gc.isenabled()
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()


def run_steps(dec, sids, q, kn, vn, out, first, count, stats, spin=0):
    import torch

    for i in range(first, first + count):
        if spin:
            torch.cuda._sleep(spin)
        dec.begin_step(sids)
        st = dec.pool.step_stats()
        stats["resident_tokens"] += st["resident_tokens"]
        stats["host_tokens"] += st["host_tokens"]
        stats["copies"] += st["copies"]
        stats["launches"] += st["launches"]
        for layer in range(dec.num_layers):
            dec.decode_layer(layer, q[i], kn[i], vn[i], out)
        dec.end_step(collect=False)


def hbm_all_resident(layers, steps, warmup, target_wg=0, blocks_per_wg=32):
    """The same batch with every block resident in HBM, over `layers` layers (one launch pair
    per layer, so the K/V read per step exceeds the 256 MB MALL and comes from HBM)."""
    import torch

    dec, sids, ctx, q, kn, vn, out = build(warmup + 3 * steps, resident_blocks=1100, layers=layers,
                                          target_wg=target_wg, blocks_per_wg=blocks_per_wg)
    stats = {"resident_tokens": 0, "host_tokens": 0, "copies": 0, "launches": 0}
    run_steps(dec, sids, q, kn, vn, out, 0, warmup, stats)
    # Pass 1: step rate (no per-launch events): the GPU's time over the steps, between two
    # events on the stream, the first queued behind a spin kernel so that the host has queued
    # the first step when the GPU reaches it, as in a decode loop; and the wall clock.
    stats = {"resident_tokens": 0, "host_tokens": 0, "copies": 0, "launches": 0}
    torch.cuda.synchronize()
    dec.pool.sync()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with gc_paused():
        t0 = time.perf_counter()
        torch.cuda._sleep(TIMING_SPIN_CYCLES)
        e0.record()
        run_steps(dec, sids, q, kn, vn, out, warmup, steps, stats)
        e1.record()
        torch.cuda.synchronize()
        dec.pool.sync()
        wall = time.perf_counter() - t0
    dt = e0.elapsed_time(e1) / 1e3
    # Pass 2: the attention kernel's own execution time, event-stamped per launch.
    dec.pool.kernel_time()
    dec.pool.set_timing(True)
    run_steps(dec, sids, q, kn, vn, out, warmup + steps, steps, {"resident_tokens": 0, "host_tokens": 0,
                                                                  "copies": 0, "launches": 0},
              spin=TIMING_SPIN_CYCLES)
    torch.cuda.synchronize()
    dec.pool.sync()
    k_ms, k_launches, k_bytes = dec.pool.kernel_time()
    dec.pool.set_timing(False)
    # Pass 3: the same launches back to back, one pair of events around each step's launches
    # (pgr_kv_bench_attention, after the step's own layers; every launch reads its work items
    # from the device copy of the plan, as the step's launches after its first do).
    b2b_us = b2b_bytes = 0.0
    first = warmup + 2 * steps
    for i in range(first, first + steps):
        torch.cuda._sleep(TIMING_SPIN_CYCLES)
        dec.begin_step(sids)
        for layer in range(layers):
            dec.decode_layer(layer, q[i], kn[i], vn[i], out)
        us, nb = dec.pool.bench_attention([q[i]] * layers, [kn[i]] * layers, [vn[i]] * layers)
        b2b_us += us
        b2b_bytes += nb
        dec.end_step(collect=False)
    torch.cuda.synchronize()
    dec.pool.sync()
    dec.pool.close()
    b2b_us /= steps
    b2b_bytes = int(b2b_bytes // steps)
    ceiling = plain_read_ceiling(k_bytes // max(k_launches, 1), layers)
    ceiling_b2b = plain_read_ceiling(b2b_bytes, layers, back_to_back=True)
    c = CFG
    tok_bytes = 2 * c["hkv"] * c["d"] * 2
    layer_bytes = stats["resident_tokens"] * tok_bytes // steps  # K/V bytes one layer-step reads
    kernel_gbs = k_bytes / (k_ms / 1e3) / 1e9
    step_gbs = layer_bytes * layers * steps / dt / 1e9
    return {
        "workload": f"the same batch with every block resident in HBM, {layers} layers",
        "layers": layers,
        "steps": steps,
        "kv_bytes_per_layer_step": layer_bytes,
        "ms_per_step": round(dt / steps * 1e3, 4),
        "wall_ms_per_step": round(wall / steps * 1e3, 4),
        "tokens_per_s": round(c["batch"] * steps / dt, 2),
        "kernel": {"name": "paged_attn_kernel", "launches": k_launches,
                   "avg_launch_us": round(k_ms * 1e3 / max(k_launches, 1), 3),
                   "bytes_per_launch": k_bytes // max(k_launches, 1),
                   "achieved": round(kernel_gbs, 2), "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
                   "timing": "each launch of the steps between its own pair of fence-free events"},
        "kernel_back_to_back": {"name": "paged_attn_kernel", "launches": layers * steps,
                                "avg_launch_us": round(b2b_us, 3), "bytes_per_launch": b2b_bytes,
                                "achieved": round(b2b_bytes / b2b_us / 1e3, 2),
                                "frac": round(b2b_bytes / b2b_us / 1e3 / HBM_PEAK_GBS, 4),
                                "timing": f"each step's attention launches again, the {layers} back to back between "
                                          "one pair of fence-free events (plan on the device)"},
        "step": {"achieved": round(step_gbs, 2), "frac": round(step_gbs / HBM_PEAK_GBS, 4),
                 "note": "whole decode step per layer (planning, both kernels, host glue) over K/V bytes, "
                         "GPU time between stream events around the steps (ms_per_step)"},
        "plain_read_ceiling": ceiling,
        "plain_read_ceiling_back_to_back": ceiling_b2b,
        "unit": "GB/s",
        "peak": HBM_PEAK_GBS,
    }


def plain_read_ceiling(nbytes, buffers, reps=96, back_to_back=False):
    """A plain streaming read of `nbytes` in one launch (768 workgroups x 256 threads, the decode
    kernel's grid at batch 8), rotating over `buffers` buffers so that the bytes come from HBM,
    each launch between fence-free events (pgr_bench_stream_read), or with `back_to_back` the
    launches back to back between one pair of events (pgr_bench_stream_read_back_to_back): what
    one launch reading the kernel's bytes can reach on this device."""
    import ctypes

    import torch

    import _pgr_native as nat

    lib = nat.load()
    nbytes = nbytes // 16 * 16
    bufs = [torch.zeros(nbytes, dtype=torch.uint8, device="cuda") for _ in range(buffers)]
    ptrs = (ctypes.c_void_p * buffers)(*[b.data_ptr() for b in bufs])
    us = ctypes.c_double(0)
    stream = torch.cuda.current_stream().cuda_stream
    fn = lib.pgr_bench_stream_read_back_to_back if back_to_back else lib.pgr_bench_stream_read
    nat.check(fn(ptrs, buffers, nbytes, 768, 24, ctypes.byref(us), stream), "warmup")
    nat.check(fn(ptrs, buffers, nbytes, 768, reps, ctypes.byref(us), stream), "stream read")
    del bufs
    gbs = nbytes / (us.value * 1e3)
    return {"bytes": nbytes, "workgroups": 768, "avg_launch_us": round(us.value, 3), "achieved": round(gbs, 2),
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def h2d_copy_ceiling(nbytes, reps=16):
    """hipMemcpyAsync host-to-device from pinned memory (torch's non-blocking copy), `reps`
    copies of `nbytes` back to back between HIP events: what the copy engines reach over the
    host link on this device."""
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True).fill_(1)
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src, non_blocking=True)
    e1.record()
    e1.synchronize()
    gbs = nbytes * reps / (e0.elapsed_time(e1) * 1e6)
    del src, dst
    return {"bytes": nbytes, "reps": reps, "achieved": round(gbs, 2), "frac": round(gbs / LINK_PEAK_GBS, 4)}


def host_read_ceiling(nbytes, workgroups=(16, 32, 64, 128, 256, 512), buffers=4, reps=48):
    """A plain streaming read of `nbytes` of pinned host memory, read in place over the host
    link by one launch (pgr_bench_stream_read, fence-free events), at each grid size in
    `workgroups`, rotating over `buffers` buffers: the fastest read of a launch's host bytes."""
    import ctypes

    import torch

    import _pgr_native as nat

    lib = nat.load()
    nbytes = nbytes // 16 * 16
    bufs = [torch.empty(nbytes, dtype=torch.uint8, pin_memory=True).zero_() for _ in range(buffers)]
    ptrs = (ctypes.c_void_p * buffers)(*[b.data_ptr() for b in bufs])
    us = ctypes.c_double(0)
    stream = torch.cuda.current_stream().cuda_stream
    by_wg = {}
    for wg in workgroups:
        nat.check(lib.pgr_bench_stream_read(ptrs, buffers, nbytes, wg, 8, ctypes.byref(us), stream), "warmup")
        nat.check(lib.pgr_bench_stream_read(ptrs, buffers, nbytes, wg, reps, ctypes.byref(us), stream), "host read")
        by_wg[wg] = round(us.value, 3)
    del bufs
    best = min(by_wg, key=by_wg.get)
    gbs = nbytes / (by_wg[best] * 1e3)
    return {"bytes": nbytes, "best_workgroups": best, "avg_launch_us": by_wg[best], "achieved": round(gbs, 2),
            "frac": round(gbs / LINK_PEAK_GBS, 4), "us_by_workgroups": by_wg}


KERNEL_SOURCES = ("rust-llm-pager_amd/csrc/attn_kernels.hip", "rust-llm-pager_amd/csrc/pgr_common.h",
                  "rust-llm-pager_amd/build.py")


def kernel_source_hash():
    """sha256 (first 16 hex digits) of the decode kernel's source and build flags: a counter
    summary measured on other sources is not reported as this kernel's traffic."""
    import hashlib

    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def committed_traffic(workload_layers):
    """HBM bytes per launch of the all-resident kernel from the committed counter summary
    (FETCH_SIZE and WRITE_SIZE scaled by a plain copy's readings), or None when the summary
    was measured on other kernel sources or another workload."""
    path = os.path.join(ROOT, "profiles", "paged_attn_all_resident_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    if t.get("layers") != workload_layers or t.get("batch") != CFG["batch"]:
        return None
    if t.get("kernel_source_sha256_16") != kernel_source_hash():
        return None
    return t.get("traffic_bytes_per_launch")


def continuous(args):
    """Continuous-batching decode: Qwen2.5-1.5B architecture (28 layers, hidden 1536, 12 query
    heads, 2 KV heads, head_dim 128, bf16, random init), 64 concurrent requests, prompts
    lognormal(median 4096, sigma 1) clipped to [256, 65536], outputs U[64, 512], a new request
    admitted whenever one finishes; 4 GB of HBM K/V budget (68 logical blocks per session) and
    the rest in pinned host RAM. Times `rounds` scheduler rounds after the first (which opens
    the first 64 requests); returns one JSON-able dict."""
    import numpy as np
    import torch
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from pager_hf.serving.scheduler import ContinuousBatchingScheduler

    conc, T = 64, 32
    cfg = Qwen2Config(hidden_size=1536, intermediate_size=8960, num_hidden_layers=28, num_attention_heads=12,
                      num_key_value_heads=2, vocab_size=151936, max_position_embeddings=131072, rope_theta=1e6,
                      tie_word_embeddings=True)
    torch.manual_seed(0)
    with torch.device("cuda"):
        model = Qwen2ForCausalLM(cfg)
    model = model.to(torch.bfloat16).eval()
    rng = np.random.default_rng(5)
    n_req = conc + args.cb_extra_requests
    lens = np.clip(np.exp(rng.normal(np.log(4096), 1.0, n_req)), 256, 65536).astype(int).tolist()
    outs = rng.integers(64, 513, n_req).tolist()
    per_session_blocks = int(4e9 // (conc * (2 * 2 * 128 * 2 * T * 28)))  # 68: real bytes -> logical blocks
    sched = ContinuousBatchingScheduler(
        model, SimpleTokenizer(), max_concurrent_sessions=conc,
        total_vram_budget=conc * per_session_blocks * MIB16, total_ram_budget=1 << 42, policy=args.cb_policy,
        tokens_per_block=T, max_context_tokens=65536 + 1024, host_token_capacity=args.cb_host_tokens,
        max_queue_depth=n_req, device="cuda", stream_mode=args.cb_stream_mode, staging_blocks=args.cb_staging_blocks,
        staging_buffers=args.cb_staging_buffers,
    )
    g = torch.Generator().manual_seed(6)
    reqs = [sched.submit(torch.randint(0, cfg.vocab_size, (1, n), generator=g), torch.ones(1, n, dtype=torch.long),
                         max_new_tokens=m) for n, m in zip(lens, outs)]
    eng = sched.engine()
    host_bytes = [0]
    hbm_bytes = [0]
    orig_step = eng.step
    kv_tok = 2 * 2 * 128 * 2 * 28  # K+V bytes of one token over all layers

    def step(sessions, tokens):
        out = orig_step(sessions, tokens)
        if len(sessions) > 1:
            host_bytes[0] += eng.host_bytes_per_step()
            hbm_bytes[0] += eng.decoder.pool.step_stats()["resident_tokens"] * kv_tok
        return out

    eng.step = step
    t_open = time.perf_counter()
    sched._admit_new_requests()
    sched._run_once()  # opens and first-steps the first 64 requests
    torch.cuda.synchronize()
    t_open = time.perf_counter() - t_open
    tokens0 = sum(len(r.generated_tokens) for r in reqs)
    host_bytes[0] = hbm_bytes[0] = 0
    live = sum(r.context_tokens for r in sched._active)
    live_lens = [r.context_tokens for r in sched._active]
    with gc_paused():
        t0 = time.perf_counter()
        for _ in range(args.cb_rounds):
            sched._admit_new_requests()
            sched._run_once()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
    tokens = sum(len(r.generated_tokens) for r in reqs) - tokens0
    hbm_store = eng.decoder.pool.hbm_bytes()
    sched.stop()
    link = host_bytes[0] / dt / 1e9
    hbm = hbm_bytes[0] / dt / 1e9
    return {
        "metric": "continuous-batching decode tokens/s (64 concurrent, Qwen2.5-1.5B arch, 4 GB HBM K/V budget)",
        "value": round(tokens / dt, 2),
        "unit": "tokens/s",
        "rounds": args.cb_rounds,
        "ms_per_round": round(dt / args.cb_rounds * 1e3, 2),
        "tokens": tokens,
        "live_tokens_at_start": live,
        "first_round_s": round(t_open, 2),
        "host_link": {"achieved": round(link, 3), "peak": LINK_PEAK_GBS, "unit": "GB/s",
                      "frac": round(link / LINK_PEAK_GBS, 4),
                      "bytes_per_round": host_bytes[0] // args.cb_rounds},
        "hbm": {"achieved": round(hbm, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(hbm / HBM_PEAK_GBS, 4),
                "bytes_per_round": hbm_bytes[0] // args.cb_rounds},
        "live_context_lengths": live_lens,
        "hbm_kv_bytes": hbm_store,
        "dtype": "bf16",
        "data": "synthetic: random-init weights, random token ids",
        "config": {"workload": "continuous batching, Qwen2.5-1.5B architecture, 64 concurrent, prompts lognormal("
                               "median 4096, sigma 1) clipped [256, 65536], outputs U[64, 512], admit on finish",
                   "policy": args.cb_policy, "per_session_hbm_blocks": per_session_blocks, "tokens_per_block": T,
                   "stream_mode": args.cb_stream_mode, "staging_blocks": args.cb_staging_blocks,
                   "staging_buffers": args.cb_staging_buffers,
                   "requests": n_req},
    }


def register(args):
    """Prompt registration at Qwen2.5-0.5B geometry (24 layers, 2 KV heads, head_dim 64, fp16,
    32-token blocks, 64 resident blocks, recent_only): for prompts of 8k, 32k and 64k tokens,
    (a) prefill with placement: every block written straight to its tier, host blocks into
    the pinned mirror over the host link; (b) prefill in HBM, then the first step's placement
    burst that evicts all but the recent blocks. Reports the time and the host-link rate of
    each (K/V bytes that crossed the link / time)."""
    import torch

    from pager_hf import PagedDecoder

    L, HQ, HKV, D, T = 24, 14, 2, 64, 32
    rows = []
    for n in (8192, 32768, 65536):
        g = torch.Generator(device="cuda").manual_seed(n)
        ks = [(torch.randn(1, HKV, n, D, device="cuda", generator=g) * 0.5).half() for _ in range(L)]
        vs = [(torch.randn(1, HKV, n, D, device="cuda", generator=g) * 0.5).half() for _ in range(L)]
        line = {"prompt_tokens": n}
        for place in (True, False):
            best = None
            for _ in range(args.register_reps):
                dec = PagedDecoder(num_layers=L, num_query_heads=HQ, num_kv_heads=HKV, head_dim=D, tokens_per_block=T,
                                   dtype=torch.float16, device="cuda", pool_blocks=n // T + 16,
                                   host_blocks=n // T + 16, staging_blocks=256, staging_buffers=2)
                sid = dec.add_session(capacity_tokens=n + 64, vram_budget=64 * MIB16, ram_budget=1 << 40,
                                      recent_window=63, policy="recent_only")
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                moves = dec.prefill(sid, ks, vs, n - 1, place=place)
                if not place:  # the first step's placement (no attention: the tiers the pager picks)
                    s = dec.sessions[sid]
                    nb = (n - 1) // T
                    s.pager.on_step(nb - 1, 0, [1.0 / nb] * nb)
                    s.pager.force_rebalance(nb - 1)
                    _, to_cpu, _, _ = dec.pool.apply_tiers(sid, s.pager.tiers())
                    moves = {"to_cpu": to_cpu}
                torch.cuda.synchronize()
                dec.pool.sync()
                dt = time.perf_counter() - t0
                host_blocks = len(moves["to_cpu"]) if not place else sum(1 for _ in dec.pool.block_ids(sid, False))
                best = dt if best is None or dt < best else best
                dec.pool.close()
            link = host_blocks * T * 2 * HKV * D * 2 * L
            key = "prefill_placed" if place else "prefill_then_evict"
            line[key] = {"ms": round(best * 1e3, 2), "host_bytes": link, "host_link_GBs": round(link / best / 1e9, 2)}
        rows.append(line)
        del ks, vs
    return {
        "metric": "prompt registration time and host-link GB/s (Qwen2.5-0.5B geometry, 24 layers)",
        "value": rows[1]["prefill_then_evict"]["host_link_GBs"],
        "unit": "GB/s",
        "higher_is_better": True,
        "sizes": rows,
        "dtype": "fp16",
        "data": "synthetic K/V",
        "config": {"workload": "prompt registration, 8k/32k/64k tokens, 64 resident blocks of 32 tokens, recent_only",
                   "value_is": "32k prompt, HBM prefill then the first placement burst"},
    }


def _cpu_attention_rate(groups, n_rep, d, budget_s):
    """Dense fp32 attention plus block mass in torch on the host threads over (k, v) groups
    ([Hkv, n, D] fp16/bf16 each, upcast included); returns (seconds per pass, threads)."""
    import os

    import torch

    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    previous = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        gen = torch.Generator().manual_seed(1)
        qs = [(torch.randn(k.shape[0], n_rep, d, generator=gen) * 0.5).to(k.dtype) for k, _ in groups]
        passes = 0
        t0 = time.perf_counter()
        while True:
            for q, (k, v) in zip(qs, groups):
                n = k.shape[1]
                w = torch.softmax((q.float() @ k.float().transpose(1, 2)) / d ** 0.5, dim=-1)
                _ = w @ v.float()
                nb = -(-n // 32)
                _ = torch.nn.functional.pad(w, (0, nb * 32 - n)).view(k.shape[0], n_rep, nb, 32).sum(-1)
            passes += 1
            if time.perf_counter() - t0 > budget_s:
                break
        return (time.perf_counter() - t0) / passes, threads
    finally:
        torch.set_num_threads(previous)


def _rate(bytes_per_step, seconds_per_step, peak):
    gbs = bytes_per_step / seconds_per_step / 1e9
    return {"bytes_per_step": int(bytes_per_step), "GBs": round(gbs, 3), "peak": peak, "frac": round(gbs / peak, 4)}


def _cpu_record(kv_bytes, seconds, tokens, threads, sample):
    """The reference's CPU path on the same in-scope K/V: GB/s and tokens/s."""
    return {"value": round(kv_bytes / seconds / 1e9, 3), "unit": "GB/s", "tokens_per_s": round(tokens / seconds, 2),
            "cores": threads, "kind": "port", "sample": sample}


def _layer_config(args, name, *, hq, hkv, d, dtype, batch, ctx, resident, window, steps, warmup):
    """One decoder layer over `batch` sequences of `ctx` tokens, the `resident` most recent blocks
    in HBM (recent_only) and the rest on host, optionally a sliding window; `steps` decode steps,
    each appending one token per sequence. The prompt holds ctx - warmup tokens, so that the
    untimed warmup steps bring every sequence to ctx tokens when the timed steps start."""
    import torch

    from pager_hf import PagedDecoder

    T = 32
    nb = ctx // T
    dec = PagedDecoder(num_layers=1, num_query_heads=hq, num_kv_heads=hkv, head_dim=d, tokens_per_block=T,
                       dtype=dtype, device="cuda", pool_blocks=batch * (resident + 8),
                       host_blocks=batch * (nb + (3 * steps + warmup) // T + 16), staging_blocks=64, staging_buffers=2)
    g = torch.Generator(device="cuda").manual_seed(ctx)
    sids, cpu_groups = [], []
    for _ in range(batch):
        sid = dec.add_session(capacity_tokens=ctx + 3 * steps + warmup + 64, vram_budget=resident * MIB16,
                              ram_budget=1 << 42, recent_window=resident - 1, policy="recent_only")
        pre = ctx - warmup
        k = (torch.randn(1, hkv, pre, d, device="cuda", generator=g) * 0.5).to(dtype)
        v = (torch.randn(1, hkv, pre, d, device="cuda", generator=g) * 0.5).to(dtype)
        dec.prefill(sid, [k], [v], pre)
        lo = max(pre - (window or pre), 0)
        cpu_groups.append((k[0, :, lo:].cpu(), v[0, :, lo:].cpu()))
        del k, v
        sids.append(sid)
    q = (torch.randn(batch, hq, d, device="cuda", generator=g) * 0.5).to(dtype)
    kn = (torch.randn(batch, hkv, d, device="cuda", generator=g) * 0.5).to(dtype)
    host = res_tok = 0

    def one(i):
        if window:
            for sid in sids:
                dec.set_lo(sid, [ctx - warmup + i - window + 1])
        dec.begin_step(sids)
        st = dec.pool.step_stats()
        dec.decode_layer(0, q, kn, kn)
        dec.end_step(collect=False)
        return st

    for i in range(warmup):
        one(i)
    torch.cuda.synchronize()
    dec.pool.sync()
    with gc_paused():
        t0 = time.perf_counter()
        for i in range(warmup, warmup + steps):
            st = one(i)
            host += st["host_tokens"]
            res_tok += st["resident_tokens"]
        torch.cuda.synchronize()
        dec.pool.sync()
        dt = (time.perf_counter() - t0) / steps
    # The host's time per step: the same calls timed one by one, without synchronizing;
    # begin_step's wait for the GPU to finish reading the plan buffer it reuses (the host runs
    # at most a step ahead) is reported apart, the rest is the host's own work.
    host_s = wait_s = 0.0
    with gc_paused():
        for i in range(warmup + steps, warmup + 2 * steps):
            h0 = time.perf_counter()
            st = one(i)
            host_s += time.perf_counter() - h0
            wait_s += st["plan_wait_ns"] * 1e-9
    torch.cuda.synchronize()
    dec.pool.sync()
    # The attention launch's own execution time, event-stamped per launch.
    dec.pool.kernel_time()
    dec.pool.set_timing(True)
    for i in range(warmup + 2 * steps, warmup + 3 * steps):
        torch.cuda._sleep(TIMING_SPIN_CYCLES)
        one(i)
    torch.cuda.synchronize()
    dec.pool.sync()
    k_ms, k_launches, k_bytes = dec.pool.kernel_time()
    dec.pool.set_timing(False)
    hbm_store = dec.pool.hbm_bytes()
    dec.pool.close()
    tok_bytes = 2 * hkv * d * 2
    host_b, hbm_b = host / steps * tok_bytes, res_tok / steps * tok_bytes
    cpu_s, threads = _cpu_attention_rate(cpu_groups, hq // hkv, d, args.cpu_seconds / 3)
    cpu_bytes = sum(k.numel() * 2 * 2 for k, _ in cpu_groups)
    return {
        "workload": name,
        "steps": steps,
        "ms_per_step": round(dt * 1e3, 4),
        "host_ms_per_step": round(host_s / steps * 1e3, 4),
        "host_plan_wait_ms_per_step": round(wait_s / steps * 1e3, 4),
        "host_work_ms_per_step": round((host_s - wait_s) / steps * 1e3, 4),
        "tokens_per_s": round(batch / dt, 1),
        "kv_GBs": round((host_b + hbm_b) / dt / 1e9, 2),
        "host_link": _rate(host_b, dt, LINK_PEAK_GBS),
        "hbm": _rate(hbm_b, dt, HBM_PEAK_GBS),
        "hbm_kv_bytes": hbm_store,
        "attention_launch": {"avg_us": round(k_ms * 1e3 / max(k_launches, 1), 3), "launches": k_launches,
                             "kv_bytes": k_bytes // max(k_launches, 1)},
        "host_read_ceiling": host_read_ceiling(int(host_b)) if host_b else None,
        "cpu_baseline": _cpu_record(cpu_bytes, cpu_s, batch, threads,
                                    f"dense fp32 attention and block mass in torch over the same in-scope K/V of "
                                    f"all {batch} sequences, repeated for ~{args.cpu_seconds / 3:.0f} s"),
    }


def config1(args):
    import torch

    return _layer_config(args, "one Qwen2.5-0.5B layer (14q/2kv, D 64, fp16), batch 1, 4096 tokens in 32-token "
                               "blocks: the 8 most recent in HBM, 120 on host (recent_only); 128 timed steps from "
                               "4096 tokens after 512 warmup steps",
                         hq=14, hkv=2, d=64, dtype=torch.float16, batch=1, ctx=4096, resident=8, window=None,
                         steps=128, warmup=512)


def config4(args):
    import torch

    return _layer_config(args, "one Mistral-7B layer (32q/8kv, D 128, bf16), batch 4, 131072 tokens, window 4096: "
                               "32 in-window blocks in HBM, 96 on host; 32 timed steps from 131072 tokens after 32 "
                               "warmup steps",
                         hq=32, hkv=8, d=128, dtype=torch.bfloat16, batch=4, ctx=131072, resident=32, window=4096,
                         steps=32, warmup=32)


def config3(args):
    """TinyLlama-1.1B architecture (22 layers, 32q/4kv, D 64, intermediate 5632, fp16, random
    init), 8192 random prompt ids, 256 greedy tokens, sinks_heavy_hitter with a 41-block budget
    (4 sinks + 8 recent + 29 by score) and 32-token blocks; decode steps replayed from HIP
    graphs in the direct and staged stream modes (the faster one reported; eager direct for
    comparison). The prompt is registered by a first generate() call."""
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM

    from pager_hf import PagedModel

    cfg = LlamaConfig(hidden_size=2048, intermediate_size=5632, num_hidden_layers=22, num_attention_heads=32,
                      num_key_value_heads=4, vocab_size=32000, max_position_embeddings=8448 + 64, rms_norm_eps=1e-5)
    torch.manual_seed(7)
    with torch.device("cuda"):
        model = LlamaForCausalLM(cfg)
    model = model.to(torch.float16).eval()
    g = torch.Generator().manual_seed(8)
    ids = torch.randint(0, 32000, (1, 8192), generator=g).cuda()
    n_new = args.c3_tokens
    timed = {}
    mirror_copies = None
    # (eager or graphs, stream mode): host blocks read in place by the attention kernel
    # ("direct"), copied to an HBM staging buffer on a second stream, each layer's under the
    # layer before it ("staged"), or copied by DMA into per-layer HBM mirrors beside the
    # whole replayed step ("mirror"). --c3-runs selects some of them (for traces).
    runs = [r for r in args.c3_runs.split(",") if r]
    known = ("eager_direct", "graphs_direct", "graphs_staged", "graphs_mirror")
    if not runs or any(r not in known for r in runs):
        raise SystemExit(f"--c3-runs takes a comma list of {', '.join(known)}; got {args.c3_runs!r}")
    for graphs, mode in ((False, "direct"), (True, "direct"), (True, "staged"), (True, "mirror")):
        if ("graphs_" if graphs else "eager_") + mode not in runs:
            continue
        pm = PagedModel(model, vram_budget=41 * MIB16, ram_budget=1 << 40, recent_window=8,
                        policy="sinks_heavy_hitter", tokens_per_block=32, max_context_tokens=8192 + 512,
                        use_hip_graphs=graphs, stream_mode=mode)
        first = pm.generate(ids, torch.ones_like(ids), 1)
        ids2 = torch.cat([ids, torch.tensor([first], device="cuda")], dim=1)
        torch.cuda.synchronize()
        with gc_paused():
            t0 = time.perf_counter()
            out = pm.generate(ids2, torch.ones_like(ids2), n_new)
            torch.cuda.synchronize()
            t_tok = (time.perf_counter() - t0) / n_new
        timed[(graphs, mode)] = (t_tok, pm.last_run_stats, pm.decoder.pool.hbm_bytes())
        if mode == "mirror":
            # The DMA copies of each layer's host share, event-timed by the store on its copy
            # stream over 16 more tokens (apart from the timed run, which they would perturb).
            ids3 = torch.cat([ids2, torch.tensor([out], device="cuda")], dim=1)
            pm.decoder.pool.set_timing(True)
            pm.generate(ids3, torch.ones_like(ids3), 16)
            pm.decoder.pool.set_timing(False)
            ms, n_cp, nbytes = pm.decoder.pool.copy_time()
            pm.decoder.pool.kernel_time()  # drop the eager launches' timings
            mirror_copies = {"layer_copy_groups": n_cp, "avg_us": round(ms * 1e3 / max(n_cp, 1), 2),
                             "avg_bytes": nbytes // max(n_cp, 1),
                             "GBs": round(nbytes / max(ms, 1e-9) / 1e6, 2),
                             "note": "each layer's DMA copies into its ring buffer, HIP events on the store's copy "
                                     "stream, 16 tokens after the timed run"}
        pm.reset()
    best = min(timed, key=lambda k: (not k[0], timed[k][0]))  # the fastest graph run
    dt, st, hbm_store = timed[best]
    del model
    torch.cuda.empty_cache()
    kv_tok = 2 * 4 * 64 * 2 * 22  # K+V bytes of one token over all layers
    in_scope = 8192 + n_new // 2  # mean context over the timed tokens
    host_b = st.total_cpu_to_gpu_mb * 1e6 / n_new
    hbm_b = in_scope * kv_tok - host_b
    # CPU: the attention of one decode step over all 22 layers at the mean context.
    gen = torch.Generator().manual_seed(9)
    groups = [((torch.randn(4, in_scope, 64, generator=gen) * 0.5).half(),
               (torch.randn(4, in_scope, 64, generator=gen) * 0.5).half()) for _ in range(22)]
    cpu_s, threads = _cpu_attention_rate(groups, 8, 64, args.cpu_seconds / 3)
    return {
        "workload": "TinyLlama-1.1B architecture (22 layers, 32q/4kv, D 64, fp16, random init), 8192-token prompt, "
                    "256 greedy tokens, sinks_heavy_hitter 41 blocks (4 sinks + 8 recent + 29 scored), 32-token "
                    "blocks, decode steps from HIP graphs",
        "tokens": n_new,
        "stream_mode": best[1],
        "ms_per_token": round(dt * 1e3, 3),
        "tokens_per_s": round(1 / dt, 1),
        "ms_per_token_by_run": {("graphs_" if g else "eager_") + m: round(timed[(g, m)][0] * 1e3, 3)
                                for g, m in timed},
        "kv_GBs": round(in_scope * kv_tok / dt / 1e9, 2),
        "host_link": _rate(host_b, dt, LINK_PEAK_GBS),
        "hbm": _rate(hbm_b, dt, HBM_PEAK_GBS),
        "mean_attention_in_gpu": round(st.mean_attention_in_gpu, 4),
        "hbm_kv_bytes": hbm_store,
        "hbm_kv_bytes_by_run": {("graphs_" if g else "eager_") + m: timed[(g, m)][2]["total"] for g, m in timed},
        "hbm_budget_bytes": 41 * 32 * kv_tok,  # the 41-block placement budget, all layers
        "mirror_copies": mirror_copies,
        "cpu_baseline": _cpu_record(in_scope * kv_tok, cpu_s, 1, threads,
                                    f"dense fp32 attention and block mass in torch for all 22 layers of one decode "
                                    f"step at the mean context ({in_scope} tokens), repeated for "
                                    f"~{args.cpu_seconds / 3:.0f} s; attention only, not the model's other layers"),
    }


def config5(args):
    """Continuous batching (see continuous()), as a sub-record with the reference's CPU attention
    path timed on a bounded sample of the same round."""
    import numpy as np
    import torch

    res = continuous(args)
    lens = res["live_context_lengths"]
    kv_tok_layer = 2 * 2 * 128 * 2
    round_bytes = sum(lens) * kv_tok_layer * 28  # every layer's in-scope K/V of one round
    # CPU sample: 8 sessions drawn from the live ones (contexts capped at 16384), 2 layers each.
    rng = np.random.default_rng(7)
    pick = [min(int(n), 16384) for n in rng.choice(lens, 8, replace=False)]
    gen = torch.Generator().manual_seed(10)
    groups = [((torch.randn(2, n, 128, generator=gen) * 0.5).bfloat16(),
               (torch.randn(2, n, 128, generator=gen) * 0.5).bfloat16()) for n in pick for _ in range(2)]
    cpu_s, threads = _cpu_attention_rate(groups, 6, 128, args.cpu_seconds / 3)
    sample_bytes = sum(k.numel() * 2 * 2 for k, _ in groups)
    cpu_gbs = sample_bytes / cpu_s / 1e9
    round_s = round_bytes / (cpu_gbs * 1e9)
    dt = res["ms_per_round"] / 1e3
    return {
        "workload": res["config"]["workload"] + "; 4 GB real HBM K/V bytes = 68 logical blocks per session; "
                                                "recent_only; staged host streaming with cross-layer prefetch",
        "rounds": res["rounds"],
        "ms_per_round": res["ms_per_round"],
        "tokens_per_s": res["value"],
        "live_tokens_at_start": res["live_tokens_at_start"],
        "host_link": {"bytes_per_step": res["host_link"]["bytes_per_round"], "GBs": res["host_link"]["achieved"],
                      "peak": LINK_PEAK_GBS, "frac": res["host_link"]["frac"]},
        "hbm": {"bytes_per_step": res["hbm"]["bytes_per_round"], "GBs": res["hbm"]["achieved"],
                "peak": HBM_PEAK_GBS, "frac": res["hbm"]["frac"]},
        "kv_GBs": round((res["host_link"]["bytes_per_round"] + res["hbm"]["bytes_per_round"]) / dt / 1e9, 2),
        "hbm_kv_bytes": res["hbm_kv_bytes"],
        "cpu_baseline": {"value": round(cpu_gbs, 3), "unit": "GB/s", "tokens_per_s": round(64 / round_s, 2),
                         "cores": threads, "kind": "port",
                         "sample": f"dense bf16->fp32 attention and block mass in torch over 8 of the live sessions "
                                   f"(contexts {pick}, capped at 16384) x 2 layers for ~{args.cpu_seconds / 3:.0f} s; "
                                   f"tokens/s = 64 / (one round's {round_bytes / 1e9:.1f} GB of in-scope K/V at "
                                   f"that rate)"},
    }


CONFIG_RUNNERS = {"1": config1, "3": config3, "4": config4, "5": config5}


def configs(args):
    """The other configurations, each as a sub-record (see config1/3/4/5)."""
    names = [c for c in args.configs.split(",") if c]
    out = {}
    for name in names:
        print(f"[bench] configuration {name}", file=sys.stderr, flush=True)
        out[name] = CONFIG_RUNNERS[name](args)
    return out


def hbm_scale_rows(batches=(8, 16, 32, 64), mistral=True, full_context=True):
    """The all-resident attention kernel as the bytes per launch grow: Qwen2.5-0.5B geometry
    (14q/2kv, D 64, fp16) at the given batches with contexts U[1024, 32768], the same layer at
    batch 8 with every context 32768 tokens (with the plain-read ceiling of its bytes), and a
    Mistral-7B layer (32q/8kv, D 128, bf16) at batch 4 x 32768 tokens. Every block resident,
    several layers so the K/V read per step exceeds the MALL. Per row: the attention launches
    back to back, each step's launches again between one pair of fence-free events
    (pgr_kv_bench_attention), and each between its own pair of events (`per_launch_events`;
    each step queued behind a spin kernel); and the whole per-layer step (both kernels,
    planning, host glue) between two events around 16 steps."""
    import torch

    from pager_hf import PagedDecoder

    T = 32
    out = []

    def measure(name, hq, hkv, d, dtype, ctxs, layers, steps=16, warmup=2, ceiling=False):
        nb = [c // T + 2 for c in ctxs]
        dec = PagedDecoder(num_layers=layers, num_query_heads=hq, num_kv_heads=hkv, head_dim=d, tokens_per_block=T,
                           dtype=dtype, device="cuda", pool_blocks=sum(nb) + 16 * len(ctxs),
                           host_blocks=sum(nb) + 16 * len(ctxs), staging_blocks=16)
        g = torch.Generator(device="cuda").manual_seed(len(ctxs))
        sids = []
        for c, n in zip(ctxs, nb):
            sid = dec.add_session(capacity_tokens=c + 64, vram_budget=(n + 8) * MIB16, ram_budget=1 << 40,
                                  recent_window=n + 4, policy="recent_only")
            ks = [(torch.randn(1, hkv, c, d, device="cuda", generator=g) * 0.5).to(dtype) for _ in range(layers)]
            vs = [(torch.randn(1, hkv, c, d, device="cuda", generator=g) * 0.5).to(dtype) for _ in range(layers)]
            dec.prefill(sid, ks, vs, c, place=False)
            del ks, vs
            sids.append(sid)
        S = len(ctxs)
        q = (torch.randn(S, hq, d, device="cuda", generator=g) * 0.5).to(dtype)
        kn = (torch.randn(S, hkv, d, device="cuda", generator=g) * 0.5).to(dtype)

        def run(n, spin=0):
            for _ in range(n):
                if spin:
                    torch.cuda._sleep(spin)
                dec.begin_step(sids)
                for layer in range(layers):
                    dec.decode_layer(layer, q, kn, kn)
                dec.end_step(collect=False)

        run(warmup)
        # Whole steps (planning, both kernels per layer, host glue), no per-launch events: the
        # GPU's time from the first step's start to the last step's end, between two events on
        # the stream, the first queued behind a spin kernel so that the host has queued the
        # first step when the GPU reaches it (as in a decode loop, where the host plans a step
        # while the GPU runs the one before).
        torch.cuda.synchronize()
        dec.pool.sync()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with gc_paused():
            torch.cuda._sleep(4 * TIMING_SPIN_CYCLES)  # ~2 ms: longer than planning a batch-64 step
            e0.record()
            run(steps)
            e1.record()
            torch.cuda.synchronize()
            dec.pool.sync()
        layer_us = e0.elapsed_time(e1) * 1e3 / (steps * layers)
        # The attention launches alone, each between its own pair of events.
        dec.pool.kernel_time()
        dec.pool.set_timing(True)
        run(steps, spin=TIMING_SPIN_CYCLES)
        torch.cuda.synchronize()
        dec.pool.sync()
        ms, n, by = dec.pool.kernel_time()
        dec.pool.set_timing(False)
        per_us = ms * 1e3 / n
        # The same launches back to back: each step's launches again between one pair of events.
        b2b = 0.0
        for _ in range(steps):
            torch.cuda._sleep(TIMING_SPIN_CYCLES)
            dec.begin_step(sids)
            for layer in range(layers):
                dec.decode_layer(layer, q, kn, kn)
            b2b += dec.pool.bench_attention([q] * layers, [kn] * layers, [kn] * layers)[0]
            dec.end_step(collect=False)
        torch.cuda.synchronize()
        dec.pool.sync()
        dec.pool.close()
        us = b2b / steps
        nbytes = by // n
        row = {"workload": name, "bytes_per_launch": nbytes, "avg_launch_us": round(us, 2),
               "achieved": round(nbytes / us / 1e3, 1), "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4),
               "per_launch_events_us": round(per_us, 2),
               "per_launch_events_frac": round(nbytes / per_us / 1e3 / HBM_PEAK_GBS, 4),
               "layer_step_us": round(layer_us, 2),
               "layer_step_frac": round(nbytes / layer_us / 1e3 / HBM_PEAK_GBS, 4)}
        if ceiling:
            c = plain_read_ceiling(nbytes, layers, back_to_back=True)
            row["plain_read_ceiling"] = c
            row["frac_of_ceiling"] = round(nbytes / us / 1e3 / c["achieved"], 4)
        out.append(row)

    # Qwen2.5-0.5B's 24 layers per step: the K/V read per step is past the MALL, and the host's
    # planning and placement per step (O(blocks)) run beside the GPU's layers, as in the model.
    for batch in batches:
        ctxs = draw_contexts(CFG["seed"], batch, CFG["ctx_lo"], CFG["ctx_hi"])
        measure(f"0.5B layer, batch {batch}, contexts U[1024,32768], 24 layers", 14, 2, 64, torch.float16,
                ctxs, 24)
    if full_context:
        measure("0.5B layer, batch 8, every context 32768, 24 layers", 14, 2, 64, torch.float16,
                [32768] * 8, 24, ceiling=True)
    if mistral:
        measure("Mistral-7B layer (32q/8kv, D 128, bf16), batch 4 x 32768, 4 layers", 32, 8, 128, torch.bfloat16,
                [32768] * 4, 4)
    return out


def hbm_scale(args):
    """--workload hbm-scale: hbm_scale_rows() at batch 8 to 64, batch 8 x 32768 and the Mistral-7B layer."""
    out = hbm_scale_rows()
    return {
        "metric": "all-resident paged attention HBM GB/s against bytes per launch",
        "value": out[-1]["achieved"],
        "unit": "GB/s",
        "higher_is_better": True,
        "rows": out,
        "peak": HBM_PEAK_GBS,
        "dtype": "fp16 / bf16",
        "data": "synthetic K/V",
        "config": {"workload": "all-resident decode attention at growing batch; value is the D=128 case"},
    }


def operator_api(dtype_name="float16"):
    """The six-function operator API (streaming_attention_state_init, _step, _finalize) on one
    contiguous K/V chunk, the way the reference's own kernel probe times it
    (bench/streaming_attention_kernel_scaling_probe.py:42-53, 56-65: Qwen2.5-7B shape, 28
    query heads, 4 KV heads, head_dim 128, batch 1, 3 warmup calls, 20 timed between two
    events, state init + step + finalize per call), at the probe's chunk sizes and at 32768
    tokens, with torch's eager attention (matmul, softmax, matmul over repeated KV heads) on
    the same inputs beside it as the probe does. K/V GB/s counts the chunk's K and V bytes."""
    import ctypes

    import torch

    import _pgr_native as nat
    from pager_hf.streaming_attention import (streaming_attention_finalize, streaming_attention_state_init,
                                              streaming_attention_step)

    lib = nat.load()

    dtype = getattr(torch, dtype_name)
    hq, hkv, d = 28, 4, 128
    n_rep = hq // hkv
    g = torch.Generator(device="cuda").manual_seed(3)

    def time_cuda(fn, warmup=3, reps=20):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / reps

    rows = []
    for tokens in (64, 256, 1024, 2048, 4096, 32768):
        q = (torch.randn(1, hq, d, device="cuda", generator=g) * 0.5).to(dtype)
        k = (torch.randn(1, hkv, tokens, d, device="cuda", generator=g) * 0.5).to(dtype)
        v = (torch.randn(1, hkv, tokens, d, device="cuda", generator=g) * 0.5).to(dtype)

        def ours():
            m, l, acc = streaming_attention_state_init(1, hq, d, q.device)
            streaming_attention_step(q, k, v, m, l, acc)
            streaming_attention_finalize(acc, l, q.dtype)

        def eager():
            kd = k.repeat_interleave(n_rep, dim=1)
            vd = v.repeat_interleave(n_rep, dim=1)
            scores = torch.matmul(kd, q.unsqueeze(3)) * (1.0 / d ** 0.5)  # [1, Hq, T, 1]
            probs = torch.softmax(scores.float(), dim=2).to(dtype)
            torch.matmul(probs.transpose(2, 3).contiguous(), vd)  # [1, Hq, 1, D]

        ms = time_cuda(ours)
        ms_eager = time_cuda(eager)
        # The same call captured once and replayed: the device's own time per call, without the
        # host's launch overhead (an eager call is host-bound below a few thousand tokens).
        ours()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            ours()
        ms_graph = time_cuda(graph.replay)
        del graph
        # The fold kernel alone: event pairs around each of 20 attention launches (the library's
        # operator timing), without the state init, merge and finalize launches of a call. The
        # timed calls rotate over copies of the chunk whose bytes together exceed the 256 MB
        # MALL (up to 8 copies), so that a launch's K/V come from HBM, and each call is queued
        # behind a spin kernel of ~100 us, so that the GPU reaches a launch's start event after
        # the host has queued the launch: the events then hold the GPU's time only, not the
        # host's time between recording the start event and submitting the launch (an eager
        # call is host-bound).
        n_copy = max(1, min(8, -(-(320 << 20) // (2 * k.numel() * k.element_size()))))
        chunks = [(k, v)] + [(k.clone(), v.clone()) for _ in range(n_copy - 1)]

        def ours_on(kc, vc):
            m, l, acc = streaming_attention_state_init(1, hq, d, q.device)
            streaming_attention_step(q, kc, vc, m, l, acc)
            streaming_attention_finalize(acc, l, q.dtype)

        for kc, vc in chunks:
            ours_on(kc, vc)
        torch.cuda.synchronize()
        nat.check(lib.pgr_attn_set_timing(1), "pgr_attn_set_timing")
        for i in range(20):
            torch.cuda._sleep(250_000)
            ours_on(*chunks[i % n_copy])
        fold_ms, fold_n, fold_bytes = ctypes.c_double(0), ctypes.c_int64(0), ctypes.c_int64(0)
        nat.check(lib.pgr_attn_kernel_time(ctypes.byref(fold_ms), ctypes.byref(fold_n), ctypes.byref(fold_bytes)),
                  "pgr_attn_kernel_time")
        nat.check(lib.pgr_attn_set_timing(0), "pgr_attn_set_timing")
        fold_us = fold_ms.value * 1e3 / max(fold_n.value, 1)
        fold_gbs = fold_bytes.value / max(fold_n.value, 1) / (fold_us * 1e3)
        # The same fold launches back to back over the chunk copies, without the merges, at
        # least 20 of them between one pair of events (pgr_attn_bench_step), queued behind a
        # spin kernel so that the host has queued them when the GPU reaches the first.
        ws_bytes = lib.pgr_attn_workspace_bytes(1, hq, hkv, tokens, d, nat.MODE_FOLD, 16)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
        karr = (ctypes.c_void_p * n_copy)(*[kc.data_ptr() for kc, _ in chunks])
        varr = (ctypes.c_void_p * n_copy)(*[vc.data_ptr() for _, vc in chunks])
        b2b_us, b2b_bytes = ctypes.c_double(0), ctypes.c_int64(0)
        code = {torch.float16: nat.DTYPE_F16, torch.bfloat16: nat.DTYPE_BF16}[q.dtype]
        torch.cuda._sleep(TIMING_SPIN_CYCLES)
        nat.check(lib.pgr_attn_bench_step(q.data_ptr(), karr, varr, n_copy, 1, hq, hkv, tokens, d, code, 1.0 / d**0.5,
                                          ws.data_ptr(), ws_bytes,
                                          max(3, -(-20 // n_copy)), ctypes.byref(b2b_us), ctypes.byref(b2b_bytes),
                                          torch.cuda.current_stream().cuda_stream), "pgr_attn_bench_step")
        b2b_gbs = b2b_bytes.value / (b2b_us.value * 1e3)
        del chunks, ws
        kv = 2 * hkv * tokens * d * k.element_size()
        rows.append({"tokens": tokens, "ms_per_call": round(ms, 4), "torch_eager_ms": round(ms_eager, 4),
                     "ms_per_call_graph": round(ms_graph, 4), "kv_GBs_graph": round(kv / ms_graph / 1e6, 1),
                     "hbm_frac_graph": round(kv / ms_graph / 1e6 / HBM_PEAK_GBS, 4),
                     "fold_us": round(fold_us, 3), "fold_GBs": round(fold_gbs, 1),
                     "fold_frac": round(fold_gbs / HBM_PEAK_GBS, 4),
                     "fold_us_back_to_back": round(b2b_us.value, 3), "fold_GBs_back_to_back": round(b2b_gbs, 1),
                     "fold_frac_back_to_back": round(b2b_gbs / HBM_PEAK_GBS, 4)})
    return {
        "workload": "operator API, Qwen2.5-7B shape (28q/4kv, D 128), batch 1, one contiguous chunk per call; "
                    "state_init + step + finalize per call, 20 calls between two events (ms_per_call: eager calls, "
                    "as the reference's probe times them; ms_per_call_graph: replays of the call captured in a HIP "
                    "graph; fold_us / fold_frac: the attention kernel alone, events around each launch, its K+V "
                    "bytes over 8 TB/s, timed calls rotating over chunk copies beyond the MALL and queued behind a "
                    "spin kernel so that the events hold GPU time only; fold_*_back_to_back: the same launches over "
                    "the same copies back to back between one pair of events)",
        "dtype": dtype_name, "rows": rows,
    }


def calibrate_host_read(mib):
    """Reads `mib` MiB of host-resident records once with records_to_hf_kernel, which reads the
    pinned host mirror in place through its device mapping: a known number of bytes over the
    host link (K and V of every host block of one layer), for the host-link read counters.
    Returns the bytes read from host memory."""
    import torch

    from pager_hf import PagedDecoder

    T, hkv, d = 32, 2, 64
    rec = 2 * hkv * T * d * 2
    n_blocks = (mib << 20) // rec
    n = n_blocks * T
    dec = PagedDecoder(num_layers=1, num_query_heads=14, num_kv_heads=hkv, head_dim=d, tokens_per_block=T,
                       dtype=torch.float16, device="cuda", pool_blocks=8, host_blocks=n_blocks + 8, staging_blocks=8)
    sid = dec.add_session(capacity_tokens=n + 64, vram_budget=MIB16, ram_budget=1 << 42, recent_window=0,
                          policy="recent_only")
    k = torch.zeros(1, hkv, n, d, dtype=torch.float16, device="cuda")
    dec.prefill(sid, [k], [k], n)
    host_blocks = len(dec.pool.block_ids(sid, False))
    torch.cuda.synchronize()
    dec.pool.export_tokens(sid, 0, 0, n)  # one launch: host records read in place, resident ones from HBM
    torch.cuda.synchronize()
    dec.pool.close()
    return host_blocks * rec


class SimpleTokenizer:
    eos_token_id = None


def cpu_baseline(ctx, budget_s=15.0):
    """The reference's CPU path timed on the host: dense fp32 GQA attention plus the per-block
    attention mass (the math of tests/test_streaming_attention.py:20-40, as the reference's
    torch prototype runs it on CPU), over a bounded sample of whole steps of the same batch
    (fp16 K/V upcast included), with torch on the host threads this job may use.
    Returns KV GB/s and tokens/s."""
    import os

    import torch

    c = CFG
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    previous = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        g = torch.Generator().manual_seed(0)
        n_rep, d, T = c["hq"] // c["hkv"], c["d"], c["tpb"]
        kv = [((torch.randn(c["hkv"], n + 1, d, generator=g) * 0.5).half(),
               (torch.randn(c["hkv"], n + 1, d, generator=g) * 0.5).half()) for n in ctx]
        q = (torch.randn(c["hkv"], n_rep, d, generator=g) * 0.5).half()
        scale = 1.0 / d ** 0.5
        bytes_per_step = sum((n + 1) * 2 * c["hkv"] * d * 2 for n in ctx)
        steps = 0
        t0 = time.perf_counter()
        while True:
            for k, v in kv:
                n = k.shape[1]
                w = torch.softmax((q.float() @ k.float().transpose(1, 2)) * scale, dim=-1)  # [Hkv, n_rep, n]
                _ = w @ v.float()
                nb = -(-n // T)
                _ = torch.nn.functional.pad(w, (0, nb * T - n)).view(c["hkv"], n_rep, nb, T).sum(-1)
            steps += 1
            if time.perf_counter() - t0 > budget_s or steps >= 2000:
                break
        dt = time.perf_counter() - t0
    finally:
        torch.set_num_threads(previous)
    return {
        "value": round(bytes_per_step * steps / dt / 1e9, 3),
        "unit": "GB/s",
        "tokens_per_s": round(c["batch"] * steps / dt, 2),
        "cores": threads,
        "kind": "port",
        "sample": f"{steps} full decode steps of the batch-8 workload: dense fp32 attention and block mass in torch "
                  f"on {threads} host threads (fp16 K/V upcast included), {dt:.1f} s",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-operator", action="store_true",
                    help="leave out operator_api (the streaming_attention_* operators at the reference probe's shapes)")
    ap.add_argument("--no-launch-scale", action="store_true",
                    help="leave out roofline_by_launch_size (the all-resident kernel at batch 16 to 64)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--staging-blocks", type=int, default=2048, help="records per staging buffer")
    ap.add_argument("--staging-buffers", type=int, default=3)
    ap.add_argument("--blocks-per-wg", type=int, default=32, help="largest block count per workgroup")
    ap.add_argument("--resident-blocks", type=int, default=CFG["resident_blocks"],
                    help="HBM-resident blocks per sequence (1100 keeps every block resident)")
    ap.add_argument("--target-wg", type=int, default=0, help="workgroups per attention launch (0 = library default)")
    ap.add_argument("--stream-mode", choices=["direct", "staged"], default="direct",
                    help="host blocks read in place over the host link, or copied into a staging ring")
    ap.add_argument("--resident-layers", type=int, default=24,
                    help="layers of the all-resident HBM measurement (0 skips it)")
    ap.add_argument("--workload", choices=["batch8", "continuous", "register", "configs", "hbm-scale", "operator"],
                    default="batch8",
                    help="batch8: the headline line (configuration 2, plus the configurations in --configs as "
                         "sub-records); continuous: the 64-request continuous-batching run alone; register: prompt "
                         "registration at 8k-64k tokens; configs: only the configurations in --configs; "
                         "hbm-scale: the all-resident kernel against bytes per launch; operator: the operator API "
                         "rows alone")
    ap.add_argument("--configs", default="1,3,4,5",
                    help="other configurations measured into the line (comma list of 1, 3, 4, 5; empty for none)")
    ap.add_argument("--register-reps", type=int, default=3)
    ap.add_argument("--c3-runs", default="eager_direct,graphs_direct,graphs_staged,graphs_mirror",
                    help="configuration 3: which runs to time (eager_direct, graphs_direct, graphs_staged, "
                         "graphs_mirror)")
    ap.add_argument("--c3-tokens", type=int, default=256, help="configuration 3: greedy tokens per run")
    ap.add_argument("--cb-rounds", type=int, default=24)
    ap.add_argument("--cb-extra-requests", type=int, default=64)
    ap.add_argument("--cb-policy", default="recent_only")
    ap.add_argument("--cb-host-tokens", type=int, default=800_000)
    ap.add_argument("--cb-stream-mode", choices=["direct", "staged"], default="staged")
    ap.add_argument("--cb-staging-blocks", type=int, default=8192, help="records per staging buffer (staged mode)")
    ap.add_argument("--cb-staging-buffers", type=int, default=2, help="staging buffers (staged mode)")
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="after timing, run one device copy of this size (HBM counter calibration)")
    ap.add_argument("--calibration-host-mib", type=int, default=0,
                    help="after timing, read this many MiB of host-resident records once through the host mirror's "
                         "device mapping (host-link counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1).", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    if args.workload == "hbm-scale":
        line = hbm_scale(args)
        line.update({"n_gpus": 1, "steps": 8, "warmup": 2, "scaling": "weak", "vs_baseline": None})
        print(json.dumps(line), flush=True)
        return 0
    if args.workload == "operator":
        line = {"metric": "operator API calls (streaming_attention_state_init / _step / _finalize)",
                "operator_api": operator_api(), "n_gpus": 1, "scaling": "weak", "vs_baseline": None,
                "data": "synthetic N(0,1)*0.5, seeded"}
        print(json.dumps(line), flush=True)
        return 0
    if args.workload == "configs":
        line = {"metric": "per-configuration decode-attention measurements", "configs": configs(args),
                "n_gpus": 1, "scaling": "weak", "vs_baseline": None, "data": "synthetic K/V and random-init weights"}
        print(json.dumps(line), flush=True)
        return 0
    if args.workload == "register":
        line = register(args)
        line.update({"n_gpus": 1, "steps": args.register_reps, "warmup": 0, "scaling": "weak", "vs_baseline": None})
        print(json.dumps(line), flush=True)
        return 0
    if args.workload == "continuous":
        line = continuous(args)
        line.update({"n_gpus": 1, "steps": args.cb_rounds, "warmup": 1, "higher_is_better": True, "scaling": "weak",
                     "vs_baseline": None})
        print(json.dumps(line), flush=True)
        return 0
    c = CFG
    total = args.warmup + 2 * args.steps
    dec, sids, ctx, q, kn, vn, out = build(total, args.staging_blocks, args.staging_buffers, args.blocks_per_wg,
                                          args.resident_blocks, args.target_wg, 1, args.stream_mode)
    warm = {"resident_tokens": 0, "host_tokens": 0, "copies": 0, "launches": 0}
    run_steps(dec, sids, q, kn, vn, out, 0, args.warmup, warm)
    # Pass 1: step rate, with no per-launch events (each start/stop pair costs the step ~4.6 us).
    stats = {"resident_tokens": 0, "host_tokens": 0, "copies": 0, "launches": 0}
    torch.cuda.synchronize()
    dec.pool.sync()
    with gc_paused():
        t0 = time.perf_counter()
        run_steps(dec, sids, q, kn, vn, out, args.warmup, args.steps, stats)
        torch.cuda.synchronize()
        dec.pool.sync()
        dt = time.perf_counter() - t0
    # Pass 2: the attention kernel's own execution time, event-stamped per launch.
    dec.pool.kernel_time()
    dec.pool.set_timing(True)
    run_steps(dec, sids, q, kn, vn, out, args.warmup + args.steps, args.steps,
              {"resident_tokens": 0, "host_tokens": 0, "copies": 0, "launches": 0}, spin=TIMING_SPIN_CYCLES)
    torch.cuda.synchronize()
    dec.pool.sync()
    k_ms, k_launches, k_bytes = dec.pool.kernel_time()

    tok_bytes = 2 * c["hkv"] * c["d"] * 2  # K + V per token per layer
    # What the host link carries at best on this device (outside the timed region): copy
    # engines (pinned hipMemcpyAsync H2D) and one kernel launch reading a step's host bytes in
    # place over the link, as the attention launch does.
    step_host_bytes = stats["host_tokens"] * tok_bytes // args.steps
    link_ceilings = {
        "h2d_copy": h2d_copy_ceiling(64 << 20),
        "kernel_read": host_read_ceiling(step_host_bytes, workgroups=(64, 128, 256, 512, 768, 1024), reps=12),
    }
    io_bytes = args.steps * c["batch"] * c["hq"] * c["d"] * 2 * 2  # q in + out
    hbm_bytes = stats["resident_tokens"] * tok_bytes + io_bytes
    host_bytes = stats["host_tokens"] * tok_bytes
    value = (hbm_bytes + host_bytes) / dt / 1e9
    kernel_gbs = k_bytes / (k_ms / 1e3) / 1e9 if k_ms > 0 else 0.0
    link_gbs = host_bytes / dt / 1e9
    line = {
        "metric": "decode-attn KV GB/s (HBM + host link, % peak) & tokens/s, 32k ctx",
        "value": round(value, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic N(0,1)*0.5, seeded",
        "config": {
            "workload": "single-layer streaming decode attention, Qwen2.5-0.5B geometry (14q/2kv, d64, fp16), "
                        "batch 8, contexts U[1024,32768] seed 2, 32-token blocks, 64 recent blocks per sequence in "
                        "HBM and the rest in pinned host RAM, 1 token appended per sequence per step",
            "contexts": ctx,
            "batch": c["batch"],
            "stream_mode": args.stream_mode,
            "blocks_per_workgroup": args.blocks_per_wg,
            "staging": {"records_per_buffer": args.staging_blocks, "buffers": args.staging_buffers},
        },
        "tokens_per_s": round(c["batch"] * args.steps / dt, 2),
        "host_link": {
            "achieved": round(link_gbs, 3),
            "peak": LINK_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(link_gbs / LINK_PEAK_GBS, 4),
            "bytes_per_step": host_bytes // args.steps,
            "copies_per_step": stats["copies"] / args.steps,
            "note": "host-resident K/V bytes per step over the step time; peak = PCIe Gen5 x16 nominal",
            "ceilings": link_ceilings,
            "frac_of_kernel_read": round(link_gbs / link_ceilings["kernel_read"]["achieved"], 4),
        },
        "hbm_resident": {"bytes_per_step": hbm_bytes // args.steps, "blocks_per_sequence": args.resident_blocks},
        "kernel": {
            "name": "paged_attn_kernel",
            "launches": k_launches,
            "avg_launch_us": round(k_ms * 1e3 / max(k_launches, 1), 3),
            "bytes_per_launch": k_bytes // max(k_launches, 1),
            "achieved": round(kernel_gbs, 2),
            "unit": "GB/s",
            "note": "K/V bytes (HBM + host) per launch over the launch time in this workload (a second pass of "
                    "the same number of steps, event-stamped per launch)",
        },
    }
    if args.calibration_copy_mib:
        n = args.calibration_copy_mib << 20
        src = torch.ones(n // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        line["calibration_copy_bytes"] = n
        del src, dst
    if args.calibration_host_mib:
        line["calibration_host_read_bytes"] = calibrate_host_read(args.calibration_host_mib)
    dec.pool.close()
    del dec
    line["roofline"] = None
    if args.resident_layers > 0:
        res = hbm_all_resident(args.resident_layers, max(4, min(args.steps, 16)), 2, args.target_wg, args.blocks_per_wg)
        line["hbm_all_resident"] = res
        # The launch's duration: each step's 24 attention launches again, back to back between
        # one pair of events (the kernel's own time plus the gaps between launches); beside it
        # the conservative figure of the step's launches each between its own pair of events.
        kern, per = res["kernel_back_to_back"], res["kernel"]
        line["roofline"] = {
            "bound": "hbm",
            "kernel": "paged_attn_kernel",
            "workload": res["workload"],
            "achieved": kern["achieved"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": kern["frac"],
            "traffic": committed_traffic(args.resident_layers),
            "kernel_source_sha256_16": kernel_source_hash(),
            "launches": kern["launches"],
            "avg_launch_us": kern["avg_launch_us"],
            "bytes_per_launch": kern["bytes_per_launch"],
            "timing": kern["timing"],
            # A plain streaming read of the same bytes in one launch, same timing: the part of
            # the gap to peak that a kernel of this size can close.
            "plain_read_ceiling": res["plain_read_ceiling_back_to_back"],
            "frac_of_ceiling": round(kern["achieved"] / res["plain_read_ceiling_back_to_back"]["achieved"], 4),
            "per_launch_events": {
                "avg_launch_us": per["avg_launch_us"], "achieved": per["achieved"], "frac": per["frac"],
                "launches": per["launches"], "timing": per["timing"],
                "plain_read_ceiling": res["plain_read_ceiling"],
                "frac_of_ceiling": round(per["achieved"] / res["plain_read_ceiling"]["achieved"], 4),
            },
        }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(ctx, args.cpu_seconds)
    if args.configs:
        line["configs"] = configs(args)
    if not args.no_operator:
        line["operator_api"] = operator_api()
    if not args.no_launch_scale:
        # The same kernel, every block resident, as a launch carries more bytes: batch 8 is the
        # roofline above; a launch of several rounds of workgroups amortizes each workgroup's
        # fixed start, query wait and partial store. Batch 8 with every context at 32768 tokens
        # carries 134 MB per launch.
        line["roofline_by_launch_size"] = {
            "kernel": "paged_attn_kernel", "bound": "hbm", "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "rows": hbm_scale_rows(batches=(16, 32, 64), mistral=True),
        }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
