"""Seeded random decode scenarios: the fused paged decode against the CPU oracle under mixed
conditions that the targeted tests cover one at a time.

Each scenario draws a geometry, a stream mode (direct, staged with small or large staging
buffers, mirror), 1-3 layers, sessions of 1-2 rows (the second row left-padded) with their
own policies and budgets, a per-layer sliding window on some layers, and in about a third
of them steps captured into HIP graphs (one per launch signature, replayed when a signature
recurs); sessions then join and leave between steps, and some steps run only a subset of
the sessions. Every step is
checked as in the targeted tests: gather lists, move lists and new-block ids bit-exact, and
attention within max-abs 2e-3 of the fp32 oracle beyond two roundings to the model dtype
that the reference's kernel makes as well (P before P.V, and the output). Short contexts
give outputs near single V rows, where in bf16 each of them can exceed 2e-3 by itself; the
targeted tests, whose outputs average many tokens, hold the plain 2e-3.
"""
from __future__ import annotations

import random

import pytest
import torch

from test_paged_decode_gpu import MIB16, TOL, Pair

pytestmark = pytest.mark.gpu

GEOMETRIES = [
    # hq, hkv, d, tokens per block, dtype
    (8, 2, 64, 16, torch.float16),
    (14, 2, 64, 32, torch.float16),
    (32, 8, 128, 32, torch.bfloat16),
    (8, 1, 256, 16, torch.bfloat16),
    (4, 4, 32, 16, torch.float16),
]
POLICIES = ["recent_only", "sinks_recent", "heavy_hitter", "sinks_heavy_hitter"]
MODES = [("direct", 1024), ("staged", 48), ("staged", 4096), ("mirror", 1024)]


def _scenario(seed):
    r = random.Random(seed)
    hq, hkv, d, tpb, dtype = r.choice(GEOMETRIES)
    mode, staging = r.choice(MODES)
    layers = r.randint(1, 3)
    windows = [r.choice([None, None, 3 * tpb + 5, 7 * tpb]) for _ in range(layers)]
    graphs = r.random() < 0.35
    return r, dict(hq=hq, hkv=hkv, d=d, tpb=tpb, dtype=dtype, mode=mode, staging=staging, layers=layers,
                   windows=windows if any(w is not None for w in windows) else None, graphs=graphs)


@pytest.mark.parametrize("seed", range(40))
def test_random_scenario_matches_the_oracle(seed):
    r, sc = _scenario(seed)
    print(f"scenario {seed}: {sc}", flush=True)
    tpb = sc["tpb"]
    g = torch.Generator().manual_seed(1000 + seed)
    p = Pair(layers=sc["layers"], hq=sc["hq"], hkv=sc["hkv"], d=sc["d"], tpb=tpb, dtype=sc["dtype"],
             pool_blocks=600, host_blocks=2400, staging_blocks=sc["staging"], stream_mode=sc["mode"])
    live = []

    def join():
        rows = r.choice([1, 1, 2])
        ctx = r.randint(1, 40 * tpb)
        lo = None if rows == 1 else [0, r.randint(0, ctx // 2)]
        policy = r.choice(POLICIES)
        live.append(p.add(ctx=ctx, rows=rows, capacity=ctx + 48, gen=g, lo=lo,
                          vram_budget=r.randint(1, 8) * MIB16, ram_budget=r.choice([4, 1024]) * MIB16,
                          recent_window=r.randint(0, 4), rebalance_interval=r.choice([1, 2, 4]),
                          policy=policy))

    for _ in range(r.randint(2, 4)):
        join()
    errs = []
    graphs = {} if sc["graphs"] else None
    for step in range(24):
        if r.random() < 0.2:
            join()
        if r.random() < 0.15 and len(live) > 2:
            sid = live.pop(r.randrange(len(live)))
            p.dec.remove_session(sid)
            del p.ora.sessions[sid]
            p.sids.remove(sid)
        sids = list(live) if r.random() < 0.7 else sorted(r.sample(live, r.randint(1, len(live))))
        _, _, err = p.step(g, sids=sids, windows=sc["windows"], graphs=graphs, rounding_allowance=True)
        errs.append(err)
    assert max(errs) < TOL
