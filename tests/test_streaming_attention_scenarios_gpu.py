"""Seeded random operator-API sequences against the CPU oracle.

Each case draws a geometry (n_rep 1-16, head_dim 8-256, fp16, bf16 or fp32 q/k/v), a batch
of rows with their own padding masks and some rows inactive, a scale and softcap or the
defaults, a chunk length and a flow: one pass (state_init, fold steps, finalize) or two
passes (stats steps, accumulate steps with per-block mass over the full blocks, the tail by
fold_fixed, finalize), as paged_model.py:992-1067 drives the reference's kernels.

Checks, per case: inactive rows keep their state bit for bit; the outputs of the active rows
are within max-abs 2e-3 of the fp32 oracle (1e-4 for fp32 q/k/v) beyond two roundings to
the 16-bit dtype that the reference's kernel makes as well (P before P.V, at most
u sum p|v| / l <= u max|v|, and the output, at most u |out|; u = 2^-11 fp16, 2^-8 bf16);
block mass within 1e-4.
"""
from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from oracle import attention as oa
from pager_hf.streaming_attention import (
    streaming_attention_accumulate_step,
    streaming_attention_finalize,
    streaming_attention_fold_fixed_step,
    streaming_attention_state_init,
    streaming_attention_stats_step,
    streaming_attention_step,
)

pytestmark = pytest.mark.gpu

GEOMETRIES = [(14, 2, 64), (32, 8, 128), (8, 8, 64), (16, 1, 32), (28, 4, 128), (8, 1, 256), (4, 2, 16),
              (6, 3, 8), (12, 2, 128), (16, 16, 64)]
DTYPES = [torch.float16, torch.bfloat16, torch.float32]
UNIT = {torch.float16: 2.0**-11, torch.bfloat16: 2.0**-8, torch.float32: 0.0}


def _case(seed):
    r = random.Random(seed)
    hq, hkv, d = r.choice(GEOMETRIES)
    return r, dict(hq=hq, hkv=hkv, d=d, dtype=r.choice(DTYPES), batch=r.randint(1, 4),
                   total=r.choice([1, 15, 16, 17, r.randint(2, 300), r.randint(300, 3000)]),
                   group=r.choice([16, 64, 100, 512, 1024]), two_pass=r.random() < 0.5,
                   tpb=r.choice([16, 32]), scale=r.choice([None, 0.05, 0.2]), softcap=r.choice([None, None, 30.0]))


@pytest.mark.parametrize("seed", range(40))
def test_random_operator_sequence_matches_the_oracle(seed):
    r, c = _case(seed)
    print(f"operator case {seed}: {c}", flush=True)
    B, hq, hkv, d, dt, total = c["batch"], c["hq"], c["hkv"], c["d"], c["dtype"], c["total"]
    g = torch.Generator().manual_seed(500 + seed)
    q = (torch.randn(B, hq, d, generator=g) * 0.5).to(dt)
    k = (torch.randn(B, hkv, total, d, generator=g) * 0.5).to(dt)
    v = (torch.randn(B, hkv, total, d, generator=g) * 0.5).to(dt)
    valid = (torch.rand(B, total, generator=g) > r.choice([0.0, 0.2, 0.6])).to(torch.int32)
    for b in range(B):
        valid[b, : r.randint(0, total // 2)] = 0  # left padding
        valid[b, r.randrange(total)] = 1  # every row has a valid position
    active = torch.ones(B, dtype=torch.int32)
    if B > 1:
        active[r.randrange(B)] = 0
    qd, kd, vd, vald, actd = q.cuda(), k.cuda(), v.cuda(), valid.cuda(), active.cuda()
    kw = dict(scale=c["scale"], softcap=c["softcap"])
    group, tpb = c["group"], c["tpb"]
    m, l, acc = streaming_attention_state_init(B, hq, d, torch.device("cuda"))
    # A state from an earlier call for the inactive rows: it must survive bit for bit.
    m0 = torch.randn(B, hq, generator=g)
    l0 = torch.rand(B, hq, generator=g) + 0.5
    a0 = torch.randn(B, hq, d, generator=g)
    for b in range(B):
        if not active[b]:
            m[b], l[b], acc[b] = m0[b].cuda(), l0[b].cuda(), a0[b].cuda()
    nbl = total // tpb
    mass = torch.zeros(B, hq, max(nbl, 1), dtype=torch.float32, device="cuda")
    if not c["two_pass"]:
        for s in range(0, total, group):
            e = min(s + group, total)
            streaming_attention_step(qd, kd[:, :, s:e], vd[:, :, s:e], m, l, acc, valid=vald[:, s:e], active=actd,
                                     **kw)
    else:
        full = nbl * tpb
        group = max(tpb, group // tpb * tpb)  # accumulate groups start on block boundaries
        for s in range(0, full, group):
            e = min(s + group, full)
            streaming_attention_stats_step(qd, kd[:, :, s:e], m, l, valid=vald[:, s:e], active=actd, **kw)
        if total > full:
            streaming_attention_stats_step(qd, kd[:, :, full:], m, l, valid=vald[:, full:], active=actd, **kw)
        for s in range(0, full, group):
            e = min(s + group, full)
            streaming_attention_accumulate_step(qd, kd[:, :, s:e], vd[:, :, s:e], m, l, acc, mass, s // tpb, tpb,
                                                valid=vald[:, s:e], active=actd, **kw)
        if total > full:
            # fold_fixed has no `active`: the tail of an inactive row is folded only for active rows here.
            rows = [b for b in range(B) if active[b]]
            sub = [t[rows] for t in (m, l, acc)]
            streaming_attention_fold_fixed_step(qd[rows], kd[rows][:, :, full:], vd[rows][:, :, full:], *sub,
                                                valid=vald[rows][:, full:], **kw)
            acc[rows] = sub[2]
    torch.cuda.synchronize()
    for b in range(B):
        if not active[b]:
            assert torch.equal(m[b].cpu(), m0[b]) and torch.equal(l[b].cpu(), l0[b])
            assert torch.equal(acc[b].cpu(), a0[b])
    out_dtype = dt if dt != torch.float32 else torch.float32
    out = streaming_attention_finalize(acc, l, out_dtype).float().cpu().numpy()
    ref, rmass = oa.dense_reference(q.float().numpy(), k.float().numpy(), v.float().numpy(), n_rep=hq // hkv,
                                    tokens_per_block=tpb, valid=valid.numpy(), scale=c["scale"],
                                    softcap=c["softcap"])
    u = UNIT[dt]
    tol = 2e-3 if dt != torch.float32 else 1e-4
    for b in range(B):
        if not active[b]:
            continue
        vmax = float(np.abs(v[b].float().numpy()).max())
        excess = np.abs(out[b] - ref[b]) - u * (np.abs(ref[b]) + vmax)
        assert excess.max() < tol, f"row {b}: error {excess.max():.3g} beyond the dtype's roundings"
        if c["two_pass"] and nbl:
            err = np.abs(mass[b].cpu().numpy()[:, :nbl] - rmass[b][:, :nbl]).max()
            assert err < 1e-4, f"row {b}: block mass error {err:.3g}"
