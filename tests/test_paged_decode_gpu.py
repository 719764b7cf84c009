"""Fused paged decode (pager_hf.PagedDecoder over libpgr.so) against the CPU oracle.

Per step: attention output within max-abs 2e-3 of the fp32 oracle, and bit-exact
integer results: the gather index lists (host-resident in-scope block ids per sequence),
the apply_tiers move lists and the new-block ids. Geometries are the measured
configurations: Qwen2.5-0.5B layer (14q/2kv, D 64, fp16, 32-token blocks) at 4096 context
with 8 resident blocks, the same at batch 8 with contexts drawn in [1024, 32768] and 64
resident blocks over 128 steps, and a Mistral-7B layer (32q/8kv, D 128, bf16) at 131072
context with a 4096-token window, 32 HBM + 96 host blocks in the window.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.paged_decode import PagedDecodeOracle
from oracle.pager_policy import selection_margin
from pager_hf import PagedDecoder

pytestmark = pytest.mark.gpu

MIB16 = 16 * 1024 * 1024
TOL = 2e-3


def np32(t):
    return t.detach().float().cpu().numpy()


class Pair:
    """A PagedDecoder and the oracle driven with the same inputs."""

    def __init__(self, *, layers, hq, hkv, d, tpb, dtype, pool_blocks, host_blocks, staging_blocks=1024,
                 staging_buffers=2, blocks_per_workgroup=32, stream_mode="direct", scale=None, softcap=None):
        self.dtype = dtype
        self.dec = PagedDecoder(num_layers=layers, num_query_heads=hq, num_kv_heads=hkv, head_dim=d,
                                tokens_per_block=tpb, dtype=dtype, device="cuda", pool_blocks=pool_blocks,
                                host_blocks=host_blocks, staging_blocks=staging_blocks,
                                staging_buffers=staging_buffers, blocks_per_workgroup=blocks_per_workgroup, stream_mode=stream_mode, scale=scale,
                                softcap=softcap)
        self.ora = PagedDecodeOracle(num_layers=layers, num_query_heads=hq, num_kv_heads=hkv, head_dim=d,
                                     tokens_per_block=tpb, scale=scale, softcap=softcap)
        self.layers, self.hq, self.hkv, self.d, self.tpb = layers, hq, hkv, d, tpb
        self.sids = []
        self.margins = []  # (selection gap, score error) per scored session-step

    def add(self, *, ctx, rows=1, capacity, gen, scale=0.5, zero_before=0, **pager_kw):
        sid = self.dec.add_session(capacity_tokens=capacity, rows=rows, **pager_kw)
        self.ora.add_session(sid, rows=rows, **pager_kw)
        keys, values = [], []
        for _ in range(self.layers):
            # Positions before `zero_before` are never in scope; they hold zeros.
            k = torch.zeros(rows, self.hkv, ctx, self.d, dtype=self.dtype)
            v = torch.zeros(rows, self.hkv, ctx, self.d, dtype=self.dtype)
            n = ctx - zero_before
            k[:, :, zero_before:] = (torch.randn(rows, self.hkv, n, self.d, generator=gen) * scale).to(self.dtype)
            v[:, :, zero_before:] = (torch.randn(rows, self.hkv, n, self.d, generator=gen) * scale).to(self.dtype)
            keys.append(k)
            values.append(v)
        moves = self.dec.prefill(sid, [k.cuda() for k in keys], [v.cuda() for v in values], ctx)
        omoves = self.ora.prefill(sid, [np32(k) for k in keys], [np32(v) for v in values], ctx)
        assert (moves["to_gpu"], moves["to_cpu"]) == tuple(omoves)
        self.sids.append(sid)
        return sid

    def set_lo(self, sid, lo):
        self.dec.set_lo(sid, lo)
        self.ora.set_lo(sid, lo)

    def step(self, gen, *, compute=True, scale=0.5, sids=None, order=None, end_stream=None, graphs=None,
             windows=None, settle=False, rounding_allowance=False):
        """One decode step of `sids` (every session by default), checked against the oracle.
        With `graphs` (a dict) the layers run from a captured HIP graph, one per launch
        signature: captured when the signature is new, replayed otherwise. windows[layer]:
        that layer's own sliding window (None: none). settle: wait for the store's side-stream
        work after begin_step (in the mirror mode every layer then reads its mirror).
        rounding_allowance: the error is measured beyond two roundings of the model dtype that
        the reference's own kernel makes as well: P rounded before P.V (streaming_attention.py:178;
        at most u sum_i p_i |v_i| / l <= u max|v|) and the output rounded by the finalize
        (at most u |ref|), with unit roundoff u = 2^-11 (fp16) or 2^-8 (bf16). With few tokens
        in scope they exceed 2e-3 in bf16 (at |v| = 1 up to 3.9e-3 each)."""
        win = windows if windows is not None else [None] * self.layers
        sids = self.sids if sids is None else sids
        order = list(range(self.layers)) if order is None else order
        S = sum(self.dec.sessions[s].rows for s in sids)
        qs, ks, vs = [], [], []
        for _ in range(self.layers):
            qs.append((torch.randn(S, self.hq, self.d, generator=gen) * scale).to(self.dtype))
            ks.append((torch.randn(S, self.hkv, self.d, generator=gen) * scale).to(self.dtype))
            vs.append((torch.randn(S, self.hkv, self.d, generator=gen) * scale).to(self.dtype))
        self.dec.begin_step(sids)
        if settle:
            self.dec.pool.sync()
        if graphs is None:
            outs = [None] * self.layers
            for l in order:
                outs[l] = self.dec.decode_layer(l, qs[l].cuda(), ks[l].cuda(), vs[l].cuda(), window=win[l])
        else:
            mass = self.dec._mass
            sig = (self.dec.pool.step_signature(), None if mass is None else mass.data_ptr(), S)
            entry = graphs.get(sig)
            if entry is None:
                ins = [[x.cuda() for x in xs] for xs in (qs, ks, vs)]
                outs = [None] * self.layers
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    for l in order:
                        outs[l] = self.dec.decode_layer(l, ins[0][l], ins[1][l], ins[2][l], window=win[l])
                entry = graphs[sig] = (graph, ins, outs)
            else:
                for dst, src in zip(entry[1], (qs, ks, vs)):
                    for d_, s_ in zip(dst, src):
                        d_.copy_(s_)
            entry[0].replay()
            self.dec.pool.step_replayed()
            outs = entry[2]
        gather = [self.dec.step_host_blocks(i) for i in range(S)]
        if end_stream is None:
            res = self.dec.end_step()
        else:  # placement copies queued on another stream than the step's launches
            with torch.cuda.stream(end_stream):
                res = self.dec.end_step()
        ref = self.ora.step(sids, [np32(x) for x in qs], [np32(x) for x in ks], [np32(x) for x in vs],
                            compute=compute, windows=windows)
        assert gather == ref["gather"], "gather index lists differ"
        for sid in sids:
            got, want = res[sid], ref["placement"][sid]
            assert got["added_block_ids"] == want["added"]
            assert (got["to_gpu"], got["to_cpu"]) == (want["to_gpu"], want["to_cpu"])
            if self.dec.sessions[sid].needs_attention and want["scores"]:
                # Placement margin: the oracle's score gap at its selection boundary against the
                # HIP-vs-oracle score error; identical placement is only meaningful with a margin.
                err = float(np.abs(np.array(got["block_attention"]) - np.array(want["scores"])).max())
                gap = selection_margin(self.ora.sessions[sid].pager)["gap"]
                if gap is not None:
                    self.margins.append((gap, err))
                    if gap <= 10 * err:
                        print(f"placement margin: gap {gap:.3g} within 10x the score error {err:.3g} (session {sid})")
        err = None
        if compute:
            u = {torch.float16: 2.0**-11, torch.bfloat16: 2.0**-8}[self.dtype] if rounding_allowance else 0.0
            seqs = [(sid, r) for sid in sids for r in range(self.dec.sessions[sid].rows)]
            err = 0.0
            for layer, (o, r) in enumerate(zip(outs, ref["out"])):
                excess = np.abs(np32(o) - r)
                if u:
                    vmax = np.array([np.abs(self.ora.sessions[sid].values[layer][row]).max() for sid, row in seqs],
                                    np.float32)
                    excess = excess - u * (np.abs(r) + vmax[:, None, None])
                err = max(err, float(excess.max()))
            assert err < TOL, f"max-abs error {err}" + (" beyond the dtype's roundings" if u else "")
        return res, ref, err


@pytest.mark.parametrize("mode", ["direct", "staged", "mirror"])
def test_config1_single_layer_4096_ctx_8_resident(mode):
    g = torch.Generator().manual_seed(1)
    p = Pair(layers=1, hq=14, hkv=2, d=64, tpb=32, dtype=torch.float16, pool_blocks=32, host_blocks=256,
             stream_mode=mode)
    sid = p.add(ctx=4096, capacity=4096 + 128, gen=g, vram_budget=8 * MIB16, ram_budget=1024 * MIB16,
                recent_window=7, policy="recent_only")
    assert p.dec.pool.block_ids(sid, True) == list(range(120, 128))
    res, ref, err = p.step(g)
    assert ref["gather"] == [list(range(0, 120))]
    st = p.dec.pool.step_stats()
    assert st["host_blocks"] == 120 and st["resident_tokens"] == 8 * 32 + 1
    for _ in range(40):  # crosses a block boundary: block 128 completes, block 120 is evicted
        p.step(g)
    assert p.dec.pool.block_ids(sid, True) == list(range(121, 129))


@pytest.mark.parametrize("mode", ["direct", "staged", "mirror"])
def test_config2_batch8_ragged_contexts_128_steps(mode):
    g = torch.Generator().manual_seed(2)
    ctx = torch.randint(1024, 32769, (8,), generator=g).tolist()
    host_blocks = sum(c // 32 + 8 for c in ctx)
    p = Pair(layers=1, hq=14, hkv=2, d=64, tpb=32, dtype=torch.float16, pool_blocks=8 * 70, host_blocks=host_blocks,
             stream_mode=mode)
    for c in ctx:
        p.add(ctx=c, capacity=c + 160, gen=g, vram_budget=64 * MIB16, ram_budget=4096 * MIB16, recent_window=63,
              policy="recent_only")
    check_at = {0, 1, 31, 32, 63, 64, 100, 127}
    errs = []
    for step in range(128):
        _, _, err = p.step(g, compute=step in check_at)
        if err is not None:
            errs.append(err)
    assert len(errs) == len(check_at)
    for sid, c in zip(p.sids, ctx):
        n_full = (c + 128) // 32
        assert p.dec.pool.block_ids(sid, True) == list(range(n_full - 64, n_full))


@pytest.mark.parametrize("mode,staging_blocks", [("direct", 96), ("staged", 96), ("staged", 4096)])
def test_config4_mistral_layer_window_bf16(mode, staging_blocks):
    """131072 tokens, window 4096: valid iff position > current - 4096 (paged_model.py:981)."""
    g = torch.Generator().manual_seed(4)
    ctx, window = 131072, 4096
    p = Pair(layers=1, hq=32, hkv=8, d=128, tpb=32, dtype=torch.bfloat16, pool_blocks=4 * 40,
             host_blocks=4 * (ctx // 32 + 8), staging_blocks=staging_blocks, stream_mode=mode)
    for _ in range(4):
        p.add(ctx=ctx, capacity=ctx + 64, gen=g, zero_before=ctx - 2 * window, vram_budget=32 * MIB16,
              ram_budget=8192 * MIB16, recent_window=31, policy="recent_only")
    for step in range(3):
        pos = ctx + step  # position of the token this step appends
        for sid in p.sids:
            p.set_lo(sid, [pos - window + 1])
        p.step(g)
        if step == 0:
            st = p.dec.pool.step_stats()
            assert st["host_blocks"] == 4 * 96  # in-window host blocks only
    assert p.ora.host_ids(p.sids[0], 0)[0] == (ctx + 3 - window) // 32


@pytest.mark.parametrize("mode,staging_blocks,staging_buffers,policy", [
    ("staged", 2048, 2, "recent_only"), ("staged", 2048, 3, "sinks_heavy_hitter"), ("staged", 40, 2, "recent_only"),
    ("staged", 40, 3, "heavy_hitter"), ("direct", 2048, 2, "sinks_heavy_hitter"),
    ("mirror", 2048, 2, "sinks_heavy_hitter"), ("mirror", 2048, 2, "recent_only")])
def test_steps_replayed_from_captured_graphs(mode, staging_blocks, staging_buffers, policy):
    """Four layers per step captured into HIP graphs (one per launch signature; new blocks
    change it) and replayed, with eager steps in between. In the staged mode the graph holds
    the staging copies on the store's copy stream: each layer's copies under the layer before
    it when one buffer holds a layer's host blocks, chunk by chunk otherwise. Outputs, gather
    lists, block mass and placement match the oracle at every step."""
    g = torch.Generator().manual_seed(12)
    ctx = [1200, 2500, 700]
    p = Pair(layers=4, hq=8, hkv=2, d=64, tpb=32, dtype=torch.float16, pool_blocks=3 * 16,
             host_blocks=sum(c // 32 + 8 for c in ctx), staging_blocks=staging_blocks,
             staging_buffers=staging_buffers, stream_mode=mode)
    for c in ctx:
        p.add(ctx=c, capacity=c + 96, gen=g, vram_budget=10 * MIB16, ram_budget=1024 * MIB16, recent_window=7,
              policy=policy)
    graphs, errs = {}, []
    scored = policy != "recent_only"  # the oracle computes every step to score the blocks
    for step in range(72):
        eager = step % 24 == 23  # an eager step now and then: the graphs must stay valid around it
        _, _, err = p.step(g, compute=scored or step % 6 == 0 or step >= 69, graphs=None if eager else graphs)
        if err is not None:
            errs.append(err)
        st = p.dec.pool.step_stats()
        assert st["host_blocks"] > 100
        if mode == "staged":
            assert (st["chunks"] == 1) if staging_blocks >= 2048 else (st["chunks"] > 1)
    assert len(errs) == (72 if scored else 15) and len(graphs) >= 2
    print(f"{mode}/{staging_blocks}/{staging_buffers}/{policy}: {len(graphs)} graphs, max err {max(errs):.3g}")


@pytest.mark.parametrize("staging_blocks,staging_buffers,order", [
    (2048, 2, None), (2048, 3, None), (40, 2, None), (2048, 2, [2, 0, 3, 1]), (2048, 3, [3, 1, 0, 2])])
def test_staged_layers_prefetch_and_chunks(staging_blocks, staging_buffers, order):
    """Staged mode over four layers. With a step's host blocks in one chunk, each layer's
    copies are queued right after the previous layer's attention, into the next buffer (two
    and three buffers). With a small staging buffer the step falls back to several chunks per
    layer, copied layer by layer. Layers decoded out of order abandon the queued copies and
    reuse buffers; the results must not change. Outputs, gather lists and placement match
    the oracle."""
    g = torch.Generator().manual_seed(11)
    ctx = [1200, 2500, 700]
    p = Pair(layers=4, hq=8, hkv=2, d=64, tpb=32, dtype=torch.float16, pool_blocks=3 * 12,
             host_blocks=sum(c // 32 + 8 for c in ctx), staging_blocks=staging_blocks,
             staging_buffers=staging_buffers, stream_mode="staged")
    for c in ctx:
        p.add(ctx=c, capacity=c + 64, gen=g, vram_budget=8 * MIB16, ram_budget=1024 * MIB16, recent_window=7,
              policy="recent_only")
    errs = []
    for step in range(40):
        _, _, err = p.step(g, compute=step % 8 == 0 or step >= 37, order=order)
        if err is not None:
            errs.append(err)
        st = p.dec.pool.step_stats()
        assert st["host_blocks"] > 100
        assert (st["chunks"] == 1) if staging_blocks >= 2048 else (st["chunks"] > 1)
    assert len(errs) == 8


@pytest.mark.parametrize("mode,layers", [("direct", 1), ("direct", 2), ("staged", 2), ("mirror", 1), ("mirror", 3)])
def test_sessions_join_and_leave_between_steps(mode, layers):
    """Sessions join (the step plan grows) and leave (their ids are reused by later
    sessions) between steps. A single-layer decoder alternates between two pinned plan
    buffers, a two-layer one keeps one. In the mirror mode the host ranges that leaving
    sessions free are handed to joining ones, so a ring buffer's records change between steps
    and within one (three layers, two buffers). Every step matches the oracle."""
    g = torch.Generator().manual_seed(31)
    p = Pair(layers=layers, hq=8, hkv=2, d=64, tpb=16, dtype=torch.float16, pool_blocks=400, host_blocks=3000,
             staging_blocks=1024, stream_mode=mode)
    live = []

    def join():
        c = int(torch.randint(50, 1500, (1,), generator=g))
        live.append(p.add(ctx=c, capacity=c + 64, gen=g, vram_budget=6 * MIB16, ram_budget=1024 * MIB16,
                          recent_window=3, policy="recent_only"))

    for _ in range(3):
        join()
    reused = False
    for step in range(24):
        if step % 4 == 1:
            join()
            reused = reused or live[-1] < max(live[:-1])
        if step % 6 == 5 and len(live) > 2:
            sid = live.pop(0)
            p.dec.remove_session(sid)
            del p.ora.sessions[sid]
            p.sids.remove(sid)
        p.step(g, sids=list(live))
    assert reused  # a freed session id was handed out again


@pytest.mark.parametrize("mode", ["direct", "staged", "mirror"])
def test_tier_moves_on_another_stream(mode):
    """end_step (and with it the eviction copies) runs on a side stream on alternate steps,
    while begin_step and the attention launches run on the default stream. The evictions run
    on the stream they were issued on; the next step's launches must still wait for them
    before reading the evicted blocks from the host mirror or reusing their slots."""
    g = torch.Generator().manual_seed(51)
    ctx = [700, 1300, 2100, 410, 990]
    p = Pair(layers=2, hq=8, hkv=2, d=64, tpb=16, dtype=torch.float16, pool_blocks=5 * 12,
             host_blocks=sum(c // 16 + 8 for c in ctx), staging_blocks=1024, stream_mode=mode)
    for c in ctx:
        p.add(ctx=c, capacity=c + 64, gen=g, vram_budget=6 * MIB16, ram_budget=1024 * MIB16, recent_window=3,
              policy="recent_only")
    side = torch.cuda.Stream()
    evicted = 0
    for step in range(40):
        res, _, _ = p.step(g, end_stream=side if step % 2 else None)
        evicted += sum(len(r["to_cpu"]) for r in res.values())
    assert evicted >= 8  # blocks complete and leave HBM on many steps


@pytest.mark.parametrize("mode", ["direct", "staged", "mirror"])
def test_scoring_placement_on_another_stream(mode):
    """A scoring policy with no recent window, placement on a side stream every other step:
    the mass read-back and the eviction of the block that completed in this very step (its
    last token appended by this step's launch on the default stream) must wait for the
    step's launches."""
    g = torch.Generator().manual_seed(52)
    ctx = [3000, 5200, 4100]
    p = Pair(layers=2, hq=8, hkv=2, d=64, tpb=16, dtype=torch.float16, pool_blocks=3 * 16,
             host_blocks=sum(c // 16 + 8 for c in ctx), staging_blocks=1024, stream_mode=mode)
    for c in ctx:
        p.add(ctx=c, capacity=c + 80, gen=g, scale=1.0, vram_budget=12 * MIB16, ram_budget=1024 * MIB16,
              recent_window=0, rebalance_interval=4, policy="sinks_heavy_hitter")
    side = torch.cuda.Stream()
    evicted = 0
    for step in range(40):
        res, _, _ = p.step(g, scale=1.0, end_stream=side if step % 2 else None)
        evicted += sum(len(r["to_cpu"]) for r in res.values())
    assert evicted >= 3


@pytest.mark.parametrize("mode,layers", [("direct", 1), ("direct", 2), ("staged", 1), ("mirror", 3)])
def test_back_to_back_steps_without_host_sync(mode, layers):
    """Steps issued back to back with no host synchronisation, as a serving loop issues them.
    Each step reads ~45 MB of host blocks per layer, so the host plans the next steps while
    the GPU still runs this one: only the plan buffers' reuse guard (the merge's flag word in
    direct mode, an event in staged mode) keeps every launch on its own step's plan. Every
    step's output is checked against the oracle afterwards."""
    g = torch.Generator().manual_seed(41)
    ctx = [30000, 21000, 12500, 25000]
    S, hq, hkv, d, n = len(ctx), 14, 2, 64, 40
    p = Pair(layers=layers, hq=hq, hkv=hkv, d=d, tpb=32, dtype=torch.float16, pool_blocks=S * 40,
             host_blocks=sum(c // 32 + 8 for c in ctx), staging_blocks=4096, stream_mode=mode)
    for c in ctx:
        p.add(ctx=c, capacity=c + n + 32, gen=g, vram_budget=32 * MIB16, ram_budget=4096 * MIB16,
              recent_window=31, policy="recent_only")
    qs = [[(torch.randn(S, hq, d, generator=g) * 0.5).half() for _ in range(layers)] for _ in range(n)]
    ks = [[(torch.randn(S, hkv, d, generator=g) * 0.5).half() for _ in range(layers)] for _ in range(n)]
    vs = [[(torch.randn(S, hkv, d, generator=g) * 0.5).half() for _ in range(layers)] for _ in range(n)]
    qd = [[x.cuda() for x in step] for step in qs]
    kd = [[x.cuda() for x in step] for step in ks]
    vd = [[x.cuda() for x in step] for step in vs]
    outs = torch.empty(n, layers, S, hq, d, dtype=torch.float16, device="cuda")
    torch.cuda.synchronize()
    for i in range(n):
        p.dec.begin_step(p.sids)
        for l in range(layers):
            p.dec.decode_layer(l, qd[i][l], kd[i][l], vd[i][l], outs[i, l])
        p.dec.end_step(collect=False)
    torch.cuda.synchronize()
    for i in range(n):
        ref = p.ora.step(p.sids, [np32(x) for x in qs[i]], [np32(x) for x in ks[i]], [np32(x) for x in vs[i]])
        err = max(np.abs(np32(outs[i, l]) - ref["out"][l]).max() for l in range(layers))
        assert err < TOL, f"step {i}: max-abs error {err}"


@pytest.mark.parametrize("mode", ["direct", "staged", "mirror"])
def test_work_items_of_many_blocks(mode):
    """Work items of more than 16 blocks: 16-token blocks, batch 12 at 7k-14k tokens (about
    8,000 in-scope blocks for one round of work items, 3 workgroups per CU), so a wave folds
    five or six blocks and reads their entries one block ahead. The planner sizes items in
    whole rounds. A scoring policy checks the per-block mass as well."""
    g = torch.Generator().manual_seed(21)
    ctx = torch.randint(7000, 14001, (12,), generator=g).tolist()
    p = Pair(layers=1, hq=8, hkv=2, d=64, tpb=16, dtype=torch.bfloat16, pool_blocks=12 * 40,
             host_blocks=sum(c // 16 + 16 for c in ctx), staging_blocks=8192, stream_mode=mode)
    for c in ctx:
        p.add(ctx=c, capacity=c + 64, gen=g, vram_budget=32 * MIB16, ram_budget=4096 * MIB16, recent_window=8,
              rebalance_interval=4, policy="sinks_heavy_hitter")
    per_round = 3 * torch.cuda.get_device_properties(0).multi_processor_count // 2  # workgroups / Hkv
    for step in range(6):
        res, ref, err = p.step(g)
        st = p.dec.pool.step_stats()
        assert st["work_items"] % per_round == 0
        assert st["host_blocks"] + st["resident_tokens"] // 16 > 16 * st["work_items"]  # > 16 blocks per item
        for sid in p.sids:
            got = np.array(res[sid]["block_attention"])
            want = np.array(ref["placement"][sid]["scores"])
            assert np.abs(got - want).max() < 2e-5


@pytest.mark.parametrize("mode", ["direct", "staged", "mirror"])
def test_scoring_policy_mass_drives_placement(mode):
    """sinks_heavy_hitter over two layers: the per-block mass handed to the pager matches the
    oracle's within float tolerance and, where score gaps are clear, placement is identical."""
    g = torch.Generator().manual_seed(5)
    p = Pair(layers=2, hq=32, hkv=4, d=64, tpb=32, dtype=torch.float16, pool_blocks=64, host_blocks=256,
             stream_mode=mode)
    sid = p.add(ctx=1500, capacity=1500 + 128, gen=g, scale=1.0, vram_budget=12 * MIB16, ram_budget=512 * MIB16,
                recent_window=4, rebalance_interval=4, policy="sinks_heavy_hitter")
    for _ in range(40):
        res, ref, _ = p.step(g, scale=1.0)
        got = np.array(res[sid]["block_attention"])
        want = np.array(ref["placement"][sid]["scores"])
        assert got.shape == want.shape
        assert np.abs(got - want).max() < 2e-5
        assert abs(got.sum() - 1.0) < 1e-5
    gaps = [g for g, _ in p.margins]
    errs = [e for _, e in p.margins]
    print(f"placement margin over {len(gaps)} steps: smallest gap {min(gaps):.3g}, largest score error "
          f"{max(errs):.3g}, steps within 10x: {sum(g <= 10 * e for g, e in p.margins)}")


def test_multi_row_session_with_left_padding():
    g = torch.Generator().manual_seed(6)
    p = Pair(layers=2, hq=14, hkv=2, d=64, tpb=32, dtype=torch.float16, pool_blocks=64, host_blocks=256)
    sid = p.add(ctx=700, rows=2, capacity=800, gen=g, vram_budget=6 * MIB16, ram_budget=512 * MIB16,
                recent_window=5, policy="sinks_recent", lo=[0, 133])
    for _ in range(10):
        p.step(g)
    p.step(g)
    assert p.ora.host_ids(sid, 1)[0] >= 133 // 32


def test_short_prompt_below_one_block():
    """A prompt shorter than one block: no full blocks, no placement, the open block only."""
    g = torch.Generator().manual_seed(7)
    p = Pair(layers=1, hq=14, hkv=2, d=64, tpb=32, dtype=torch.float16, pool_blocks=16, host_blocks=64)
    sid = p.add(ctx=5, capacity=200, gen=g, vram_budget=2 * MIB16, ram_budget=64 * MIB16, recent_window=1,
                policy="recent_only")
    for _ in range(60):
        p.step(g)
    assert p.dec.num_tokens(sid) == 65 and p.dec.num_blocks(sid) == 2


def test_first_token_of_an_empty_session():
    """No stored tokens: the step attends to the current token alone (output = v_new)."""
    g = torch.Generator().manual_seed(8)
    p = Pair(layers=1, hq=14, hkv=2, d=64, tpb=32, dtype=torch.float16, pool_blocks=16, host_blocks=64)
    sid = p.add(ctx=0, capacity=200, gen=g, vram_budget=2 * MIB16, ram_budget=64 * MIB16, recent_window=1,
                policy="recent_only")
    for _ in range(40):
        p.step(g)
    assert p.dec.num_tokens(sid) == 40 and p.dec.num_blocks(sid) == 1


# Geometry grid: head dims 32/64/128, n_rep 1/7/16, 16/32/64-token blocks (1, 2 and 4 tiles
# per block), both dtypes, a non-default scale and a softcap, and a scoring policy so the
# per-block mass is checked as well. Each case crosses a block boundary.
GRID = [
    # hq, hkv, d, tpb, dtype, scale, softcap, policy, mode
    (4, 4, 32, 16, torch.float16, None, None, "sinks_heavy_hitter", "direct"),
    (14, 2, 64, 64, torch.bfloat16, None, None, "heavy_hitter", "direct"),
    (32, 2, 128, 32, torch.bfloat16, 0.07, 30.0, "sinks_heavy_hitter", "staged"),
    (16, 1, 64, 16, torch.float16, None, 50.0, "recent_only", "staged"),
    (8, 8, 128, 64, torch.float16, None, None, "sinks_recent", "direct"),
    # Head dims 16 and 256 (Gemma / Gemma2 geometries: 8q/1kv and 16q/8kv at 256, with
    # Gemma2's query_pre_attn_scalar scale and attn-logit softcap).
    (4, 2, 16, 16, torch.float16, 16**-0.5, 50.0, "sinks_heavy_hitter", "direct"),
    (8, 4, 16, 32, torch.bfloat16, None, None, "heavy_hitter", "staged"),
    (8, 1, 256, 16, torch.bfloat16, None, None, "sinks_heavy_hitter", "direct"),
    (16, 8, 256, 32, torch.float16, 256**-0.5, 50.0, "recent_only", "staged"),
    (14, 2, 64, 32, torch.bfloat16, None, 30.0, "sinks_heavy_hitter", "mirror"),
    (8, 1, 256, 16, torch.float16, None, None, "heavy_hitter", "mirror"),
]


@pytest.mark.parametrize("policy", ["recent_only", "sinks_heavy_hitter"])
def test_mirror_mode_with_and_without_landed_copies(policy):
    """Mirror mode over four layers: on settled steps the side stream's copies have landed
    before the launches (every layer reads its HBM mirror), on the others the launches race
    them (a layer reads the mirror or the host in place, whichever its word says). Outputs,
    gather lists, scores and placement match the oracle on both, with blocks evicted to the
    host and re-read through the mirror on later steps."""
    g = torch.Generator().manual_seed(61)
    ctx = [1500, 2600, 800]
    p = Pair(layers=4, hq=8, hkv=2, d=64, tpb=32, dtype=torch.float16, pool_blocks=3 * 16,
             host_blocks=sum(c // 32 + 8 for c in ctx), stream_mode="mirror")
    for c in ctx:
        p.add(ctx=c, capacity=c + 96, gen=g, vram_budget=10 * MIB16, ram_budget=1024 * MIB16, recent_window=3,
              rebalance_interval=2, policy=policy)
    scored = policy != "recent_only"
    errs = []
    for step in range(72):
        _, _, err = p.step(g, compute=scored or step % 5 == 0, settle=step % 3 == 0)
        if err is not None:
            errs.append(err)
        assert p.dec.pool.step_stats()["host_blocks"] > 100
    assert max(errs) < TOL
    assert p.dec.pool.stats()["stream_bytes"] > 0


def test_mirror_store_destroyed_while_its_copies_are_queued():
    """Mirror mode: a store's host thread queues each step's copies after begin_step returns.
    Stores destroyed right after begin_step (the step left open, its copies possibly still
    being queued) and right after decode_layer release cleanly, and every store that follows
    in the process steps in agreement with the oracle."""
    g = torch.Generator().manual_seed(67)
    for rnd in range(4):
        p = Pair(layers=3, hq=8, hkv=2, d=64, tpb=32, dtype=torch.float16, pool_blocks=32, host_blocks=160,
                 stream_mode="mirror")
        p.add(ctx=2900 + 37 * rnd, capacity=3100, gen=g, vram_budget=4 * MIB16, ram_budget=1024 * MIB16,
              recent_window=2, policy="recent_only")
        for step in range(4):
            p.step(g, settle=step == 1)
        assert p.dec.pool.step_stats()["host_blocks"] > 70
        p.dec.begin_step(p.sids)
        if rnd % 2:
            q = (torch.randn(1, 8, 64, generator=g) * 0.5).half().cuda()
            kv = (torch.randn(1, 2, 64, generator=g) * 0.5).half().cuda()
            p.dec.decode_layer(0, q, kv, kv)
        p.dec.pool.close()
    torch.cuda.synchronize()


def test_mirror_ring_layers_out_of_order_and_left_out():
    """Mirror mode over four layers and a ring of two buffers: a layer's copies go into its
    buffer once the layer two below it has released it. Layers decoded out of order wait
    their bounded wait for copies that cannot come yet and read the host in place; every
    output still matches the oracle. A last step decodes two of the four layers only: the
    store's copy thread gives up on the releases that never come, the store closes, and a new
    store steps normally."""
    g = torch.Generator().manual_seed(71)
    ctx = [1500, 2600]
    p = Pair(layers=4, hq=8, hkv=2, d=64, tpb=32, dtype=torch.float16, pool_blocks=2 * 16,
             host_blocks=sum(c // 32 + 8 for c in ctx), staging_buffers=2, stream_mode="mirror")
    for c in ctx:
        p.add(ctx=c, capacity=c + 64, gen=g, vram_budget=6 * MIB16, ram_budget=1024 * MIB16, recent_window=3,
              policy="recent_only")
    for step in range(6):
        _, _, err = p.step(g, order=[2, 0, 3, 1] if step % 2 == 0 else None)
        assert err < TOL
    assert p.dec.pool.hbm_bytes()["mirror"] > 0
    S = len(ctx)
    p.dec.begin_step(p.sids)
    for layer in (2, 3):
        q = (torch.randn(S, 8, 64, generator=g) * 0.5).half().cuda()
        kv = (torch.randn(S, 2, 64, generator=g) * 0.5).half().cuda()
        p.dec.decode_layer(layer, q, kv, kv)
    p.dec.end_step(collect=False)
    p.dec.pool.close()
    torch.cuda.synchronize()
    q = Pair(layers=2, hq=8, hkv=2, d=64, tpb=32, dtype=torch.float16, pool_blocks=16, host_blocks=160,
             stream_mode="mirror")
    q.add(ctx=1000, capacity=1100, gen=g, vram_budget=4 * MIB16, ram_budget=1024 * MIB16, recent_window=2,
          policy="recent_only")
    for _ in range(3):
        _, _, err = q.step(g)
        assert err < TOL


@pytest.mark.parametrize("mode", ["direct", "staged", "mirror"])
@pytest.mark.parametrize("d,tpb,window", [(16, 16, 24), (64, 32, 100), (256, 16, 40)])
def test_per_layer_sliding_windows(d, tpb, window, mode):
    """Layers alternating between a sliding window and global attention (Gemma2): the windowed
    layers mask the stored positions <= current - window in the kernel while the global ones
    read everything, over steps that move the window across block boundaries, with a padded
    row. Outputs, block mass (scores), gather lists and placement against the oracle."""
    g = torch.Generator().manual_seed(d + window)
    p = Pair(layers=4, hq=8, hkv=4, d=d, tpb=tpb, dtype=torch.bfloat16, pool_blocks=64, host_blocks=160,
             stream_mode=mode, scale=d**-0.5, softcap=50.0, staging_blocks=128)
    ctx = 14 * tpb + 7
    sid = p.add(ctx=ctx, rows=2, capacity=ctx + 3 * tpb, gen=g, vram_budget=8 * MIB16, ram_budget=512 * MIB16,
                recent_window=1, rebalance_interval=2, policy="sinks_heavy_hitter", lo=[0, 9])
    windows = [window, None, window, None]
    errs = []
    for _ in range(2 * tpb + 3):
        res, ref, err = p.step(g, windows=windows)
        errs.append(err)
        got = np.array(res[sid]["block_attention"])
        want = np.array(ref["placement"][sid]["scores"])
        assert np.abs(got - want).max() < 2e-5
    assert max(errs) < TOL
    assert p.dec.pool.step_stats()["host_blocks"] > 0


@pytest.mark.parametrize("hq,hkv,d,tpb,dtype,scale,softcap,policy,mode", GRID)
def test_geometry_grid(hq, hkv, d, tpb, dtype, scale, softcap, policy, mode):
    g = torch.Generator().manual_seed(hq * 131 + d + tpb)
    p = Pair(layers=2, hq=hq, hkv=hkv, d=d, tpb=tpb, dtype=dtype, pool_blocks=96, host_blocks=256,
             stream_mode=mode, scale=scale, softcap=softcap, staging_blocks=64)
    ctx = 13 * tpb + 5
    sid = p.add(ctx=ctx, rows=2, capacity=ctx + 3 * tpb, gen=g, vram_budget=5 * MIB16, ram_budget=512 * MIB16,
                recent_window=2, rebalance_interval=2, policy=policy, lo=[0, tpb + 3])
    errs = []
    for _ in range(tpb + 4):  # crosses the next block boundary
        res, ref, err = p.step(g)
        errs.append(err)
    assert max(errs) < TOL
    if policy not in ("recent_only", "sinks_recent"):
        got = np.array(res[sid]["block_attention"])
        want = np.array(ref["placement"][sid]["scores"])
        assert np.abs(got - want).max() < 2e-5
    assert p.dec.pool.step_stats()["host_blocks"] > 0


@pytest.mark.parametrize("mode", ["direct", "staged"])
def test_one_long_and_many_short_sessions(mode):
    """One 24k-token session beside 30 sessions of a few dozen tokens: the long one gets
    hundreds of work items and the short ones one each, so fixed per-sequence ranges of
    split-K partial slots would take more than twice the slots the step writes, and the store
    packs them instead (the merge then reads where each sequence's slots start). Then steps
    of the long session with four of the short ones, where the ranges are fixed again. Every
    step matches the oracle."""
    g = torch.Generator().manual_seed(77)
    p = Pair(layers=1, hq=8, hkv=2, d=64, tpb=32, dtype=torch.float16, pool_blocks=600, host_blocks=1200,
             staging_blocks=1024, stream_mode=mode)
    long_sid = p.add(ctx=24000, capacity=24100, gen=g, vram_budget=8 * MIB16, ram_budget=1024 * MIB16,
                     recent_window=7, policy="recent_only")
    short = [p.add(ctx=int(torch.randint(1, 80, (1,), generator=g)), capacity=200, gen=g, vram_budget=4 * MIB16,
                   ram_budget=1024 * MIB16, recent_window=3, policy="sinks_heavy_hitter") for _ in range(30)]
    for _ in range(3):
        p.step(g)
    for _ in range(3):
        p.step(g, sids=[long_sid] + short[:4])
