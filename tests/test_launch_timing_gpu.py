"""Launch timing of the paged attention kernel, which bench.py's roofline figures are built on:
per-launch events (pgr_kv_set_timing / pgr_kv_kernel_time), counts, bytes and durations over
passes that reuse the store's timing events; back-to-back launches of an open step
(pgr_kv_bench_attention), bytes equal to the per-launch figure; neither changes the decode
results of the step or of the steps after it."""
import numpy as np
import pytest
import torch

from oracle.paged_decode import PagedDecodeOracle
from pager_hf import PagedDecoder

MIB16 = 16 * 1024 * 1024


@pytest.mark.gpu
def test_kernel_time_counts_and_bytes_over_reused_events():
    layers, hq, hkv, d, T = 3, 14, 2, 64, 32
    g = torch.Generator().manual_seed(11)
    dec = PagedDecoder(num_layers=layers, num_query_heads=hq, num_kv_heads=hkv, head_dim=d, tokens_per_block=T,
                       dtype=torch.float16, device="cuda:0", pool_blocks=64, host_blocks=64, staging_blocks=64)
    ora = PagedDecodeOracle(num_layers=layers, num_query_heads=hq, num_kv_heads=hkv, head_dim=d, tokens_per_block=T)
    kw = dict(vram_budget=4 * MIB16, ram_budget=64 * MIB16, recent_window=3, policy="recent_only")
    n = 300
    sid = dec.add_session(capacity_tokens=n + 64, **kw)
    ora.add_session(sid, **kw)
    ks = [(torch.randn(1, hkv, n, d, generator=g) * 0.5).half() for _ in range(layers)]
    vs = [(torch.randn(1, hkv, n, d, generator=g) * 0.5).half() for _ in range(layers)]
    dec.prefill(sid, [k.cuda() for k in ks], [v.cuda() for v in vs], n)
    ora.prefill(sid, [k.float().numpy() for k in ks], [v.float().numpy() for v in vs], n)
    dec.pool.kernel_time()  # clear
    dec.pool.set_timing(True)
    try:
        for rnd in range(3):  # later rounds take their events from the pool the first one filled
            steps = 2 + rnd
            for _ in range(steps):
                q = [(torch.randn(1, hq, d, generator=g) * 0.5).half() for _ in range(layers)]
                kn = [(torch.randn(1, hkv, d, generator=g) * 0.5).half() for _ in range(layers)]
                vn = [(torch.randn(1, hkv, d, generator=g) * 0.5).half() for _ in range(layers)]
                dec.begin_step([sid])
                st = dec.pool.step_stats()
                outs = [dec.decode_layer(l, q[l].cuda(), kn[l].cuda(), vn[l].cuda()).float().cpu().numpy()
                        for l in range(layers)]
                dec.end_step()
                ref = ora.step([sid], [x.float().numpy() for x in q], [x.float().numpy() for x in kn],
                               [x.float().numpy() for x in vn])
                for l in range(layers):
                    assert float(np.abs(outs[l] - ref["out"][l]).max()) < 2e-3
            torch.cuda.synchronize()
            ms, launches, nbytes = dec.pool.kernel_time()
            per_launch = st["launches"]
            assert launches == steps * layers * per_launch, (launches, steps, layers, per_launch)
            # K/V bytes read per launch: every in-scope stored block, whole blocks.
            assert nbytes > 0 and nbytes % (2 * hkv * T * d * 2) == 0
            assert ms > 0.0 and ms / launches < 5.0, ms  # milliseconds per launch: microseconds here
    finally:
        dec.pool.set_timing(False)
        dec.pool.close()


@pytest.mark.gpu
def test_back_to_back_attention_launches_keep_the_decode_intact():
    layers, hq, hkv, d, T = 3, 14, 2, 64, 32
    g = torch.Generator().manual_seed(12)
    dec = PagedDecoder(num_layers=layers, num_query_heads=hq, num_kv_heads=hkv, head_dim=d, tokens_per_block=T,
                       dtype=torch.float16, device="cuda:0", pool_blocks=64, host_blocks=64, staging_blocks=64)
    ora = PagedDecodeOracle(num_layers=layers, num_query_heads=hq, num_kv_heads=hkv, head_dim=d, tokens_per_block=T)
    kw = dict(vram_budget=4 * MIB16, ram_budget=64 * MIB16, recent_window=3, policy="recent_only")
    n = 310  # the open block fills during the steps: appends land in a new block too
    sid = dec.add_session(capacity_tokens=n + 64, **kw)
    ora.add_session(sid, **kw)
    ks = [(torch.randn(1, hkv, n, d, generator=g) * 0.5).half() for _ in range(layers)]
    vs = [(torch.randn(1, hkv, n, d, generator=g) * 0.5).half() for _ in range(layers)]
    dec.prefill(sid, [k.cuda() for k in ks], [v.cuda() for v in vs], n)
    ora.prefill(sid, [k.float().numpy() for k in ks], [v.float().numpy() for v in vs], n)
    try:
        for step in range(14):
            q = [(torch.randn(1, hq, d, generator=g) * 0.5).half() for _ in range(layers)]
            kn = [(torch.randn(1, hkv, d, generator=g) * 0.5).half() for _ in range(layers)]
            vn = [(torch.randn(1, hkv, d, generator=g) * 0.5).half() for _ in range(layers)]
            qd, knd, vnd = [x.cuda() for x in q], [x.cuda() for x in kn], [x.cuda() for x in vn]
            dec.begin_step([sid])
            if step == 0:
                with pytest.raises(RuntimeError):  # the plan is not on the device before a layer runs
                    dec.pool.bench_attention(qd, knd, vnd)
            dec.pool.kernel_time()
            dec.pool.set_timing(True)
            outs = [dec.decode_layer(l, qd[l], knd[l], vnd[l]) for l in range(layers)]
            dec.pool.set_timing(False)
            us, nbytes = dec.pool.bench_attention(qd, knd, vnd, reps=2)
            torch.cuda.synchronize()
            _, launches, per_bytes = dec.pool.kernel_time()
            assert nbytes == per_bytes // launches and nbytes > 0
            assert 0.0 < us < 5000.0
            outs = [o.float().cpu().numpy() for o in outs]
            dec.end_step()
            ref = ora.step([sid], [x.float().numpy() for x in q], [x.float().numpy() for x in kn],
                           [x.float().numpy() for x in vn])
            for l in range(layers):
                assert float(np.abs(outs[l] - ref["out"][l]).max()) < 2e-3, (step, l)
        with pytest.raises(ValueError):
            dec.pool.bench_attention(qd[:1], knd[:1], vnd[:1])
    finally:
        dec.pool.close()


@pytest.mark.gpu
def test_operator_fold_back_to_back_launches():
    """pgr_attn_bench_step: the operator's fold launches over several chunks back to back (no
    merge, no running state); bytes per launch are the chunk's K+V; a workspace too small for
    the chunk's partials is refused."""
    import ctypes

    import _pgr_native as nat

    lib = nat.load()
    b, hq, hkv, tc, d = 1, 28, 4, 1024, 128
    g = torch.Generator().manual_seed(13)
    q = (torch.randn(b, hq, d, generator=g) * 0.5).half().cuda()
    chunks = [((torch.randn(b, hkv, tc, d, generator=g) * 0.5).half().cuda(),
               (torch.randn(b, hkv, tc, d, generator=g) * 0.5).half().cuda()) for _ in range(3)]
    ws_bytes = lib.pgr_attn_workspace_bytes(b, hq, hkv, tc, d, nat.MODE_FOLD, 16)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    karr = (ctypes.c_void_p * 3)(*[kc.data_ptr() for kc, _ in chunks])
    varr = (ctypes.c_void_p * 3)(*[vc.data_ptr() for _, vc in chunks])
    us, nbytes = ctypes.c_double(0), ctypes.c_int64(0)
    stream = torch.cuda.current_stream().cuda_stream
    nat.check(lib.pgr_attn_bench_step(q.data_ptr(), karr, varr, 3, b, hq, hkv, tc, d, nat.DTYPE_F16, d**-0.5,
                                      ws.data_ptr(), ws_bytes, 2, ctypes.byref(us), ctypes.byref(nbytes), stream),
              "bench_step")
    torch.cuda.synchronize()
    assert nbytes.value == 2 * b * hkv * tc * d * 2
    assert 0.0 < us.value < 1000.0
    with pytest.raises(MemoryError):  # a workspace too small for the chunk's partials
        nat.check(lib.pgr_attn_bench_step(q.data_ptr(), karr, varr, 3, b, hq, hkv, tc, d, nat.DTYPE_F16, d**-0.5,
                                          ws.data_ptr(), 16, 1, ctypes.byref(us), ctypes.byref(nbytes), stream),
                  "bench_step")
