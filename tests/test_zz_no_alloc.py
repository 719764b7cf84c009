"""pgr_attn_step_noalloc (split-K partials in the library's static device array) against
pgr_attn_step (partials in a caller workspace), both called through the C ABI.

The two entry points run the same kernels on the same plan, so their (m, l, acc) must be
identical bit for bit. Two calls in a row, the second on a smaller chunk, so the second
runs over whatever the first left in the static array; then a chunk too large for the
array is rejected before anything is launched; then calls on two streams that do not wait
for each other, which the library orders on the GPU.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

import _pgr_native as nat

pytestmark = pytest.mark.gpu

CODES = {torch.float16: nat.DTYPE_F16, torch.bfloat16: nat.DTYPE_BF16, torch.float32: nat.DTYPE_F32}


def _inputs(b, hq, hkv, tc, d, dtype, seed, masked):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(b, hq, d, generator=g) * 0.5).to(dtype).cuda()
    k = (torch.randn(b, hkv, tc, d, generator=g) * 0.5).to(dtype).cuda()
    v = (torch.randn(b, hkv, tc, d, generator=g) * 0.5).to(dtype).cuda()
    # A running state from an earlier chunk: finite m, positive l, nonzero acc.
    m = (torch.randn(b, hq, generator=g) * 0.3).cuda()
    l = (torch.rand(b, hq, generator=g) + 0.5).cuda()
    acc = torch.randn(b, hq, d, generator=g).cuda()
    valid = active = None
    if masked:
        valid = (torch.rand(b, tc, generator=g) > 0.2).to(torch.int32).cuda()
        active = torch.ones(b, dtype=torch.int32)
        active[b // 2] = 0
        active = active.cuda()
    return q, k, v, m, l, acc, valid, active


def _ptr(t):
    return None if t is None else t.data_ptr()


def _run(lib, noalloc, case, seed, masked):
    b, hq, hkv, tc, d, dtype = case
    q, k, v, m, l, acc, valid, active = _inputs(b, hq, hkv, tc, d, dtype, seed, masked)
    stream = torch.cuda.current_stream().cuda_stream
    scale, softcap = 1.0 / d**0.5, 0.0
    if noalloc:
        rc = lib.pgr_attn_step_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), _ptr(valid), _ptr(active),
                                       m.data_ptr(), l.data_ptr(), acc.data_ptr(), b, hq, hkv, tc, d, CODES[dtype],
                                       scale, softcap, stream)
    else:
        nbytes = lib.pgr_attn_workspace_bytes(b, hq, hkv, tc, d, nat.MODE_FOLD, 16)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
        rc = lib.pgr_attn_step(q.data_ptr(), k.data_ptr(), v.data_ptr(), _ptr(valid), _ptr(active), m.data_ptr(),
                               l.data_ptr(), acc.data_ptr(), b, hq, hkv, tc, d, CODES[dtype], scale, softcap,
                               ws.data_ptr(), nbytes, stream)
    assert rc == 0, nat.last_error()
    torch.cuda.synchronize()
    return m.cpu(), l.cpu(), acc.cpu()


# The first call is the larger one; the second runs over what it left in the static array.
CASES = [
    ((8, 14, 2, 6000, 64, torch.float16), 1, True),
    ((2, 32, 8, 700, 128, torch.bfloat16), 2, False),
    # fp32 q/k/v run the generic kernel, whose plan has more, smaller partial slots.
    ((1, 16, 1, 32768, 128, torch.float32), 3, True),
    ((4, 8, 2, 3000, 64, torch.float32), 4, False),
]


def test_noalloc_matches_workspace_entry_point_on_consecutive_calls():
    lib = nat.load()
    for case, seed, masked in CASES:
        print(f"noalloc case {case} masked={masked}", flush=True)
        want = _run(lib, False, case, seed, masked)
        got = _run(lib, True, case, seed, masked)
        for name, a, b in zip(("m", "l", "acc"), got, want):
            assert torch.equal(a, b), f"{name} differs for {case}"


@pytest.mark.parametrize("case", [
    (1200, 16, 1, 16, 128, torch.float16),  # 1,200 partial slots of 16 x 130 floats: ~10 MB
    (1, 16, 1, 65536, 128, torch.float32),  # one row, but 1,024 slots of the generic kernel: ~8.5 MB
])
def test_noalloc_rejects_a_chunk_beyond_the_static_scratch(case):
    lib = nat.load()
    b, hq, hkv, tc, d, dtype = case
    q, k, v, m, l, acc, _, _ = _inputs(b, hq, hkv, tc, d, dtype, 3, False)
    before = acc.clone()
    rc = lib.pgr_attn_step_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), None, None, m.data_ptr(), l.data_ptr(),
                                   acc.data_ptr(), b, hq, hkv, tc, d, CODES[dtype], 1.0 / d**0.5, 0.0,
                                   torch.cuda.current_stream().cuda_stream)
    assert rc == nat.PGR_ERR_CAPACITY
    assert "static scratch" in nat.last_error()
    torch.cuda.synchronize()
    assert torch.equal(acc, before)


def test_noalloc_calls_on_two_streams_do_not_race_on_the_static_scratch():
    """A long chunk on one stream, then at once a short one on another stream that does not
    wait for the first: both share the static array, so without the library's ordering the
    short call's fold would overwrite partial slots before the long call's merge read them.
    Each result must equal the workspace entry point's, bit for bit."""
    lib = nat.load()
    long_case = ((8, 14, 2, 32768, 64, torch.float16), 11, False)
    short_case = ((8, 14, 2, 2048, 64, torch.float16), 12, True)
    want = [_run(lib, False, c, s, mk) for c, s, mk in (long_case, short_case)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for rep in range(3):
        print(f"two-stream noalloc rep {rep}", flush=True)
        states = []
        for (case, seed, masked), st in zip((long_case, short_case), streams):
            b, hq, hkv, tc, d, dtype = case
            q, k, v, m, l, acc, valid, active = _inputs(b, hq, hkv, tc, d, dtype, seed, masked)
            torch.cuda.synchronize()
            states.append((q, k, v, m, l, acc, valid, active, case, st))
        for q, k, v, m, l, acc, valid, active, case, st in states:
            b, hq, hkv, tc, d, dtype = case
            rc = lib.pgr_attn_step_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), _ptr(valid), _ptr(active),
                                           m.data_ptr(), l.data_ptr(), acc.data_ptr(), b, hq, hkv, tc, d,
                                           CODES[dtype], 1.0 / d**0.5, 0.0, st.cuda_stream)
            assert rc == 0, nat.last_error()
        torch.cuda.synchronize()
        for (q, k, v, m, l, acc, valid, active, case, st), w in zip(states, want):
            for name, a, b in zip(("m", "l", "acc"), (m.cpu(), l.cpu(), acc.cpu()), w):
                assert torch.equal(a, b), f"{name} differs for {case} (rep {rep})"
