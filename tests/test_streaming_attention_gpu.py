"""HIP operator API (pager_hf.streaming_attention) against the CPU oracle.

The first eight tests are the reference's own (tests/test_streaming_attention.py:43-293)
with the same shapes and tolerances; the dense check is additionally held to the
max-abs 2e-3 bar against the fp32 oracle. Then the kernel dev-history case list
(bench/streaming_attention_triton_kernel_mvp.py:481-567), bf16, head_dim 32/128, n_rep
from 1 to 16, and a tight comparison of the fp32 state against the oracle's restatement
of the fold kernels (oracle.attention.fold_step with p rounded to the K/V dtype).
Inputs are drawn on the CPU from seeded generators; the oracle sees the same stored values.
"""
from __future__ import annotations

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

HQ, HKV, D = 14, 2, 64
TOL = 2e-3  # max-abs bar on outputs against the fp32 oracle


def dev():
    return torch.device("cuda")


def draw(seed, *shapes, dtype=torch.float16, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(*s, generator=g) * scale).to(dtype) for s in shapes]


def np32(t):
    return t.detach().float().cpu().numpy()


def dense(q, k, v, n_rep, tpb=16, valid=None, scale=None, softcap=None):
    out, mass = oa.dense_reference(np32(q), np32(k), np32(v), n_rep=n_rep, tokens_per_block=tpb,
                                   valid=None if valid is None else valid.cpu().numpy(), scale=scale, softcap=softcap)
    return torch.from_numpy(out), torch.from_numpy(mass)


def close(out, ref, rtol=2e-2, atol=2e-2):
    return torch.allclose(out.float().cpu(), ref.to(out.dtype).float(), rtol=rtol, atol=atol)


def max_abs(a, b):
    return (a.float().cpu() - b.float().cpu()).abs().max().item()


@pytest.mark.parametrize("b,hq,d", [(0, 14, 64), (1, 14, 64), (3, 7, 8), (64, 128, 256)])
def test_state_init_values_shapes_and_reuse(b, hq, d):
    """state_init's one launch writes what the reference's three fills do (m = -inf, l = 0,
    acc = 0, fp32, contiguous), over memory that held other values (the caching allocator
    hands the same blocks back), including a grid-strided size of 2M acc elements."""
    for _ in range(2):
        junk = torch.full((b * hq * (d + 2) + 4096,), 7.0, device=dev())
        del junk
        m, l, acc = streaming_attention_state_init(b, hq, d, dev())
        assert (m.shape, l.shape, acc.shape) == ((b, hq), (b, hq), (b, hq, d))
        assert m.dtype == l.dtype == acc.dtype == torch.float32
        assert m.is_contiguous() and l.is_contiguous() and acc.is_contiguous()
        torch.cuda.synchronize()
        assert bool(torch.all(m == float("-inf"))) and bool(torch.all(l == 0)) and bool(torch.all(acc == 0))
        assert not bool(torch.signbit(acc).any())  # +0.0, as torch.zeros
    with pytest.raises(ValueError):
        streaming_attention_state_init(1, hq, d, torch.device("cpu"))


@pytest.mark.parametrize("tokens,dtype", [(256, torch.float16), (4096, torch.bfloat16), (32768, torch.float16)])
def test_operator_call_replayed_from_a_graph_matches_eager(tokens, dtype):
    """state_init + step + finalize captured in a HIP graph (as the operator benchmark replays
    them) and replayed over new inputs, with eager calls and synchronizations between the
    replays: every replay equals the eager call on the same inputs bit for bit."""
    g = torch.Generator().manual_seed(tokens)
    hq, hkv, d = 28, 4, 128

    def draw():
        return ((torch.randn(1, hq, d, generator=g) * 0.5).to(dtype).cuda(),
                (torch.randn(1, hkv, tokens, d, generator=g) * 0.5).to(dtype).cuda(),
                (torch.randn(1, hkv, tokens, d, generator=g) * 0.5).to(dtype).cuda())

    def call(q, k, v):
        m, l, acc = streaming_attention_state_init(1, hq, d, q.device)
        streaming_attention_step(q, k, v, m, l, acc)
        return streaming_attention_finalize(acc, l, dtype)

    sq, sk, sv = draw()
    call(sq, sk, sv)  # library and allocator set up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call(sq, sk, sv)
    for rep in range(4):
        q, k, v = draw()
        sq.copy_(q)
        sk.copy_(k)
        sv.copy_(v)
        graph.replay()
        torch.cuda.synchronize()
        want = call(q, k, v)
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        if rep == 0:
            ref, _ = dense(q.cpu(), k.cpu(), v.cpu(), hq // hkv)
            assert max_abs(out, ref) < TOL


# -- the reference's eight tests ---------------------------------------------------------


def test_single_pass_matches_dense():
    q, k, v = draw(0, (1, HQ, D), (1, HKV, 200, D), (1, HKV, 200, D))
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    m, l, acc = streaming_attention_state_init(1, HQ, D, dev())
    for s in range(0, 200, 48):
        streaming_attention_step(qd, kd[:, :, s:s + 48], vd[:, :, s:s + 48], m, l, acc)
    out = streaming_attention_finalize(acc, l, torch.float16)
    ref, _ = dense(q, k, v, 7)
    assert close(out, ref)
    assert max_abs(out, ref) < TOL


def test_two_pass_with_tail_matches_dense_mass_and_output():
    tpb, nbl, tail, group = 16, 9, 7, 32
    full = tpb * nbl
    q, k, v = draw(1, (1, HQ, D), (1, HKV, full + tail, D), (1, HKV, full + tail, D))
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    fk, fv, tk, tv = kd[:, :, :full], vd[:, :, :full], kd[:, :, full:], vd[:, :, full:]
    m, l, _ = streaming_attention_state_init(1, HQ, D, dev())
    for s in range(0, full, group):
        streaming_attention_stats_step(qd, fk[:, :, s:s + group], m, l)
    streaming_attention_stats_step(qd, tk, m, l)
    acc = torch.zeros(1, HQ, D, dtype=torch.float32, device=dev())
    mass = torch.zeros(1, HQ, nbl, dtype=torch.float32, device=dev())
    for s in range(0, full, group):
        streaming_attention_accumulate_step(qd, fk[:, :, s:s + group], fv[:, :, s:s + group], m, l, acc, mass,
                                            s // tpb, tpb)
    streaming_attention_fold_fixed_step(qd, tk, tv, m, l, acc)
    out = streaming_attention_finalize(acc, l, torch.float16)
    ref, rmass = dense(q, k, v, 7, tpb)
    assert close(out, ref) and max_abs(out, ref) < TOL
    assert torch.allclose(mass.cpu(), rmass[:, :, :nbl], rtol=2e-2, atol=2e-2)
    assert max_abs(mass, rmass[:, :, :nbl]) < 1e-4


def test_batched_rows_are_independent():
    q, k, v = draw(2, (2, HQ, D), (2, HKV, 96, D), (2, HKV, 96, D))
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    m, l, acc = streaming_attention_state_init(2, HQ, D, dev())
    for s in range(0, 96, 32):
        streaming_attention_step(qd, kd[:, :, s:s + 32], vd[:, :, s:s + 32], m, l, acc)
    out = streaming_attention_finalize(acc, l, torch.float16)
    ref, _ = dense(q, k, v, 7)
    assert close(out, ref) and max_abs(out, ref) < TOL
    # Row 1 alone gives the same bits as row 1 batched.
    m1, l1, a1 = streaming_attention_state_init(1, HQ, D, dev())
    for s in range(0, 96, 32):
        streaming_attention_step(qd[1:], kd[1:, :, s:s + 32].contiguous(), vd[1:, :, s:s + 32].contiguous(), m1, l1, a1)
    assert torch.equal(streaming_attention_finalize(a1, l1, torch.float16)[0], out[1])


def test_padding_mask_excludes_padded_positions():
    q, k, v = draw(3, (1, HQ, D), (1, HKV, 64, D), (1, HKV, 64, D))
    valid = torch.ones(1, 64, dtype=torch.int32)
    valid[:, :20] = 0
    m, l, acc = streaming_attention_state_init(1, HQ, D, dev())
    streaming_attention_step(q.cuda(), k.cuda(), v.cuda(), m, l, acc, valid=valid.cuda())
    out = streaming_attention_finalize(acc, l, torch.float16)
    masked, _ = dense(q, k, v, 7, valid=valid)
    unmasked, _ = dense(q, k, v, 7)
    assert close(out, masked) and max_abs(out, masked) < TOL
    assert not close(out, unmasked)


def test_active_zero_skips_row_regardless_of_valid_mask():
    q, k, v = draw(4, (2, HQ, D), (2, HKV, 32, D), (2, HKV, 32, D))
    active = torch.tensor([0, 1], dtype=torch.int32, device=dev())
    m, l, acc = streaming_attention_state_init(2, HQ, D, dev())
    m0, l0, a0 = m.clone(), l.clone(), acc.clone()
    streaming_attention_step(q.cuda(), k.cuda(), v.cuda(), m, l, acc, valid=torch.ones(2, 32, dtype=torch.int32,
                             device=dev()), active=active)
    assert torch.equal(m[0], m0[0]) and torch.equal(l[0], l0[0]) and torch.equal(acc[0], a0[0])
    out = streaming_attention_finalize(acc, l, torch.float16)
    ref, _ = dense(q[1:], k[1:], v[1:], 7)
    assert close(out[1:], ref) and max_abs(out[1:], ref) < TOL


def test_active_zero_skips_row_in_stats_and_accumulate_steps():
    tpb = 16
    q, k, v = draw(5, (2, HQ, D), (2, HKV, 32, D), (2, HKV, 32, D))
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    valid = torch.ones(2, 32, dtype=torch.int32, device=dev())
    active = torch.tensor([0, 1], dtype=torch.int32, device=dev())
    m, l, acc = streaming_attention_state_init(2, HQ, D, dev())
    m0, l0 = m.clone(), l.clone()
    streaming_attention_stats_step(qd, kd, m, l, valid=valid, active=active)
    assert torch.equal(m[0], m0[0]) and torch.equal(l[0], l0[0])
    mass = torch.zeros(2, HQ, 2, dtype=torch.float32, device=dev())
    a0 = acc.clone()
    streaming_attention_accumulate_step(qd, kd, vd, m, l, acc, mass, 0, tpb, valid=valid, active=active)
    assert torch.equal(acc[0], a0[0]) and torch.equal(mass[0], torch.zeros_like(mass[0]))
    ref, rmass = dense(q[1:], k[1:], v[1:], 7, tpb)
    out = streaming_attention_finalize(acc, l, torch.float16)
    assert close(out[1:], ref) and max_abs(out[1:], ref) < TOL
    assert torch.allclose(mass[1:].cpu(), rmass, rtol=2e-2, atol=2e-2)


def test_custom_scale_and_softcap_match_dense_reference():
    scale, cap = 224.0**-0.5, 50.0
    q, k, v = draw(6, (1, HQ, D), (1, HKV, 96, D), (1, HKV, 96, D))
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    m, l, acc = streaming_attention_state_init(1, HQ, D, dev())
    for s in range(0, 96, 32):
        streaming_attention_step(qd, kd[:, :, s:s + 32], vd[:, :, s:s + 32], m, l, acc, scale=scale, softcap=cap)
    out = streaming_attention_finalize(acc, l, torch.float16)
    ref, _ = dense(q, k, v, 7, scale=scale, softcap=cap)
    assert close(out, ref) and max_abs(out, ref) < TOL
    plain, _ = dense(q, k, v, 7)
    assert not close(out, plain)


def test_default_scale_and_softcap_unchanged():
    q, k, v = draw(7, (1, HQ, D), (1, HKV, 64, D), (1, HKV, 64, D))
    m, l, acc = streaming_attention_state_init(1, HQ, D, dev())
    streaming_attention_step(q.cuda(), k.cuda(), v.cuda(), m, l, acc)
    out = streaming_attention_finalize(acc, l, torch.float16)
    m2, l2, a2 = streaming_attention_state_init(1, HQ, D, dev())
    streaming_attention_step(q.cuda(), k.cuda(), v.cuda(), m2, l2, a2, scale=1.0 / 8.0, softcap=None)
    assert torch.equal(out, streaming_attention_finalize(a2, l2, torch.float16))
    ref, _ = dense(q, k, v, 7)
    assert close(out, ref) and max_abs(out, ref) < TOL


# -- dev-history case list and wider coverage ------------------------------------------------


@pytest.mark.parametrize("total", [1, 17, 64, 69, 200, 2000, 6000])
def test_single_call_lengths(total):
    q, k, v = draw(10 + total, (1, HQ, D), (1, HKV, total, D), (1, HKV, total, D))
    m, l, acc = streaming_attention_state_init(1, HQ, D, dev())
    streaming_attention_step(q.cuda(), k.cuda(), v.cuda(), m, l, acc)
    out = streaming_attention_finalize(acc, l, torch.float16)
    ref, _ = dense(q, k, v, 7)
    assert max_abs(out, ref) < TOL


@pytest.mark.parametrize("total,group", [(200, 64), (200, 16), (6000, 128), (203, 17)])
def test_grouped_folds(total, group):
    q, k, v = draw(20 + group, (1, HQ, D), (1, HKV, total, D), (1, HKV, total, D))
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    m, l, acc = streaming_attention_state_init(1, HQ, D, dev())
    for s in range(0, total, group):
        streaming_attention_step(qd, kd[:, :, s:s + group], vd[:, :, s:s + group], m, l, acc)
    out = streaming_attention_finalize(acc, l, torch.float16)
    ref, _ = dense(q, k, v, 7)
    assert max_abs(out, ref) < TOL


@pytest.mark.parametrize("total,group", [(200, 64), (200, 16), (6000, 128), (203, 32)])
def test_mass_two_pass_cases(total, group):
    tpb = 16
    q, k, v = draw(30 + group, (1, HQ, D), (1, HKV, total, D), (1, HKV, total, D))
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    full = total // tpb * tpb
    nbl = full // tpb
    m, l, _ = streaming_attention_state_init(1, HQ, D, dev())
    for s in range(0, full, group):
        streaming_attention_stats_step(qd, kd[:, :, s:min(s + group, full)], m, l)
    if total > full:
        streaming_attention_stats_step(qd, kd[:, :, full:], m, l)
    acc = torch.zeros(1, HQ, D, dtype=torch.float32, device=dev())
    mass = torch.zeros(1, HQ, max(nbl, 1), dtype=torch.float32, device=dev())
    for s in range(0, full, group):
        e = min(s + group, full)
        streaming_attention_accumulate_step(qd, kd[:, :, s:e], vd[:, :, s:e], m, l, acc, mass, s // tpb, tpb)
    if total > full:
        streaming_attention_fold_fixed_step(qd, kd[:, :, full:], vd[:, :, full:], m, l, acc)
    out = streaming_attention_finalize(acc, l, torch.float16)
    ref, rmass = dense(q, k, v, 7, tpb)
    assert max_abs(out, ref) < TOL
    assert max_abs(mass[:, :, :nbl], rmass[:, :, :nbl]) < 1e-4


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 64), (32, 8, 128), (8, 8, 64), (16, 1, 32), (32, 4, 64), (12, 2, 128)])
def test_dtypes_head_dims_and_group_sizes(dtype, hq, hkv, d):
    n_rep = hq // hkv
    q, k, v = draw(40 + hq + d, (3, hq, d), (3, hkv, 333, d), (3, hkv, 333, d), dtype=dtype, scale=0.5)
    valid = torch.ones(3, 333, dtype=torch.int32)
    valid[1, :100] = 0
    m, l, acc = streaming_attention_state_init(3, hq, d, dev())
    qd, kd, vd, vald = q.cuda(), k.cuda(), v.cuda(), valid.cuda()
    for s in range(0, 333, 111):
        streaming_attention_step(qd, kd[:, :, s:s + 111], vd[:, :, s:s + 111], m, l, acc, valid=vald[:, s:s + 111])
    out = streaming_attention_finalize(acc, l, dtype)
    ref, _ = dense(q, k, v, n_rep, valid=valid)
    assert max_abs(out, ref) < TOL
    # fp32 state against the oracle's fold with p rounded to the element type.
    om, ol, oacc = oa.state_init(3, hq, d)
    rnd = oa.round_fp16 if dtype == torch.float16 else oa.round_bf16
    for s in range(0, 333, 111):
        oa.fold_step(np32(q), np32(k[:, :, s:s + 111]), np32(v[:, :, s:s + 111]), om, ol, oacc,
                     valid=valid[:, s:s + 111].numpy(), p_round=rnd)
    fin = oa.finalize(oacc, ol)
    assert np.abs(np32(acc / l[..., None]) - fin).max() < (2e-4 if dtype == torch.float16 else 2e-3)


def test_finalize_matches_torch_division_bit_for_bit():
    g = torch.Generator().manual_seed(50)
    acc = torch.randn(3, HQ, D, generator=g).cuda()
    l = (torch.rand(3, HQ, generator=g) + 0.5).cuda()
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        want = (acc / l.unsqueeze(-1)).to(dtype)
        assert torch.equal(streaming_attention_finalize(acc, l, dtype), want)


def test_n_rep_above_16_is_rejected():
    q = torch.zeros(1, 34, 64, dtype=torch.float16, device=dev())
    k = torch.zeros(1, 2, 8, 64, dtype=torch.float16, device=dev())
    m, l, acc = streaming_attention_state_init(1, 34, 64, dev())
    with pytest.raises(NotImplementedError):
        streaming_attention_step(q, k, k, m, l, acc)


def test_empty_chunk_is_a_no_op():
    q = torch.zeros(1, HQ, D, dtype=torch.float16, device=dev())
    k = torch.zeros(1, HKV, 0, D, dtype=torch.float16, device=dev())
    m, l, acc = streaming_attention_state_init(1, HQ, D, dev())
    streaming_attention_step(q, k, k, m, l, acc)
    assert torch.isinf(m).all() and (l == 0).all()


def test_fully_masked_row_stays_nan_free():
    """A row with nothing valid yet keeps m=-inf, l=0, acc=0 (streaming_attention.py:165-172)."""
    q, k, v = draw(60, (2, HQ, D), (2, HKV, 48, D), (2, HKV, 48, D))
    valid = torch.ones(2, 48, dtype=torch.int32)
    valid[0] = 0
    m, l, acc = streaming_attention_state_init(2, HQ, D, dev())
    streaming_attention_step(q.cuda(), k.cuda(), v.cuda(), m, l, acc, valid=valid.cuda())
    assert torch.isinf(m[0]).all() and (l[0] == 0).all() and (acc[0] == 0).all()
    assert not torch.isnan(acc).any()


# -- the envelope beyond the MFMA kernel: head dims 8, 16, 256 and fp32 q/k/v -----------------


def _two_pass_with_tail(q, k, v, tpb, group, *, valid=None, out_dtype=None):
    """stats over every group and the tail, accumulate with mass over full blocks, fold_fixed
    for the tail (paged_model.py:992-1048); returns (out, mass) on the CPU."""
    b, hq, d = q.shape
    total = k.shape[2]
    full = total // tpb * tpb
    nbl = full // tpb
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    vald = None if valid is None else valid.cuda()
    sl = lambda t, s, e: None if t is None else t[:, s:e].contiguous()  # noqa: E731
    m, l, _ = streaming_attention_state_init(b, hq, d, dev())
    for s in range(0, full, group):
        e = min(s + group, full)
        streaming_attention_stats_step(qd, kd[:, :, s:e], m, l, valid=sl(vald, s, e))
    if total > full:
        streaming_attention_stats_step(qd, kd[:, :, full:], m, l, valid=sl(vald, full, total))
    acc = torch.zeros(b, hq, d, dtype=torch.float32, device=dev())
    mass = torch.zeros(b, hq, max(nbl, 1), dtype=torch.float32, device=dev())
    for s in range(0, full, group):
        e = min(s + group, full)
        streaming_attention_accumulate_step(qd, kd[:, :, s:e], vd[:, :, s:e], m, l, acc, mass, s // tpb, tpb,
                                            valid=sl(vald, s, e))
    if total > full:
        streaming_attention_fold_fixed_step(qd, kd[:, :, full:], vd[:, :, full:], m, l, acc,
                                            valid=sl(vald, full, total))
    out = streaming_attention_finalize(acc, l, out_dtype or q.dtype)
    return out, mass[:, :, :nbl].cpu()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 8), (8, 8, 16), (16, 1, 256), (14, 2, 256), (12, 2, 16)])
def test_head_dims_outside_the_mfma_kernel(dtype, hq, hkv, d):
    """Head dims 8 and 16 (the reference zero-pads Q/K to 16 columns below 16, which leaves every
    dot product unchanged) and 256: one-pass folds and the two-pass-with-tail path with mass,
    with a padding mask, against the dense oracle."""
    n_rep = hq // hkv
    q, k, v = draw(70 + d + hq, (3, hq, d), (3, hkv, 337, d), (3, hkv, 337, d), dtype=dtype, scale=0.5)
    valid = torch.ones(3, 337, dtype=torch.int32)
    valid[2, :150] = 0
    m, l, acc = streaming_attention_state_init(3, hq, d, dev())
    qd, kd, vd, vald = q.cuda(), k.cuda(), v.cuda(), valid.cuda()
    for s in range(0, 337, 100):
        streaming_attention_step(qd, kd[:, :, s:s + 100], vd[:, :, s:s + 100], m, l, acc,
                                 valid=vald[:, s:s + 100].contiguous())
    ref, rmass = dense(q, k, v, n_rep, tpb=16, valid=valid)
    assert max_abs(streaming_attention_finalize(acc, l, dtype), ref) < TOL
    out, mass = _two_pass_with_tail(q, k, v, 16, 64, valid=valid)
    assert max_abs(out, ref) < TOL
    assert max_abs(mass, rmass[:, :, :mass.shape[2]]) < 1e-4


def test_fp32_dev_cases_at_1e4():
    """The reference's fp32 dev cases (bench/streaming_attention_triton_kernel_mvp.py:488 and
    :557-566): 200 tokens in one fold, and the grouped two-pass with 16-token block mass, at
    rtol = atol = 1e-4 against the dense fp32 result."""
    q, k, v = draw(80, (1, HQ, D), (1, HKV, 200, D), (1, HKV, 200, D), dtype=torch.float32)
    m, l, acc = streaming_attention_state_init(1, HQ, D, dev())
    streaming_attention_step(q.cuda(), k.cuda(), v.cuda(), m, l, acc)
    out = streaming_attention_finalize(acc, l, torch.float32)
    ref, rmass = dense(q, k, v, 7, tpb=16)
    assert torch.allclose(out.cpu(), ref, rtol=1e-4, atol=1e-4)
    out2, mass = _two_pass_with_tail(q, k, v, 16, 64)
    assert torch.allclose(out2.cpu(), ref, rtol=1e-4, atol=1e-4)
    assert torch.allclose(mass, rmass[:, :, :mass.shape[2]], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("hq,hkv,d", [(14, 2, 8), (8, 2, 16), (14, 2, 32), (14, 2, 64), (32, 8, 128), (16, 2, 256)])
def test_fp32_qkv_every_head_dim(hq, hkv, d):
    """fp32 q/k/v at every head dim, ragged chunks with a padding mask and an inactive row,
    softcap, against the oracle at 1e-4; P is not rounded (its dtype is fp32)."""
    n_rep = hq // hkv
    q, k, v = draw(90 + d, (3, hq, d), (3, hkv, 411, d), (3, hkv, 411, d), dtype=torch.float32, scale=0.5)
    valid = torch.ones(3, 411, dtype=torch.int32)
    valid[0, 300:] = 0
    active = torch.tensor([1, 1, 0], dtype=torch.int32)
    m, l, acc = streaming_attention_state_init(3, hq, d, dev())
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    for s in range(0, 411, 137):
        streaming_attention_step(qd, kd[:, :, s:s + 137], vd[:, :, s:s + 137], m, l, acc,
                                 valid=valid[:, s:s + 137].contiguous().cuda(), active=active.cuda(), softcap=30.0)
    out = streaming_attention_finalize(acc, l, torch.float32)
    ref, _ = dense(q, k, v, n_rep, valid=valid, softcap=30.0)
    assert torch.allclose(out[:2].cpu(), ref[:2], rtol=1e-4, atol=1e-4)
    assert torch.isinf(m[2]).all() and (l[2] == 0).all() and (acc[2] == 0).all()  # inactive row untouched


def test_unsupported_head_dim_is_rejected():
    q = torch.zeros(1, 8, 48, dtype=torch.float16, device=dev())
    k = torch.zeros(1, 2, 8, 48, dtype=torch.float16, device=dev())
    m, l, acc = streaming_attention_state_init(1, 8, 48, dev())
    with pytest.raises(NotImplementedError):
        streaming_attention_step(q, k, k, m, l, acc)


# -- long chunks: many split-K slots per merge group ------------------------------------------


@pytest.mark.parametrize("b, hq, hkv, d, tokens, dtype", [
    (2, 28, 4, 128, 32768, torch.float16),    # 64 splits per (row, KV head), 4 merge groups
    (1, 14, 2, 64, 65536, torch.bfloat16),    # 256 splits, 8 groups: four batches of slots per group
    (1, 8, 1, 256, 16384, torch.float16),     # head dim 256 (VALU kernel), 2 groups
    (1, 8, 2, 32, 8192, torch.float32),       # fp32 q/k/v
])
def test_long_chunk_merges_many_split_slots(b, hq, hkv, d, tokens, dtype):
    """A chunk long enough that each merge thread group combines several batches of split-K
    slots, folded after a first short chunk (so the merge also rescales an existing state),
    with a masked stretch longer than a split (slots with m = -inf)."""
    q, k, v = draw(40 + d, (b, hq, d), (b, hkv, 64 + tokens, d), (b, hkv, 64 + tokens, d), dtype=dtype, scale=0.5)
    valid = torch.ones(b, 64 + tokens, dtype=torch.int32)
    valid[:, 64 + tokens // 3: 64 + tokens // 3 + tokens // 4] = 0
    qd, kd, vd, vald = q.cuda(), k.cuda(), v.cuda(), valid.cuda()
    m, l, acc = streaming_attention_state_init(b, hq, d, dev())
    streaming_attention_step(qd, kd[:, :, :64], vd[:, :, :64], m, l, acc, valid=vald[:, :64])
    streaming_attention_step(qd, kd[:, :, 64:], vd[:, :, 64:], m, l, acc, valid=vald[:, 64:])
    out = streaming_attention_finalize(acc, l, torch.float32)
    ref, _ = dense(q, k, v, hq // hkv, valid=valid)
    tol = 1e-4 if dtype == torch.float32 else TOL
    assert max_abs(out, ref) < tol


def test_long_two_pass_with_mass_merges_many_split_slots():
    """Stats then accumulate over one 32768-token chunk (128 splits per KV head at this shape),
    with 32-token block mass: output and mass against the dense oracle."""
    hq, hkv, d, tokens, tpb = 28, 4, 128, 32768, 32
    q, k, v = draw(77, (1, hq, d), (1, hkv, tokens, d), (1, hkv, tokens, d), scale=0.5)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    m = torch.full((1, hq), float("-inf"), dtype=torch.float32, device=dev())
    l = torch.zeros(1, hq, dtype=torch.float32, device=dev())
    streaming_attention_stats_step(qd, kd, m, l)
    acc = torch.zeros(1, hq, d, dtype=torch.float32, device=dev())
    nbl = tokens // tpb
    mass = torch.zeros(1, hq, nbl, dtype=torch.float32, device=dev())
    streaming_attention_accumulate_step(qd, kd, vd, m, l, acc, mass, 0, tpb)
    out = streaming_attention_finalize(acc, l, torch.float32)
    ref, rmass = dense(q, k, v, hq // hkv, tpb)
    assert max_abs(out, ref) < TOL
    assert max_abs(mass, rmass) < 1e-4
