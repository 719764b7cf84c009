"""Pins the attention oracle (oracle/attention.py) against textbook math, not against itself.

* float64 brute force with scalar math.exp loops over (batch, head, token);
* closed forms: identical keys give the mean of the valid V rows; a dominant key selects
  its V row; which query heads read which KV head (repeat-interleave, streaming_attention.py:119-123);
* the fold kernels' semantics: any chunking of a fold equals the dense form; two-pass
  stats + accumulate + fold_fixed reproduces dense output and mass
  (tests/test_streaming_attention.py:65-119 structure); active=0 is an exact no-op;
* mass over all blocks (tail included) sums to 1 per query head;
* bf16 rounding helper agrees with torch's float32 -> bfloat16 conversion.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa

HQ, HKV, D = 14, 2, 64  # tests/test_streaming_attention.py:15-17


def rand(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def brute_force(q, k, v, n_rep, tpb, valid=None, scale=None, softcap=None):
    b_, hq, d = q.shape
    t_ = k.shape[2]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = np.zeros((b_, hq, d))
    nb = (t_ + tpb - 1) // tpb
    mass = np.zeros((b_, hq, nb))
    for b in range(b_):
        for h in range(hq):
            kh = h // n_rep
            s = []
            for t in range(t_):
                if valid is not None and valid[b, t] == 0:
                    s.append(None)
                    continue
                x = sum(float(q[b, h, i]) * float(k[b, kh, t, i]) for i in range(d)) * scale
                if softcap is not None:
                    x = softcap * math.tanh(x / softcap)
                s.append(x)
            mx = max(x for x in s if x is not None)
            w = [0.0 if x is None else math.exp(x - mx) for x in s]
            z = sum(w)
            w = [x / z for x in w]
            for t in range(t_):
                out[b, h] += w[t] * v[b, kh, t].astype(np.float64)
                mass[b, h, t // tpb] += w[t]
    return out, mass


@pytest.mark.parametrize("softcap", [None, 2.0])
def test_dense_matches_brute_force(softcap):
    rng = np.random.default_rng(0)
    q, k, v = rand(rng, 2, 6, 8), rand(rng, 2, 2, 11, 8), rand(rng, 2, 2, 11, 8)
    valid = np.ones((2, 11), np.int32)
    valid[1, :3] = 0
    out, mass = oa.dense_reference(q, k, v, n_rep=3, tokens_per_block=4, valid=valid, scale=0.37, softcap=softcap)
    bo, bm = brute_force(q, k, v, 3, 4, valid=valid, scale=0.37, softcap=softcap)
    np.testing.assert_allclose(out, bo, rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(mass, bm, rtol=2e-5, atol=2e-6)


def test_identical_keys_give_mean_of_valid_values():
    rng = np.random.default_rng(1)
    q = rand(rng, 1, 4, 8)
    k = np.repeat(rand(rng, 1, 2, 1, 8), 9, axis=2)
    v = rand(rng, 1, 2, 9, 8)
    valid = np.ones((1, 9), np.int32)
    valid[0, :2] = 0
    out, mass = oa.dense_reference(q, k, v, n_rep=2, tokens_per_block=3, valid=valid)
    for h in range(4):
        np.testing.assert_allclose(out[0, h], v[0, h // 2, 2:].mean(axis=0), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(mass[0, :, 0], 1 / 7, rtol=1e-5)  # block 0 = tokens 0..2, only 2 valid


def test_dominant_key_selects_its_value_row():
    rng = np.random.default_rng(2)
    q = np.zeros((1, 2, 8), np.float32)
    q[0, :, 0] = 1.0
    k = rand(rng, 1, 1, 10, 8, scale=0.01)
    k[0, 0, 6, 0] = 400.0
    v = rand(rng, 1, 1, 10, 8)
    out, mass = oa.dense_reference(q, k, v, n_rep=2, tokens_per_block=5)
    np.testing.assert_allclose(out[0, 0], v[0, 0, 6], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(mass[0, 0], [0.0, 1.0], atol=1e-6)


def test_query_heads_read_kv_heads_by_repeat_interleave():
    q = np.ones((1, HQ, 4), np.float32)
    k = np.zeros((1, HKV, 5, 4), np.float32)
    v = np.zeros((1, HKV, 5, 4), np.float32)
    v[0, 1] = 1.0  # kv head 1 carries ones
    out, _ = oa.dense_reference(q, k, v, n_rep=HQ // HKV, tokens_per_block=5)
    assert np.all(out[0, :7] == 0.0) and np.all(out[0, 7:] == 1.0)
    m, l, acc = oa.state_init(1, HQ, 4)
    oa.fold_step(q, k, v, m, l, acc)
    fin = oa.finalize(acc, l)
    assert np.all(fin[0, :7] == 0.0) and np.all(fin[0, 7:] == 1.0)


@pytest.mark.parametrize("chunk", [1, 13, 64, 200])
def test_fold_in_any_chunking_equals_dense(chunk):
    rng = np.random.default_rng(3)
    t = 200
    q, k, v = rand(rng, 2, HQ, D), rand(rng, 2, HKV, t, D), rand(rng, 2, HKV, t, D)
    valid = np.ones((2, t), np.int32)
    valid[0, :37] = 0
    m, l, acc = oa.state_init(2, HQ, D)
    for s in range(0, t, chunk):
        oa.fold_step(q, k[:, :, s:s + chunk], v[:, :, s:s + chunk], m, l, acc, valid=valid[:, s:s + chunk])
    dense, _ = oa.dense_reference(q, k, v, n_rep=7, tokens_per_block=16, valid=valid)
    np.testing.assert_allclose(oa.finalize(acc, l), dense, rtol=1e-4, atol=1e-5)


def test_two_pass_with_tail_matches_dense_output_and_mass():
    rng = np.random.default_rng(4)
    tpb, nb, tail = 16, 9, 7
    full = tpb * nb
    q, k, v = rand(rng, 1, HQ, D), rand(rng, 1, HKV, full + tail, D), rand(rng, 1, HKV, full + tail, D)
    fk, fv = k[:, :, :full], v[:, :, :full]
    m, l, _ = oa.state_init(1, HQ, D)
    for s in range(0, full, 32):
        oa.stats_step(q, fk[:, :, s:s + 32], m, l)
    oa.stats_step(q, k[:, :, full:], m, l)
    acc = np.zeros((1, HQ, D), np.float32)
    mass = np.zeros((1, HQ, nb), np.float32)
    for s in range(0, full, 32):
        oa.accumulate_step(q, fk[:, :, s:s + 32], fv[:, :, s:s + 32], m, l, acc, mass, s // tpb, tpb)
    oa.fold_fixed_step(q, k[:, :, full:], v[:, :, full:], m, l, acc)
    dense, dmass = oa.dense_reference(q, k, v, n_rep=7, tokens_per_block=tpb)
    np.testing.assert_allclose(oa.finalize(acc, l), dense, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(mass, dmass[:, :, :nb], rtol=1e-4, atol=1e-6)
    # The tail's share is what the block masses leave out of 1.
    np.testing.assert_allclose(mass.sum(-1) + dmass[:, :, nb], 1.0, rtol=1e-5)


def test_active_zero_is_an_exact_no_op():
    rng = np.random.default_rng(5)
    q, k, v = rand(rng, 2, HQ, D), rand(rng, 2, HKV, 32, D), rand(rng, 2, HKV, 32, D)
    m, l, acc = oa.state_init(2, HQ, D)
    oa.fold_step(q, k, v, m, l, acc)
    m0, l0, a0 = m.copy(), l.copy(), acc.copy()
    oa.fold_step(q, k, v, m, l, acc, active=np.array([0, 1], np.int32))
    assert np.array_equal(m[0], m0[0]) and np.array_equal(l[0], l0[0]) and np.array_equal(acc[0], a0[0])
    assert not np.array_equal(l[1], l0[1])


def test_masked_positions_do_not_matter():
    rng = np.random.default_rng(6)
    q, k, v = rand(rng, 1, HQ, D), rand(rng, 1, HKV, 64, D), rand(rng, 1, HKV, 64, D)
    valid = np.ones((1, 64), np.int32)
    valid[0, :20] = 0
    a, _ = oa.dense_reference(q, k, v, n_rep=7, tokens_per_block=16, valid=valid)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, :20] = 50.0
    v2[:, :, :20] = -9.0
    b, _ = oa.dense_reference(q, k2, v2, n_rep=7, tokens_per_block=16, valid=valid)
    np.testing.assert_array_equal(a, b)
    c, _ = oa.dense_reference(q, k, v, n_rep=7, tokens_per_block=16)
    assert not np.allclose(a, c, atol=1e-3)


def test_p_rounding_to_fp16_stays_within_tolerance():
    rng = np.random.default_rng(7)
    q = oa.round_fp16(rand(rng, 1, HQ, D, scale=0.5))
    k = oa.round_fp16(rand(rng, 1, HKV, 300, D, scale=0.5))
    v = oa.round_fp16(rand(rng, 1, HKV, 300, D, scale=0.5))
    m, l, acc = oa.state_init(1, HQ, D)
    oa.fold_step(q, k, v, m, l, acc, p_round=oa.round_fp16)
    dense, _ = oa.dense_reference(q, k, v, n_rep=7, tokens_per_block=16)
    assert np.abs(oa.finalize(acc, l) - dense).max() < 2e-3


def test_round_bf16_matches_torch():
    rng = np.random.default_rng(8)
    x = np.concatenate([rand(rng, 4096, scale=3.0), np.array([0.0, -0.0, 1e-40, 3.4e38, -1.5], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(oa.round_bf16(x), want)


def test_chunked_prototype_matches_dense():
    rng = np.random.default_rng(9)
    q, k, v = rand(rng, 8, 16), rand(rng, 8, 300, 16), rand(rng, 8, 300, 16)
    chunks = [(k[:, s:s + 13], v[:, s:s + 13]) for s in range(0, 300, 13)]
    got = oa.chunked_online_softmax(q, chunks)
    want, _ = oa.dense_reference(q[None], k[None], v[None], n_rep=1, tokens_per_block=16)
    np.testing.assert_allclose(got, want[0], rtol=1e-4, atol=1e-5)


def test_n_rep_guard():
    with pytest.raises(NotImplementedError):
        oa.validate_n_rep(17)
    oa.validate_n_rep(16)
