"""CPU restatement of the reference's decode-attention math, for use as a test oracle only.

TEST INFRASTRUCTURE. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only to check or time the product.
The product path (HIP kernels behind ``pager_hf.streaming_attention``) never calls it.

Two restatements live here:

``dense_reference``
    The reference test suite's dense fp32 oracle, ``tests/test_streaming_attention.py:20-40``:
    GQA by repeat-interleave of KV heads, ``softmax(q.k * scale)`` with optional softcap
    ``c*tanh(s/c)`` and a 0/1 validity mask, output ``weights @ v`` and per-block attention
    mass (the weights summed over each ``tokens_per_block`` slice).

``fold_step`` / ``stats_step`` / ``accumulate_step`` / ``fold_fixed_step`` / ``finalize``
    The semantics of the four Triton kernels in ``pager_hf/streaming_attention.py:77-430``
    and their wrappers ``:444-670``: online-softmax state ``(m, l, acc)`` carried across
    calls, 64-token tiles, the "nothing valid yet" guard (``:165-172``, ``:253-257``), the
    per-row ``active`` skip (``:140-143``), ``p`` rounded to the K/V dtype before the P.V
    product (``:178``, ``:347``, ``:428``), and block mass ``sum(p)/l_final`` per
    ``tokens_per_block`` tile (``:349-350``).

All arrays are numpy. Inputs in fp16/bf16 are represented as float32 arrays holding the
exact fp16/bf16 values (the caller upcasts), plus a ``p_round`` callable that rounds to
the storage dtype.

Pinned by tests/test_oracle_attention.py: float64 brute force with scalar ``math.exp``
loops on small cases, closed forms (identical keys give the mean of V; a dominant key
selects its V row; which query heads read which KV head), chunking invariance of the
fold against the dense form, the active=0 no-op, and mass summing to one.
"""
from __future__ import annotations

import numpy as np

BLOCK_KV = 64  # streaming_attention.py:11
M_TILE = 16  # streaming_attention.py:55


def validate_n_rep(n_rep: int) -> None:
    """streaming_attention.py:69-74."""
    if n_rep > M_TILE:
        raise NotImplementedError(
            f"streaming attention's GQA query-head packing supports n_rep up to {M_TILE}, got {n_rep}."
        )


def round_fp16(x: np.ndarray) -> np.ndarray:
    return x.astype(np.float16).astype(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to bfloat16, returned as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.uint64)
    rounding = ((bits >> 16) & 1) + 0x7FFF
    out = ((bits + rounding) >> 16) << 16
    out = out.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def no_round(x: np.ndarray) -> np.ndarray:
    return x


def _scores(q_rows: np.ndarray, k_tile: np.ndarray, scale: float, softcap: float) -> np.ndarray:
    """q_rows [R, D] . k_tile [C, D]^T * scale, then softcap (streaming_attention.py:158-160)."""
    s = (q_rows @ k_tile.T).astype(np.float32) * np.float32(scale)
    if softcap > 0.0:
        s = np.float32(softcap) * np.tanh(s / np.float32(softcap))
    return s.astype(np.float32)


def dense_reference(q, k, v, *, n_rep, tokens_per_block, valid=None, scale=None, softcap=None):
    """tests/test_streaming_attention.py:20-40.

    q [B, Hq, D]; k, v [B, Hkv, T, D]; valid optional [B, T] 0/1.
    Returns (out [B, Hq, D], block_mass [B, Hq, ceil(T / tokens_per_block)]) in float32.
    """
    q = np.asarray(q, dtype=np.float32)
    key = np.repeat(np.asarray(k, dtype=np.float32), n_rep, axis=1)
    value = np.repeat(np.asarray(v, dtype=np.float32), n_rep, axis=1)
    if scale is None:
        scale = 1.0 / (q.shape[-1] ** 0.5)
    scores = np.einsum("bhd,bhtd->bht", q, key).astype(np.float32) * np.float32(scale)
    if softcap is not None:
        scores = np.float32(softcap) * np.tanh(scores / np.float32(softcap))
    if valid is not None:
        scores = np.where(np.asarray(valid)[:, None, :] == 0, np.float32(-np.inf), scores)
    with np.errstate(invalid="ignore"):
        smax = scores.max(axis=-1, keepdims=True)
        e = np.exp(scores - smax)
        weights = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
    out = np.einsum("bht,bhtd->bhd", weights, value).astype(np.float32)
    total = k.shape[2]
    num_blocks = (total + tokens_per_block - 1) // tokens_per_block
    mass = np.stack(
        [weights[:, :, b * tokens_per_block : (b + 1) * tokens_per_block].sum(axis=-1) for b in range(num_blocks)],
        axis=2,
    ) if num_blocks else np.zeros(weights.shape[:2] + (0,), np.float32)
    return out, mass.astype(np.float32)


def state_init(batch_size: int, num_query_heads: int, head_dim: int):
    """streaming_attention.py:444-449."""
    m = np.full((batch_size, num_query_heads), -np.inf, dtype=np.float32)
    l = np.zeros((batch_size, num_query_heads), dtype=np.float32)
    acc = np.zeros((batch_size, num_query_heads, head_dim), dtype=np.float32)
    return m, l, acc


def _defaults(q, k, valid, active, scale):
    batch, num_query_heads, head_dim = q.shape
    _, num_kv_heads, total, _ = k.shape
    n_rep = num_query_heads // num_kv_heads
    validate_n_rep(n_rep)
    if valid is None:
        valid = np.ones((batch, total), dtype=np.int32)
    if active is None:
        active = np.ones((batch,), dtype=np.int32)
    if scale is None:
        scale = 1.0 / (head_dim**0.5)
    return batch, num_kv_heads, total, n_rep, np.asarray(valid), np.asarray(active), float(scale)


def fold_step(q, k, v, m, l, acc, valid=None, active=None, scale=None, softcap=None, p_round=no_round):
    """In-place online-softmax fold of one chunk (streaming_attention.py:77-185, :452-513)."""
    batch, hkv, total, n_rep, valid, active, scale = _defaults(q, k, valid, active, scale)
    softcap = float(softcap or 0.0)
    for b in range(batch):
        if active[b] == 0:
            continue
        for h in range(hkv):
            rows = slice(h * n_rep, (h + 1) * n_rep)
            qr = q[b, rows]
            mr, lr, ar = m[b, rows].copy(), l[b, rows].copy(), acc[b, rows].copy()
            for start in range(0, total, BLOCK_KV):
                end = min(start + BLOCK_KV, total)
                mask = valid[b, start:end] != 0
                s = _scores(qr, k[b, h, start:end], scale, softcap)
                s = np.where(mask[None, :], s, np.float32(-np.inf))
                m_new = np.maximum(mr, s.max(axis=1))
                empty = m_new == -np.inf
                with np.errstate(invalid="ignore"):
                    alpha = np.where(empty, np.float32(0.0), np.exp(mr - m_new)).astype(np.float32)
                    p = np.where(empty[:, None], np.float32(0.0), np.exp(s - m_new[:, None])).astype(np.float32)
                vt = np.where(mask[:, None], v[b, h, start:end], np.float32(0.0))
                ar = ar * alpha[:, None] + p_round(p) @ vt
                lr = lr * alpha + p.sum(axis=1)
                mr = m_new
            m[b, rows], l[b, rows], acc[b, rows] = mr, lr, ar


def stats_step(q, k, m, l, valid=None, active=None, scale=None, softcap=None):
    """In-place (m, l) fold of one chunk's K (streaming_attention.py:188-261, :516-560)."""
    batch, hkv, total, n_rep, valid, active, scale = _defaults(q, k, valid, active, scale)
    softcap = float(softcap or 0.0)
    for b in range(batch):
        if active[b] == 0:
            continue
        for h in range(hkv):
            rows = slice(h * n_rep, (h + 1) * n_rep)
            qr = q[b, rows]
            mr, lr = m[b, rows].copy(), l[b, rows].copy()
            for start in range(0, total, BLOCK_KV):
                end = min(start + BLOCK_KV, total)
                mask = valid[b, start:end] != 0
                s = _scores(qr, k[b, h, start:end], scale, softcap)
                s = np.where(mask[None, :], s, np.float32(-np.inf))
                m_new = np.maximum(mr, s.max(axis=1))
                empty = m_new == -np.inf
                with np.errstate(invalid="ignore"):
                    lr = lr * np.where(empty, np.float32(0.0), np.exp(mr - m_new))
                    lr = lr + np.where(empty[:, None], np.float32(0.0), np.exp(s - m_new[:, None])).sum(axis=1)
                mr = m_new
            m[b, rows], l[b, rows] = mr, lr.astype(np.float32)


def _fixed_fold(q, k, v, m, l, acc, valid, active, scale, softcap, p_round, block_mass, block_id_offset, tpb):
    batch, hkv, total, n_rep, valid, active, scale = _defaults(q, k, valid, active, scale)
    softcap = float(softcap or 0.0)
    tile = tpb if block_mass is not None else BLOCK_KV
    for b in range(batch):
        if active[b] == 0:
            continue
        for h in range(hkv):
            rows = slice(h * n_rep, (h + 1) * n_rep)
            qr = q[b, rows]
            m_final, l_final = m[b, rows], l[b, rows]
            ar = acc[b, rows].copy()
            for j, start in enumerate(range(0, total, tile)):
                end = min(start + tile, total)
                mask = valid[b, start:end] != 0
                s = _scores(qr, k[b, h, start:end], scale, softcap)
                # A masked position contributes exactly 0 (the reference's exp(-inf - m)
                # for finite m); written as a select so it stays 0 when m is -inf too.
                with np.errstate(invalid="ignore", over="ignore"):
                    p = np.where(mask[None, :], np.exp(s - m_final[:, None]), np.float32(0.0)).astype(np.float32)
                vt = np.where(mask[:, None], v[b, h, start:end], np.float32(0.0))
                ar = ar + p_round(p) @ vt
                if block_mass is not None:
                    with np.errstate(invalid="ignore", divide="ignore"):
                        block_mass[b, rows, block_id_offset + j] = p.sum(axis=1) / l_final
            acc[b, rows] = ar


def accumulate_step(
    q, k, v, m, l, acc, block_mass, block_id_offset, tokens_per_block,
    valid=None, active=None, scale=None, softcap=None, p_round=no_round,
):
    """Pass 2 with final (m, l): acc += P.V and per-block mass (streaming_attention.py:264-352, :563-621)."""
    _fixed_fold(q, k, v, m, l, acc, valid, active, scale, softcap, p_round, block_mass, block_id_offset, tokens_per_block)


def fold_fixed_step(q, k, v, m, l, acc, valid=None, scale=None, softcap=None, p_round=no_round):
    """Tail fold with fixed (m, l), no mass, no active (streaming_attention.py:355-430, :624-665)."""
    _fixed_fold(q, k, v, m, l, acc, valid, None, scale, softcap, p_round, None, 0, BLOCK_KV)


def finalize(acc, l):
    """streaming_attention.py:668-670 before the dtype cast: acc / l."""
    with np.errstate(invalid="ignore", divide="ignore"):
        return (acc / l[..., None]).astype(np.float32)


def chunked_online_softmax(q, kv_chunks, scale=None):
    """Single-query online softmax over (key, value) chunks, bench/streaming_attention_prototype_mvp.py:13-52.

    q [H, D]; each chunk (k [H, C, D], v [H, C, D]) already expanded to H heads.
    """
    heads, head_dim = q.shape
    scale = 1.0 / (head_dim**0.5) if scale is None else scale
    m = np.full((heads, 1), -np.inf, np.float32)
    l = np.zeros((heads, 1), np.float32)
    acc = np.zeros((heads, head_dim), np.float32)
    for kc, vc in kv_chunks:
        s = np.einsum("hd,hcd->hc", q, kc).astype(np.float32) * np.float32(scale)
        m_new = np.maximum(m, s.max(axis=-1, keepdims=True))
        rescale = np.exp(m - m_new)
        acc = acc * rescale
        l = l * rescale
        p = np.exp(s - m_new)
        acc = acc + np.einsum("hc,hcd->hd", p, vc)
        l = l + p.sum(axis=-1, keepdims=True)
        m = m_new
    return acc / l
