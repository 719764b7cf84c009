"""Streaming single-token GQA decode attention: the reference's operator API over HIP kernels.

Same six functions, signatures, defaults and in-place semantics as the reference module
pager_hf/streaming_attention.py:444-670. Each call launches the CDNA4 kernels of libpgr.so
(split-K MFMA fold + merge) on torch's current stream; there is no Python or CPU fallback.

Conventions kept from the reference:
  * q [batch, num_query_heads, head_dim]; k, v [batch, num_kv_heads, chunk_tokens, head_dim]
    (made contiguous here, as the reference's wrappers do, :477-480, :495-497);
  * m, l [batch, num_query_heads] and acc [batch, num_query_heads, head_dim] are fp32 and are
    updated in place; block_mass [batch, num_query_heads, max_blocks] fp32, written in place;
  * valid: optional [batch, chunk_tokens] 0/1 (None = all valid); active: optional [batch]
    0/1 (None = all active; a row with active=0 is left bit-for-bit untouched);
  * scale defaults to 1/sqrt(head_dim); softcap None or 0.0 disables c*tanh(s/c);
  * NotImplementedError when num_query_heads / num_kv_heads > 16 (:69-74).

Differences, by design: p is rounded to the K/V dtype before P.V exactly as the reference
does, but the chunk is folded by many workgroups in parallel and merged, so fp32 results
differ from the reference's sequential fold in the last bits. q/k/v may be float16, bfloat16
or float32, and head_dim one of 8, 16, 32, 64, 128, 256 (NotImplementedError otherwise);
16-bit inputs at head_dim 32/64/128 run the MFMA kernel, the rest a VALU kernel. The
reference zero-pads Q and K to 16 columns below head_dim 16 so that tl.dot applies
(:56-66, :125-133); the dot products are the same without the padding. A masked position
contributes exactly zero in every kernel, also when the fixed max m is -inf.
"""
from __future__ import annotations

import torch

from . import _native as N

_M_TILE = 16  # streaming_attention.py:55: query heads packed per KV head
_QKV_CODES = {torch.float16: N.nat.DTYPE_F16, torch.bfloat16: N.nat.DTYPE_BF16, torch.float32: N.nat.DTYPE_F32}


def _validate_n_rep(n_rep: int) -> None:
    """streaming_attention.py:69-74."""
    if n_rep > _M_TILE:
        raise NotImplementedError(
            f"streaming attention's GQA query-head packing supports n_rep up to {_M_TILE}, got {n_rep}. "
            "This architecture's query/KV head ratio is wider than any currently supported model."
        )


def _state(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} is updated in place and must be contiguous")
    return t


def _mask(t: torch.Tensor | None, shape: tuple, name: str) -> torch.Tensor | None:
    if t is None:
        return None
    if tuple(t.shape) != shape:
        raise ValueError(f"{name} must have shape {shape}, got {tuple(t.shape)}")
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


def _prep(q, k, v, m, l, acc, valid, active, scale):
    batch, num_query_heads, head_dim = q.shape
    kb, num_kv_heads, total_tokens, kd = k.shape
    if kb != batch or kd != head_dim:
        raise ValueError(f"k shape {tuple(k.shape)} does not match q shape {tuple(q.shape)}")
    if v is not None and tuple(v.shape) != tuple(k.shape):
        raise ValueError(f"v shape {tuple(v.shape)} differs from k shape {tuple(k.shape)}")
    if num_query_heads % num_kv_heads != 0:
        raise ValueError("num_query_heads must be a multiple of num_kv_heads")
    n_rep = num_query_heads // num_kv_heads
    _validate_n_rep(n_rep)
    if k.dtype != q.dtype or (v is not None and v.dtype != q.dtype):
        raise TypeError("q, k and v must share one dtype")
    if q.dtype not in _QKV_CODES:
        raise NotImplementedError(f"streaming attention takes float16, bfloat16 or float32 q/k/v, got {q.dtype}")
    code = _QKV_CODES[q.dtype]
    device = N.require_cuda(q, k, v, m, l, acc, valid, active)
    for t, name in ((m, "m"), (l, "l")):
        _state(t, name)
        if tuple(t.shape) != (batch, num_query_heads):
            raise ValueError(f"{name} must have shape {(batch, num_query_heads)}")
    if acc is not None:
        _state(acc, "acc")
        if tuple(acc.shape) != (batch, num_query_heads, head_dim):
            raise ValueError(f"acc must have shape {(batch, num_query_heads, head_dim)}")
    valid = _mask(valid, (batch, total_tokens), "valid")
    active = _mask(active, (batch,), "active")
    if scale is None:
        scale = 1.0 / (head_dim**0.5)
    q = q.contiguous()
    k = k.contiguous()
    v = v.contiguous() if v is not None else None
    return batch, num_query_heads, num_kv_heads, total_tokens, head_dim, code, device, q, k, v, valid, active, scale


def _workspace(device, batch, hq, hkv, tokens, head_dim, mode, tpb=16):
    nbytes = N.lib().pgr_attn_workspace_bytes(batch, hq, hkv, tokens, head_dim, mode, tpb)
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device), nbytes


def streaming_attention_state_init(batch_size: int, num_query_heads: int, head_dim: int, device: torch.device):
    """Fresh online-softmax accumulator state, before any KV chunk has been folded in (:444-449):
    m = -inf, l = 0, acc = 0 in fp32, written by one native launch."""
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("streaming attention expects CUDA (HIP) tensors")
    m = torch.empty((batch_size, num_query_heads), dtype=torch.float32, device=device)
    l = torch.empty((batch_size, num_query_heads), dtype=torch.float32, device=device)
    acc = torch.empty((batch_size, num_query_heads, head_dim), dtype=torch.float32, device=device)
    N.nat.check(
        N.lib().pgr_attn_state_init(m.data_ptr(), l.data_ptr(), acc.data_ptr(), batch_size * num_query_heads,
                                    head_dim, N.stream_of(device)),
        "streaming_attention_state_init",
    )
    return m, l, acc


def streaming_attention_step(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    m: torch.Tensor,
    l: torch.Tensor,
    acc: torch.Tensor,
    valid: torch.Tensor | None = None,
    active: torch.Tensor | None = None,
    scale: float | None = None,
    softcap: float | None = None,
) -> None:
    """Fold one KV chunk into the running (m, l, acc) state, in place (:452-513)."""
    b, hq, hkv, tc, d, code, dev, q, k, v, valid, active, scale = _prep(q, k, v, m, l, acc, valid, active, scale)
    if tc == 0 or b == 0:
        return
    ws, nbytes = _workspace(dev, b, hq, hkv, tc, d, N.nat.MODE_FOLD)
    N.nat.check(
        N.lib().pgr_attn_step(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), N.ptr(valid), N.ptr(active), m.data_ptr(), l.data_ptr(),
            acc.data_ptr(), b, hq, hkv, tc, d, code, float(scale), float(softcap or 0.0), ws.data_ptr(), nbytes,
            N.stream_of(dev),
        ),
        "streaming_attention_step",
    )


def streaming_attention_stats_step(
    q: torch.Tensor,
    k: torch.Tensor,
    m: torch.Tensor,
    l: torch.Tensor,
    valid: torch.Tensor | None = None,
    active: torch.Tensor | None = None,
    scale: float | None = None,
    softcap: float | None = None,
) -> None:
    """Pass 1: fold one KV chunk's K into running (m, l) only (:516-560)."""
    b, hq, hkv, tc, d, code, dev, q, k, _, valid, active, scale = _prep(q, k, None, m, l, None, valid, active, scale)
    if tc == 0 or b == 0:
        return
    ws, nbytes = _workspace(dev, b, hq, hkv, tc, d, N.nat.MODE_STATS)
    N.nat.check(
        N.lib().pgr_attn_stats_step(
            q.data_ptr(), k.data_ptr(), N.ptr(valid), N.ptr(active), m.data_ptr(), l.data_ptr(), b, hq, hkv, tc, d,
            code, float(scale), float(softcap or 0.0), ws.data_ptr(), nbytes, N.stream_of(dev),
        ),
        "streaming_attention_stats_step",
    )


def streaming_attention_accumulate_step(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    m: torch.Tensor,
    l: torch.Tensor,
    acc: torch.Tensor,
    block_mass: torch.Tensor,
    block_id_offset: int,
    tokens_per_block: int,
    valid: torch.Tensor | None = None,
    active: torch.Tensor | None = None,
    scale: float | None = None,
    softcap: float | None = None,
) -> None:
    """Pass 2: fold one block-aligned KV group into acc and write its per-block mass (:563-621)."""
    b, hq, hkv, tc, d, code, dev, q, k, v, valid, active, scale = _prep(q, k, v, m, l, acc, valid, active, scale)
    _state(block_mass, "block_mass")
    N.require_cuda(block_mass)
    if block_mass.dim() != 3 or tuple(block_mass.shape[:2]) != (b, hq):
        raise ValueError(f"block_mass must have shape ({b}, {hq}, max_blocks)")
    max_blocks = block_mass.shape[2]
    if tc == 0 or b == 0:
        return
    ws, nbytes = _workspace(dev, b, hq, hkv, tc, d, N.nat.MODE_ACCUMULATE, tokens_per_block)
    N.nat.check(
        N.lib().pgr_attn_accumulate_step(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), N.ptr(valid), N.ptr(active), m.data_ptr(), l.data_ptr(),
            acc.data_ptr(), block_mass.data_ptr(), max_blocks, int(block_id_offset), int(tokens_per_block), b, hq,
            hkv, tc, d, code, float(scale), float(softcap or 0.0), ws.data_ptr(), nbytes, N.stream_of(dev),
        ),
        "streaming_attention_accumulate_step",
    )


def streaming_attention_fold_fixed_step(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    m: torch.Tensor,
    l: torch.Tensor,
    acc: torch.Tensor,
    valid: torch.Tensor | None = None,
    scale: float | None = None,
    softcap: float | None = None,
) -> None:
    """Pass 2 fold for a non-block chunk (the tail): accumulate acc only, no mass (:624-665)."""
    b, hq, hkv, tc, d, code, dev, q, k, v, valid, _, scale = _prep(q, k, v, m, l, acc, valid, None, scale)
    if tc == 0 or b == 0:
        return
    ws, nbytes = _workspace(dev, b, hq, hkv, tc, d, N.nat.MODE_FOLD_FIXED)
    N.nat.check(
        N.lib().pgr_attn_fold_fixed_step(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), N.ptr(valid), m.data_ptr(), l.data_ptr(), acc.data_ptr(), b,
            hq, hkv, tc, d, code, float(scale), float(softcap or 0.0), ws.data_ptr(), nbytes, N.stream_of(dev),
        ),
        "streaming_attention_fold_fixed_step",
    )


_FINALIZE_CODES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def streaming_attention_finalize(acc: torch.Tensor, l: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """(acc / l) cast to dtype, once every chunk has been folded in (:668-670)."""
    if dtype not in _FINALIZE_CODES:
        raise NotImplementedError(f"finalize supports float16, bfloat16 and float32 outputs, got {dtype}")
    dev = N.require_cuda(acc, l)
    acc = _state(acc.contiguous(), "acc")
    l = _state(l.contiguous(), "l")
    if tuple(l.shape) != tuple(acc.shape[:-1]):
        raise ValueError("l must have acc's shape without the last dimension")
    out = torch.empty(acc.shape, dtype=dtype, device=dev)
    rows = l.numel()
    N.nat.check(
        N.lib().pgr_attn_finalize(acc.data_ptr(), l.data_ptr(), out.data_ptr(), rows, acc.shape[-1],
                                  _FINALIZE_CODES[dtype], N.stream_of(dev)),
        "streaming_attention_finalize",
    )
    return out
