"""HF past_key_values <-> KV block bookkeeping (the reference's pager_hf/kv_utils.py:8-61).

These functions only reshape and slice tensors; they run wherever the tensors live. The
decode hot path does not use them (the native store appends tokens in place); they serve
prefill-time block registration and the reference-layout block API.
"""
from __future__ import annotations

import torch


def get_legacy_past_key_values(outputs):
    """kv_utils.py:8-21: normalize past_key_values into a list of (key, value) per layer."""
    past = outputs.past_key_values
    if past is None:
        raise RuntimeError("Model did not return past_key_values.")
    if isinstance(past, (tuple, list)):
        return list(past)
    if hasattr(past, "key_cache") and hasattr(past, "value_cache"):
        return list(zip(past.key_cache, past.value_cache))
    layers = getattr(past, "layers", None)  # transformers >= 4.56 Cache objects
    if layers is not None:
        return [(layer.keys, layer.values) for layer in layers]
    raise TypeError(f"Unsupported past_key_values type: {type(past)!r}")


def split_full_blocks_and_tail(past_key_values, *, tokens_per_block: int):
    """kv_utils.py:24-35: (full_past, tail_past, full_tokens) at the last block boundary."""
    seq_len = past_key_values[0][0].shape[2]
    full_tokens = seq_len - seq_len % tokens_per_block
    full_past = [(k[:, :, :full_tokens].contiguous(), v[:, :, :full_tokens].contiguous()) for k, v in past_key_values]
    tail_past = [(k[:, :, full_tokens:].contiguous(), v[:, :, full_tokens:].contiguous()) for k, v in past_key_values]
    return full_past, tail_past, full_tokens


def extract_single_block_from_past(past_key_values, *, block_id: int, tokens_per_block: int):
    """kv_utils.py:38-53: one block across layers, as [num_layers, batch, block_len, kv_heads, head_dim]."""
    lo = block_id * tokens_per_block
    hi = lo + tokens_per_block
    keys = torch.stack([k[:, :, lo:hi].transpose(1, 2) for k, _ in past_key_values])
    values = torch.stack([v[:, :, lo:hi].transpose(1, 2) for _, v in past_key_values])
    return keys.contiguous(), values.contiguous()


def real_past_to_blocks(past_key_values, *, tokens_per_block: int):
    """kv_utils.py:56-61: every full block of past_key_values, in order."""
    n = past_key_values[0][0].shape[2] // tokens_per_block
    return [extract_single_block_from_past(past_key_values, block_id=i, tokens_per_block=tokens_per_block) for i in range(n)]
