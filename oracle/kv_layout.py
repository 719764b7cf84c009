"""CPU restatement of the reference's block split/extract (pager_hf/kv_utils.py:24-61): TEST ONLY.

TEST INFRASTRUCTURE. Only ``tests/`` may import it. numpy arrays stand in for tensors.
Pinned by tests/test_kv_utils.py with the reference's own assertions
(tests/test_kv_utils.py:41-131: 35 tokens -> 32 + 3 at 16 per block, exact multiples,
block 1 = tokens 16..31 transposed to [batch, block_len, kv_heads, head_dim]).
"""
from __future__ import annotations

import numpy as np


def split_full_blocks_and_tail(past, tokens_per_block):
    """kv_utils.py:24-35: past is a list of (key, value) [batch, kv_heads, seq, head_dim]."""
    full_tokens = (past[0][0].shape[2] // tokens_per_block) * tokens_per_block
    full = [(k[:, :, :full_tokens].copy(), v[:, :, :full_tokens].copy()) for k, v in past]
    tail = [(k[:, :, full_tokens:].copy(), v[:, :, full_tokens:].copy()) for k, v in past]
    return full, tail, full_tokens


def extract_single_block_from_past(past, block_id, tokens_per_block):
    """kv_utils.py:38-53: [num_layers, batch, block_len, kv_heads, head_dim] per key / value."""
    start = block_id * tokens_per_block
    end = start + tokens_per_block
    keys = np.stack([np.transpose(k[:, :, start:end], (0, 2, 1, 3)) for k, _ in past])
    values = np.stack([np.transpose(v[:, :, start:end], (0, 2, 1, 3)) for _, v in past])
    return keys, values


def real_past_to_blocks(past, tokens_per_block):
    """kv_utils.py:56-61."""
    n = past[0][0].shape[2] // tokens_per_block
    return [extract_single_block_from_past(past, b, tokens_per_block) for b in range(n)]
