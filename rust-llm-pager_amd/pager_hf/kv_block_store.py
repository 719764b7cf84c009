"""KV block store with the reference's API (pager_hf/kv_block_store.py:16-274) over the native pool.

A block is one ``tokens_per_block`` slice of every layer of one session, exchanged in the
reference layout ``key, value [num_layers, batch, block_len, kv_heads, head_dim]``. Storage
is the native store's layer-major HBM slot pools and block-id-addressed pinned host mirror
(see kv_pool.py); movement is asynchronous copy kernels on the caller's stream instead of
blocking, fully synchronized per-block ``.to()`` calls.

Kept from the reference: method names and return values, ascending-id ``apply_tiers`` with
tier 0 -> GPU and anything else -> CPU (ids past ``len(tiers)`` -> CPU), ``KeyError("Block N is
not on GPU.")``, ``ValueError`` for non-CUDA input or a duplicate id, the RAM-budget error
("ram_budget exceeded", logged and raised before the move) and warning ("ram_budget usage",
above 80%), incrementally tracked resident bytes and the KVBlockStoreStats counters (one copy
per block move, bytes = key + value of the whole block).

Different by design: blocks are fixed-shape (the pool has fixed-size slots), registered in
id order (the way PagedModel registers them, paged_model.py:1189-1231), and returned by
``get_any``/``get_gpu`` as copies. ``reorder_batch_rows`` (beam search) takes exactly one
source row per row: rows can be duplicated or dropped, but the batch size stays the same.
"""
from __future__ import annotations

import logging
from collections.abc import Mapping
from dataclasses import dataclass

import torch

from . import _native as N
from .kv_pool import NativeKVPool

logger = logging.getLogger(__name__)

_RAM_BUDGET_WARNING_THRESHOLD = 0.8  # kv_block_store.py:13


@dataclass
class KVBlockStoreStats:
    """kv_block_store.py:16-23."""

    gpu_to_cpu_bytes: int = 0
    cpu_to_gpu_bytes: int = 0
    gpu_to_cpu_copies: int = 0
    cpu_to_gpu_copies: int = 0
    gpu_to_cpu_sec: float = 0.0
    cpu_to_gpu_sec: float = 0.0


def tensor_nbytes(tensor: torch.Tensor) -> int:
    """kv_block_store.py:26-28."""
    return tensor.numel() * tensor.element_size()


def kv_nbytes(key: torch.Tensor, value: torch.Tensor) -> int:
    """kv_block_store.py:31-33."""
    return tensor_nbytes(key) + tensor_nbytes(value)


class _BlockView(Mapping):
    """Read-only {block_id: (key, value)} view of one tier; values are materialized copies."""

    def __init__(self, store: "KVBlockStore", gpu: bool):
        self._store = store
        self._gpu = gpu

    def _ids(self) -> list[int]:
        return self._store.gpu_block_ids() if self._gpu else self._store.cpu_block_ids()

    def __getitem__(self, block_id):
        if block_id not in set(self._ids()):
            raise KeyError(block_id)
        return self._store._read_block(block_id)

    def __iter__(self):
        return iter(self._ids())

    def __len__(self) -> int:
        return len(self._ids())

    def __contains__(self, block_id) -> bool:
        return block_id in set(self._ids())


class KVBlockStore:
    def __init__(
        self,
        tokens_per_block: int,
        ram_budget_bytes: int | None = None,
        *,
        pool: NativeKVPool | None = None,
        capacity_blocks: int = 1024,
        pool_blocks: int | None = None,
    ):
        self.tokens_per_block = tokens_per_block
        self.ram_budget_bytes = ram_budget_bytes
        self._pool = pool
        self._sid: int | None = None
        self._rows: int | None = None
        self._capacity_blocks = capacity_blocks
        self._pool_blocks = pool_blocks
        self.gpu_blocks = _BlockView(self, True)
        self.cpu_blocks = _BlockView(self, False)

    # -- native session ------------------------------------------------------------------
    def _ensure_session(self, key: torch.Tensor) -> None:
        if self._sid is not None:
            return
        if key.dim() != 5:
            raise ValueError("blocks are [num_layers, batch, block_len, kv_heads, head_dim] tensors")
        num_layers, rows, block_len, kv_heads, head_dim = key.shape
        if self._pool is None:
            self._pool = NativeKVPool(
                num_layers=num_layers,
                num_query_heads=kv_heads,
                num_kv_heads=kv_heads,
                head_dim=head_dim,
                tokens_per_block=block_len,
                dtype=key.dtype,
                device=key.device,
                pool_blocks=(self._pool_blocks or self._capacity_blocks) * rows,
                host_blocks=(self._capacity_blocks + 2) * rows,
                staging_blocks=max(rows, 64),
            )
        pool = self._pool
        if (pool.num_layers, pool.tokens_per_block, pool.num_kv_heads, pool.head_dim, pool.dtype) != (
            num_layers, block_len, kv_heads, head_dim, key.dtype
        ):
            raise ValueError("block shape/dtype does not match the store's pool geometry")
        pool.set_ram_budget(self.ram_budget_bytes)
        self._sid = pool.add_session(rows, self._capacity_blocks * block_len)
        self._rows = rows

    @property
    def pool(self) -> NativeKVPool | None:
        return self._pool

    @property
    def session_id(self) -> int | None:
        return self._sid

    def _read_block(self, block_id: int):
        return self._pool.get_block(self._sid, block_id, self._rows)

    def _block_bytes(self) -> int:
        return self._pool.block_bytes(self._sid)

    # -- reference API -------------------------------------------------------------------
    def put_gpu(self, block_id: int, key: torch.Tensor, value: torch.Tensor) -> None:
        """Register a block that already lives on the GPU (kv_block_store.py:58-67)."""
        if not key.is_cuda or not value.is_cuda:
            raise ValueError("put_gpu expects CUDA tensors.")
        if self._sid is not None and self.has_cpu(block_id):
            raise ValueError(f"Block {block_id} already exists on CPU.")
        if self._sid is not None and self.has_gpu(block_id):
            raise ValueError(f"Block {block_id} already exists on GPU.")
        if key.shape != value.shape:
            raise ValueError("key and value blocks must have the same shape")
        self._ensure_session(key)
        self._pool.put_block(self._sid, block_id, key.detach(), value.detach())

    def has_gpu(self, block_id: int) -> bool:
        return self._sid is not None and block_id in set(self._pool.block_ids(self._sid, True))

    def has_cpu(self, block_id: int) -> bool:
        return self._sid is not None and block_id in set(self._pool.block_ids(self._sid, False))

    def _current_tiers(self) -> list[int]:
        info = self._pool.session_info(self._sid)
        tiers = [1] * info[1]
        for b in self._pool.block_ids(self._sid, True):
            tiers[b] = 0
        return tiers

    def _raise_budget(self, block_id: int) -> None:
        _, cpu_bytes = self._pool.resident_bytes()
        projected = cpu_bytes + self._block_bytes()
        logger.error(
            "ram_budget exceeded: block %d would need %.2f MB, budget is %.2f MB.",
            block_id,
            projected / 1_000_000,
            self.ram_budget_bytes / 1_000_000,
        )
        raise RuntimeError(
            f"ram_budget exceeded: moving block {block_id} to CPU would need "
            f"{projected / 1_000_000:.2f} MB, budget is "
            f"{self.ram_budget_bytes / 1_000_000:.2f} MB. There is no SSD tier "
            "yet, so overflow can't be absorbed further; use a shorter context, "
            "a larger ram_budget, or a bigger tokens_per_block."
        )

    def _warn_offloads(self, to_cpu: list[int], cpu_bytes_before: int) -> None:
        if self.ram_budget_bytes is None or not to_cpu:
            return
        bb = self._block_bytes()
        for i, block_id in enumerate(to_cpu):
            projected = cpu_bytes_before + (i + 1) * bb
            if projected > _RAM_BUDGET_WARNING_THRESHOLD * self.ram_budget_bytes:
                logger.warning(
                    "ram_budget usage at %.0f%% after offloading block %d (%.2f MB of %.2f MB budget).",
                    100.0 * projected / self.ram_budget_bytes,
                    block_id,
                    projected / 1_000_000,
                    self.ram_budget_bytes / 1_000_000,
                )

    def _apply(self, tiers: list[int]) -> dict[str, list[int]]:
        _, cpu_before = self._pool.resident_bytes()
        to_gpu, to_cpu, rc, fail_block = self._pool.apply_tiers(self._sid, tiers)
        self._warn_offloads(to_cpu, cpu_before)
        if rc == N.nat.PGR_ERR_BUDGET:
            self._raise_budget(fail_block)
        return {"to_gpu": to_gpu, "to_cpu": to_cpu}

    def offload_to_cpu(self, block_id: int) -> None:
        """Move a block from GPU to CPU (kv_block_store.py:75-131)."""
        if not self.has_gpu(block_id):
            raise KeyError(f"Block {block_id} is not on GPU.")
        tiers = self._current_tiers()
        tiers[block_id] = 1
        self._apply(tiers)

    def load_to_gpu(self, block_id: int, device: torch.device | str) -> None:
        """Move a block from CPU to GPU (kv_block_store.py:133-163)."""
        if not self.has_cpu(block_id):
            raise KeyError(f"Block {block_id} is not on CPU.")
        if torch.device(device).type != "cuda":
            raise ValueError("load_to_gpu expects a CUDA device.")
        tiers = self._current_tiers()
        tiers[block_id] = 0
        self._apply(tiers)

    def ensure_gpu(self, block_id: int, device: torch.device | str) -> None:
        if self.has_gpu(block_id):
            return
        self.load_to_gpu(block_id, device)

    def ensure_cpu(self, block_id: int) -> None:
        if self.has_cpu(block_id):
            return
        self.offload_to_cpu(block_id)

    def resident_gpu_bytes(self) -> int:
        return 0 if self._sid is None else self._pool.resident_bytes()[0]

    def resident_cpu_bytes(self) -> int:
        return 0 if self._sid is None else self._pool.resident_bytes()[1]

    def gpu_block_ids(self) -> list[int]:
        return [] if self._sid is None else self._pool.block_ids(self._sid, True)

    def cpu_block_ids(self) -> list[int]:
        return [] if self._sid is None else self._pool.block_ids(self._sid, False)

    @property
    def stats(self) -> KVBlockStoreStats:
        if self._pool is None:
            return KVBlockStoreStats()
        s = self._pool.stats()
        return KVBlockStoreStats(
            gpu_to_cpu_bytes=int(s["gpu_to_cpu_bytes"]),
            cpu_to_gpu_bytes=int(s["cpu_to_gpu_bytes"]),
            gpu_to_cpu_copies=int(s["gpu_to_cpu_copies"]),
            cpu_to_gpu_copies=int(s["cpu_to_gpu_copies"]),
            gpu_to_cpu_sec=float(s["gpu_to_cpu_sec"]),
            cpu_to_gpu_sec=float(s["cpu_to_gpu_sec"]),
        )

    def summary(self) -> dict:
        """kv_block_store.py:191-204."""
        st = self.stats
        return {
            "gpu_blocks": len(self.gpu_block_ids()),
            "cpu_blocks": len(self.cpu_block_ids()),
            "resident_gpu_bytes": self.resident_gpu_bytes(),
            "resident_cpu_bytes": self.resident_cpu_bytes(),
            "gpu_to_cpu_bytes": st.gpu_to_cpu_bytes,
            "cpu_to_gpu_bytes": st.cpu_to_gpu_bytes,
            "gpu_to_cpu_copies": st.gpu_to_cpu_copies,
            "cpu_to_gpu_copies": st.cpu_to_gpu_copies,
            "gpu_to_cpu_sec": st.gpu_to_cpu_sec,
            "cpu_to_gpu_sec": st.cpu_to_gpu_sec,
        }

    def apply_tiers(self, tiers: list[int], device: torch.device | str) -> dict[str, list[int]]:
        """Move each block to the tier the pager assigned (kv_block_store.py:206-227)."""
        if self._sid is None:
            return {"to_gpu": [], "to_cpu": []}
        if torch.device(device).type != "cuda":
            raise ValueError("apply_tiers expects a CUDA device.")
        return self._apply([int(t) for t in tiers])

    def reorder_batch_rows(self, new_row_indices: list[int]) -> None:
        """kv_block_store.py:229-254: new row i takes old row new_row_indices[i]'s data in
        every block, on whichever tier the block lives, without changing the tier. An index
        listed twice duplicates that row; one never listed drops it. The native store keeps
        the batch size, so exactly one index per row is required."""
        if self._sid is None:
            return
        idx = [int(i) for i in new_row_indices]
        if len(idx) != self._rows:
            raise ValueError(f"reorder_batch_rows needs one index per row ({self._rows}), got {len(idx)}")
        if any(i < 0 or i >= self._rows for i in idx):
            raise IndexError(f"row index out of range for a batch of {self._rows}: {idx}")
        self._pool.reorder_rows(self._sid, idx)

    def get_gpu(self, block_id: int) -> tuple[torch.Tensor, torch.Tensor]:
        if not self.has_gpu(block_id):
            raise KeyError(f"Block {block_id} is not on GPU.")
        return self._read_block(block_id)

    def get_any(self, block_id: int) -> tuple[torch.Tensor, torch.Tensor]:
        """A block's (key, value) wherever it lives, without moving it (kv_block_store.py:262-274)."""
        if self.has_gpu(block_id) or self.has_cpu(block_id):
            return self._read_block(block_id)
        raise KeyError(f"Block {block_id} is not on GPU or CPU.")
