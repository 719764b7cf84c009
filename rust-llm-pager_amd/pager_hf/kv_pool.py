"""Python handle of the native paged KV store (``pgr_kv_*`` in include/pgr.h).

One NativeKVPool owns, for every layer, an HBM slot pool and a pinned host mirror (plus an HBM
staging ring in the staged mode, or a ring of HBM buffers in the mirror mode), and the
per-session block tables. ``stream_mode="direct"`` (default) has the decode kernel read
host-resident blocks in place over the host link; ``"staged"`` copies them into the staging
ring first (and, when one buffer holds a layer's host blocks, queues the next layer's copies
under the current layer); ``"mirror"`` copies each layer's host share of the step by DMA on a
side stream into a ring of ``staging_buffers`` HBM buffers (layer l into buffer l % n, once
layer l - n has finished reading it), and the decode kernel of a layer waits for that layer's
copies and reads the buffer (or the host in place, if they have not landed within its bounded
wait). Sessions are groups of rows that share one placement (the reference's
one-PagedModel-per-session model, kv_block_store.py:36-56).
"""
from __future__ import annotations

import atexit
import ctypes
import weakref

import torch

from . import _native as N

nat = N.nat


_LIVE_POOLS: "weakref.WeakSet[NativeKVPool]" = weakref.WeakSet()


@atexit.register
def _close_live_pools() -> None:
    # Release native stores while the HIP runtime is still up (before interpreter teardown).
    for pool in list(_LIVE_POOLS):
        try:
            pool.close()
        except Exception:
            pass


def _i64_array(n: int):
    return (ctypes.c_int64 * max(n, 1))()


class NativeKVPool:
    def __init__(
        self,
        *,
        num_layers: int,
        num_query_heads: int,
        num_kv_heads: int,
        head_dim: int,
        tokens_per_block: int,
        dtype: torch.dtype,
        device: torch.device | str = "cuda",
        pool_blocks: int,
        host_blocks: int,
        staging_blocks: int = 2048,
        staging_buffers: int = 2,
        blocks_per_workgroup: int = 32,
        target_workgroups: int = 0,
        stream_mode: str = "direct",
    ):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("NativeKVPool needs a CUDA (HIP) device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.num_layers = num_layers
        self.num_query_heads = num_query_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.tokens_per_block = tokens_per_block
        self.dtype = dtype
        self.lib = N.lib()
        modes = {"direct": nat.STREAM_DIRECT, "staged": nat.STREAM_STAGED, "mirror": nat.STREAM_MIRROR}
        if stream_mode not in modes:
            raise ValueError(f"stream_mode must be one of {sorted(modes)}, got {stream_mode!r}")
        self.stream_mode = stream_mode
        cfg = nat.KVConfig(
            num_layers=num_layers,
            kv_heads=num_kv_heads,
            query_heads=num_query_heads,
            head_dim=head_dim,
            tokens_per_block=tokens_per_block,
            dtype=N.dtype_code(dtype),
            pool_slots=pool_blocks,
            host_records=host_blocks,
            staging_slots=staging_blocks,
            staging_buffers=staging_buffers,
            blocks_per_workgroup=blocks_per_workgroup,
            target_workgroups=target_workgroups,
            stream_mode=modes[stream_mode],
        )
        with torch.cuda.device(self.device):
            handle = self.lib.pgr_kv_create(ctypes.byref(cfg))
        if not handle:
            raise MemoryError(f"pgr_kv_create failed: {nat.last_error()}")
        self.handle = handle
        _LIVE_POOLS.add(self)
        self.record_bytes = 2 * num_kv_heads * tokens_per_block * head_dim * torch.tensor([], dtype=dtype).element_size()

    # -- lifetime ------------------------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "handle", None):
            with torch.cuda.device(self.device):
                self.lib.pgr_kv_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _stream(self) -> int:
        return N.stream_of(self.device)

    def _call(self, what: str, fn, *args):
        with torch.cuda.device(self.device):
            return nat.check(fn(self.handle, *args), what)

    # -- sessions ------------------------------------------------------------------------
    def add_session(self, rows: int, capacity_tokens: int, lo=None) -> int:
        arr = None
        if lo is not None:
            arr = (ctypes.c_int32 * rows)(*[int(x) for x in lo])
        return self._call("add_session", self.lib.pgr_kv_add_session, rows, capacity_tokens, arr)

    def remove_session(self, sid: int) -> None:
        self._call("remove_session", self.lib.pgr_kv_remove_session, sid)

    def set_lo(self, sid: int, lo) -> None:
        arr = (ctypes.c_int32 * len(lo))(*[int(x) for x in lo])
        self._call("set_lo", self.lib.pgr_kv_set_lo, sid, arr)

    def step_signature(self) -> tuple[int, ...]:
        """Launch arguments of the open step (workspace pointers, grids, mass stride): a graph
        captured in one step may be replayed in any later step with the same signature."""
        n = nat.check(self.lib.pgr_kv_step_signature(self.handle, None, 0), "step_signature")
        arr = _i64_array(n)
        nat.check(self.lib.pgr_kv_step_signature(self.handle, arr, n), "step_signature")
        return tuple(arr[:n])

    def step_replayed(self) -> None:
        """The open step's launches were replayed from a captured graph on the current
        stream: guard the step's plan buffer until that replay has run."""
        self._call("step_replayed", self.lib.pgr_kv_step_replayed, self._stream())

    def reorder_rows(self, sid: int, src_rows) -> None:
        """New row r of session `sid` takes old row src_rows[r]'s K/V history (beam search)."""
        arr = (ctypes.c_int32 * len(src_rows))(*[int(x) for x in src_rows])
        self._call("reorder_rows", self.lib.pgr_kv_reorder_rows, sid, arr, len(src_rows), self._stream())

    def set_length(self, sid: int, n_tokens: int) -> None:
        self._call("set_length", self.lib.pgr_kv_set_length, sid, n_tokens)

    def import_tokens(self, sid: int, row: int, layer: int, k: torch.Tensor, v: torch.Tensor, n_tokens: int) -> None:
        """k, v [Hkv, n_src, D] on this device (n_src >= n_tokens)."""
        k = k.contiguous()
        v = v.contiguous()
        self._check_kv(k, v)
        self._call("import", self.lib.pgr_kv_import, sid, row, layer, k.data_ptr(), v.data_ptr(), k.shape[1],
                   n_tokens, self._stream())

    def export_tokens(self, sid: int, row: int, layer: int, n_tokens: int):
        k = torch.empty((self.num_kv_heads, n_tokens, self.head_dim), dtype=self.dtype, device=self.device)
        v = torch.empty_like(k)
        if n_tokens:
            self._call("export", self.lib.pgr_kv_export, sid, row, layer, k.data_ptr(), v.data_ptr(), n_tokens,
                       self._stream())
        return k, v

    def put_block(self, sid: int, block_id: int, key: torch.Tensor, value: torch.Tensor) -> None:
        key = key.contiguous()
        value = value.contiguous()
        self._check_kv(key, value)
        self._call("put_block", self.lib.pgr_kv_put_block, sid, block_id, key.data_ptr(), value.data_ptr(),
                   self._stream())

    def get_block(self, sid: int, block_id: int, rows: int):
        shape = (self.num_layers, rows, self.tokens_per_block, self.num_kv_heads, self.head_dim)
        key = torch.empty(shape, dtype=self.dtype, device=self.device)
        value = torch.empty_like(key)
        self._call("get_block", self.lib.pgr_kv_get_block, sid, block_id, key.data_ptr(), value.data_ptr(),
                   self._stream())
        return key, value

    def _check_kv(self, k: torch.Tensor, v: torch.Tensor) -> None:
        if k.device != self.device or v.device != self.device:
            raise ValueError(f"tensors must be on {self.device}")
        if k.dtype != self.dtype or v.dtype != self.dtype:
            raise TypeError(f"tensors must be {self.dtype}")

    # -- placement -----------------------------------------------------------------------
    def apply_tiers(self, sid: int, tiers) -> tuple[list[int], list[int], int, int]:
        """Returns (to_gpu, to_cpu, status, fail_block); status PGR_ERR_BUDGET is not raised here."""
        n = len(tiers)
        tarr = (ctypes.c_uint8 * max(n, 1))(*[int(t) for t in tiers])
        info = self.session_info(sid)
        cap = info[1] + 1
        to_gpu, to_cpu = _i64_array(cap), _i64_array(cap)
        n_gpu, n_cpu, fail_block = ctypes.c_int64(0), ctypes.c_int64(0), ctypes.c_int64(-1)
        with torch.cuda.device(self.device):
            rc = self.lib.pgr_kv_apply_tiers(
                self.handle, sid, tarr, n, to_gpu, ctypes.byref(n_gpu), to_cpu, ctypes.byref(n_cpu),
                ctypes.byref(fail_block), self._stream(),
            )
        if rc not in (nat.PGR_OK, nat.PGR_ERR_BUDGET):
            nat.check(rc, "apply_tiers")
        return list(to_gpu[: n_gpu.value]), list(to_cpu[: n_cpu.value]), rc, fail_block.value

    def set_ram_budget(self, nbytes: int | None) -> None:
        self._call("set_ram_budget", self.lib.pgr_kv_set_ram_budget, -1 if nbytes is None else int(nbytes))

    # -- decode ---------------------------------------------------------------------------
    def begin_step(self, sids) -> None:
        arr = (ctypes.c_int32 * max(len(sids), 1))(*sids)
        self._call("begin_step", self.lib.pgr_kv_begin_step, arr, len(sids), self._stream())

    def decode_layer(self, layer: int, q, k_new, v_new, out, mass_accum=None, scale=None, softcap=None,
                     window=None) -> None:
        if scale is None:
            scale = 1.0 / (self.head_dim**0.5)
        stride = mass_accum.shape[1] if mass_accum is not None else 0
        self._call(
            "decode_layer", self.lib.pgr_kv_decode_layer, layer, q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(),
            out.data_ptr(), N.ptr(mass_accum), stride, float(scale), float(softcap or 0.0), int(window or 0),
            self._stream(),
        )

    def attach_pager(self, sid: int, pager_handle: int, scores_from_mass: bool) -> None:
        self._call("attach_pager", self.lib.pgr_kv_attach_pager, sid, pager_handle, int(scores_from_mass))

    def end_step_place(self, n_sessions: int, mass_accum, num_layers: int, moves_cap: int, scores_cap: int):
        """Closes the step and runs the native placement glue. Returns (completed, counts[n, 5],
        moves, scores) with counts rows {new block id or -1, n to HBM, n to host, fail block, n scores}."""
        completed = (ctypes.c_int32 * max(n_sessions, 1))()
        n_done = ctypes.c_int32(0)
        counts = (ctypes.c_int64 * (5 * max(n_sessions, 1)))()
        moves = _i64_array(moves_cap)
        scores = (ctypes.c_double * max(scores_cap, 1))()
        stride = mass_accum.shape[1] if mass_accum is not None else 0
        with torch.cuda.device(self.device):
            rc = self.lib.pgr_kv_end_step_place(
                self.handle, N.ptr(mass_accum), stride, num_layers, completed, ctypes.byref(n_done), counts, moves,
                moves_cap, scores if scores_cap else None, scores_cap, self._stream(),
            )
        rows = [tuple(counts[5 * i: 5 * i + 5]) for i in range(n_sessions)]
        if rc not in (nat.PGR_OK, nat.PGR_ERR_BUDGET):
            nat.check(rc, "end_step_place")
        return rc, list(completed[: n_done.value]), rows, moves, scores

    def end_step(self, n_sessions: int) -> list[int]:
        arr = (ctypes.c_int32 * max(n_sessions, 1))()
        n = ctypes.c_int32(0)
        self._call("end_step", self.lib.pgr_kv_end_step, arr, ctypes.byref(n))
        return list(arr[: n.value])

    # -- introspection ----------------------------------------------------------------------
    def session_info(self, sid: int) -> tuple[int, int, int, int]:
        """(n_tokens, n_full_blocks, gpu_blocks, cpu_blocks)."""
        info = (ctypes.c_int64 * 4)()
        nat.check(self.lib.pgr_kv_session_info(self.handle, sid, info), "session_info")
        return tuple(int(x) for x in info)

    def block_ids(self, sid: int, gpu: bool) -> list[int]:
        n = nat.check(self.lib.pgr_kv_block_ids(self.handle, sid, int(gpu), None, 0), "block_ids")
        arr = _i64_array(n)
        nat.check(self.lib.pgr_kv_block_ids(self.handle, sid, int(gpu), arr, n), "block_ids")
        return list(arr[:n])

    def step_host_blocks(self, seq: int) -> list[int]:
        n = nat.check(self.lib.pgr_kv_step_host_blocks(self.handle, seq, None, 0), "step_host_blocks")
        arr = _i64_array(n)
        nat.check(self.lib.pgr_kv_step_host_blocks(self.handle, seq, arr, n), "step_host_blocks")
        return list(arr[:n])

    def step_stats(self) -> dict:
        s = nat.KVStepStats()
        nat.check(self.lib.pgr_kv_step_stats(self.handle, ctypes.byref(s)), "step_stats")
        return {name: getattr(s, name) for name, _ in nat.KVStepStats._fields_}

    def stats(self) -> dict:
        s = nat.KVStats()
        nat.check(self.lib.pgr_kv_stats(self.handle, ctypes.byref(s)), "stats")
        return {name: getattr(s, name) for name, _ in nat.KVStats._fields_}

    def resident_bytes(self) -> tuple[int, int]:
        g, c = ctypes.c_int64(0), ctypes.c_int64(0)
        nat.check(self.lib.pgr_kv_resident_bytes(self.handle, ctypes.byref(g), ctypes.byref(c)), "resident_bytes")
        return g.value, c.value

    def hbm_bytes(self) -> dict:
        """Device memory the store holds: {pool, mirror, staging, workspace, total} in bytes."""
        arr = (ctypes.c_int64 * 5)()
        nat.check(self.lib.pgr_kv_hbm_bytes(self.handle, arr), "hbm_bytes")
        return dict(zip(("pool", "mirror", "staging", "workspace", "total"), (int(x) for x in arr)))

    def block_bytes(self, sid: int) -> int:
        b = ctypes.c_int64(0)
        nat.check(self.lib.pgr_kv_block_bytes(self.handle, sid, ctypes.byref(b)), "block_bytes")
        return b.value

    def set_timing(self, on: bool) -> None:
        nat.check(self.lib.pgr_kv_set_timing(self.handle, int(on)), "set_timing")

    def kernel_time(self) -> tuple[float, int, int]:
        """(milliseconds, launches, K/V bytes read) of timed attention launches since the last call."""
        ms, launches, nbytes = ctypes.c_double(0), ctypes.c_int64(0), ctypes.c_int64(0)
        with torch.cuda.device(self.device):
            nat.check(self.lib.pgr_kv_kernel_time(self.handle, ctypes.byref(ms), ctypes.byref(launches),
                                                  ctypes.byref(nbytes)), "kernel_time")
        return ms.value, launches.value, nbytes.value

    def bench_attention(self, q, k_new, v_new, reps: int = 1, scale=None, softcap=None) -> tuple[float, int]:
        """Measurement only: the open step's attention launches for every layer, `reps` times,
        back to back between two events (pgr_kv_bench_attention). q, k_new and v_new are lists
        with each layer's inputs of the step (the launches write each layer's current token
        again). Returns (microseconds per launch, K/V bytes per launch)."""
        if not (len(q) == len(k_new) == len(v_new) == self.num_layers):
            raise ValueError(f"bench_attention needs {self.num_layers} q, k_new and v_new tensors (one per layer)")
        if scale is None:
            scale = 1.0 / (self.head_dim**0.5)

        def ptrs(ts):
            return (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])

        us, nbytes = ctypes.c_double(0), ctypes.c_int64(0)
        self._call("bench_attention", self.lib.pgr_kv_bench_attention, ptrs(q), ptrs(k_new), ptrs(v_new),
                   float(scale), float(softcap or 0.0), int(reps), ctypes.byref(us), ctypes.byref(nbytes),
                   self._stream())
        return us.value, nbytes.value

    def copy_time(self) -> tuple[float, int, int]:
        """(milliseconds, layer copy groups, bytes) of the mirror mode's DMA copies timed since the last call."""
        ms, n, nbytes = ctypes.c_double(0), ctypes.c_int64(0), ctypes.c_int64(0)
        with torch.cuda.device(self.device):
            nat.check(self.lib.pgr_kv_copy_time(self.handle, ctypes.byref(ms), ctypes.byref(n), ctypes.byref(nbytes)),
                      "copy_time")
        return ms.value, n.value, nbytes.value

    def sync(self) -> None:
        self._call("sync", self.lib.pgr_kv_sync)
