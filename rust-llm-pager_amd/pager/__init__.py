"""Drop-in for the reference's ``pager`` extension module (pager/src/lib.rs:69-74).

``PyPager`` and ``Metrics`` keep the reference's constructor signature, defaults, method
names and argument conversion rules (PyO3 0.21: unsigned ints reject negatives with
OverflowError and floats with TypeError; attention scores are read as f64 and rounded to
f32). The placement logic is the native C++ restatement of pager/src/core.rs in libpgr.so,
reached through the C ABI (include/pgr.h, ``pgr_pager_*``).
"""
from __future__ import annotations

import array
import ctypes
import operator
import os
import sys
import threading

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import _pgr_native as _nat  # noqa: E402

__all__ = ["PyPager", "Metrics"]

_U64_MAX = (1 << 64) - 1
_U32_MAX = (1 << 32) - 1


def _unsigned(value, bits_max: int, name: str) -> int:
    if isinstance(value, float):
        raise TypeError(f"argument '{name}': 'float' object cannot be interpreted as an integer")
    try:
        v = operator.index(value)
    except TypeError:
        raise TypeError(f"argument '{name}': '{type(value).__name__}' object cannot be interpreted as an integer")
    if v < 0:
        raise OverflowError(f"argument '{name}': can't convert negative int to unsigned")
    if v > bits_max:
        raise OverflowError(f"argument '{name}': int too big to convert")
    return v


def _f32(value, name: str) -> float:
    if isinstance(value, (str, bytes)):
        raise TypeError(f"argument '{name}': must be real number, not {type(value).__name__}")
    try:
        return float(value)
    except TypeError:
        raise TypeError(f"argument '{name}': must be real number, not {type(value).__name__}")


class Metrics:
    """Snapshot of the pager metrics (metrics.rs:4-27); read-only attributes."""

    __slots__ = (
        "_tokens",
        "_vram_peak",
        "_ram_peak",
        "_swap_vram_ram",
        "_swap_ram_ssd",
        "_attention_mass_total",
        "_attention_mass_vram",
    )

    def __init__(self, *args, **kwargs):
        raise TypeError("No constructor defined")

    @classmethod
    def _from_native(cls, m: _nat.PagerMetrics) -> "Metrics":
        self = object.__new__(cls)
        self._tokens = int(m.tokens)
        self._vram_peak = int(m.vram_peak)
        self._ram_peak = int(m.ram_peak)
        self._swap_vram_ram = int(m.swap_vram_ram)
        self._swap_ram_ssd = int(m.swap_ram_ssd)
        self._attention_mass_total = float(m.attention_mass_total)
        self._attention_mass_vram = float(m.attention_mass_vram)
        return self

    tokens = property(lambda self: self._tokens)
    vram_peak = property(lambda self: self._vram_peak)
    ram_peak = property(lambda self: self._ram_peak)
    swap_vram_ram = property(lambda self: self._swap_vram_ram)
    swap_ram_ssd = property(lambda self: self._swap_ram_ssd)
    attention_mass_total = property(lambda self: self._attention_mass_total)
    attention_mass_vram = property(lambda self: self._attention_mass_vram)

    def __repr__(self) -> str:
        return (
            f"Metrics(tokens={self._tokens}, vram_peak={self._vram_peak}, ram_peak={self._ram_peak}, "
            f"swap_vram_ram={self._swap_vram_ram}, swap_ram_ssd={self._swap_ram_ssd}, "
            f"attention_mass_total={self._attention_mass_total}, attention_mass_vram={self._attention_mass_vram})"
        )


class PyPager:
    """Block placement policy (lib.rs:9-67 over core.rs), backed by the native C++ core.

    PyPager(vram, ram, recent, rebalance_interval=32, promote_margin=0.10,
            ram_promote_margin=0.20, policy="heavy_hitter")
    """

    def __init__(
        self,
        vram,
        ram,
        recent,
        rebalance_interval=32,
        promote_margin=0.10,
        ram_promote_margin=0.20,
        policy="heavy_hitter",
    ):
        self._lib = _nat.load()
        vram = _unsigned(vram, _U64_MAX, "vram")
        ram = _unsigned(ram, _U64_MAX, "ram")
        recent = _unsigned(recent, _U64_MAX, "recent")
        rebalance_interval = _unsigned(rebalance_interval, _U64_MAX, "rebalance_interval")
        promote_margin = _f32(promote_margin, "promote_margin")
        ram_promote_margin = _f32(ram_promote_margin, "ram_promote_margin")
        if not isinstance(policy, str):
            raise TypeError(f"argument 'policy': '{type(policy).__name__}' object cannot be converted to 'PyString'")
        handle = self._lib.pgr_pager_new(
            vram, ram, recent, rebalance_interval, promote_margin, ram_promote_margin, policy.encode("utf-8")
        )
        if not handle:
            raise MemoryError("pgr_pager_new failed")
        self._handle = handle
        self._borrow = threading.Lock()

    def __del__(self):
        handle = getattr(self, "_handle", None)
        if handle:
            self._lib.pgr_pager_free(handle)
            self._handle = None

    def _enter(self):
        if not self._borrow.acquire(blocking=False):
            raise RuntimeError("Already borrowed")

    def on_step(self, token_idx, layer, attention) -> None:
        token_idx = _unsigned(token_idx, _U64_MAX, "token_idx")
        layer = _unsigned(layer, _U32_MAX, "layer")
        if isinstance(attention, (str, bytes)):
            raise TypeError("argument 'attention': Can't extract `str` to `Vec`")
        values = array.array("f", (_f32(a, "attention") for a in attention))
        n = len(values)
        buf = (ctypes.c_float * max(n, 1)).from_buffer(values) if n else None
        self._enter()
        try:
            rc = self._lib.pgr_pager_on_step(self._handle, token_idx, layer, buf, n)
        finally:
            self._borrow.release()
        if rc == _nat.PGR_ERR_STATE:
            raise ZeroDivisionError(_nat.last_error())
        _nat.check(rc, "on_step")

    def force_rebalance(self, token_idx) -> None:
        token_idx = _unsigned(token_idx, _U64_MAX, "token_idx")
        self._enter()
        try:
            rc = self._lib.pgr_pager_force_rebalance(self._handle, token_idx)
        finally:
            self._borrow.release()
        _nat.check(rc, "force_rebalance")

    def metrics(self) -> Metrics:
        m = _nat.PagerMetrics()
        _nat.check(self._lib.pgr_pager_metrics(self._handle, ctypes.byref(m)), "metrics")
        return Metrics._from_native(m)

    def tiers(self) -> list[int]:
        n = self._lib.pgr_pager_num_blocks(self._handle)
        buf = (ctypes.c_uint8 * max(n, 1))()
        self._lib.pgr_pager_tiers(self._handle, buf, n)
        return list(buf[:n])

    def vram_block_ids(self) -> list[int]:
        n = self._lib.pgr_pager_vram_block_ids(self._handle, None, 0)
        buf = (ctypes.c_uint64 * max(n, 1))()
        self._lib.pgr_pager_vram_block_ids(self._handle, buf, n)
        return list(buf[:n])
