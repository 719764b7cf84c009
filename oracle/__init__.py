"""CPU restatement of the reference's decode-attention path: TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this package, and only as the checker (or the timed CPU baseline). The product path
(``pager``, ``pager_hf`` over libpgr.so) never imports it.

Modules: ``attention`` (dense fp32 oracle and the fold-kernel semantics),
``pager_policy`` (placement policy of pager/src/core.rs), ``paged_decode`` (one decode step
over paged sessions: placement glue, gather indices, attention, mass), ``kv_layout``
(block split/extract of pager_hf/kv_utils.py).
"""
