"""MI355X-native streaming decode attention with the reference's ``pager_hf`` interface.

Exports follow pager_hf/__init__.py:1-4 of the reference where the path is built:
``PagedModel`` (the HuggingFace wrapper), ``KVBlockStore`` (reference API over the native
slot pools) and the fused multi-session decoder ``PagedDecoder``. Operator functions live in ``pager_hf.streaming_attention``.
"""
from .kv_block_store import KVBlockStore, KVBlockStoreStats
from .kv_pool import NativeKVPool
from .paged_decode import PagedDecoder

__all__ = ["GenerationStats", "KVBlockStore", "KVBlockStoreStats", "NativeKVPool", "PagedDecoder", "PagedModel"]


def __getattr__(name):
    # PagedModel pulls in transformers; import it on first use only.
    if name in ("PagedModel", "GenerationStats"):
        from . import paged_model

        return getattr(paged_model, name)
    raise AttributeError(name)
