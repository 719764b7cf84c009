"""Continuous-batching decode serving over the native paged store.

Import what you need directly, as in the reference (pager_hf/serving/__init__.py):
    from pager_hf.serving.scheduler import ContinuousBatchingScheduler
"""
