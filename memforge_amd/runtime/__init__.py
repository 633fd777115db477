"""Continuous-batching runtime over the paged KV pool in HBM: pool, caches,
sampling, the engine and speculative verification (the reference package
memforge_ml/runtime/__init__.py exports the same names)."""

from memforge_amd.runtime.kv_pool import ModelKVSpec, PagedKVPool
from memforge_amd.runtime.paged_cache import PagedCache, PagedCacheLayer
from memforge_amd.runtime.sampling import SamplingParams, sample_logits
from memforge_amd.runtime.continuous_engine import (
    HAS_CPP_ENGINE,
    ContinuousBatchingEngine,
    SequenceRuntime,
    StepReport,
    TokenEvent,
)

__all__ = [
    "ModelKVSpec",
    "PagedKVPool",
    "PagedCache",
    "PagedCacheLayer",
    "SamplingParams",
    "sample_logits",
    "ContinuousBatchingEngine",
    "SequenceRuntime",
    "StepReport",
    "TokenEvent",
    "HAS_CPP_ENGINE",
]
