"""Speculative decoding: rejection sampling (the reference's memforge_ml.speculative)."""

from memforge_amd.speculative.rejection_sampler import RejectionSampler

__all__ = ["RejectionSampler"]
