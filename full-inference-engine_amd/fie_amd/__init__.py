"""MI355X-native fused token sampler with the reference engine's sampler surface.

``fie_amd.batching.sampler.BatchedSampler`` and ``fie_amd.runtime.sampling`` mirror
``engine.batching.sampler`` and ``engine.runtime.sampling`` of full-inference-engine.
"""

from .batching.sampler import BatchedSampler, SampleResult
from .runtime.sampling import GREEDY, SamplingParams

__all__ = ["BatchedSampler", "SampleResult", "SamplingParams", "GREEDY"]
