"""Per-request sampling parameters: the call-surface type of the sampler.

Same fields, defaults, validation ranges and predicates as the reference's
``SamplingParams`` (engine/runtime/sampling.py:19-97), so a request built for the
reference engine is accepted unchanged.  Defaults are plain greedy decoding.
"""

from __future__ import annotations

from dataclasses import dataclass, field


@dataclass(frozen=True)
class SamplingParams:
    """One request's sampling knobs (engine/runtime/sampling.py:19-48).

    ``temperature == 0`` means greedy and overrides every other knob; ``top_k <= 0``
    and ``top_p >= 1`` switch those filters off; ``min_p == 0`` switches min-p off.
    """

    temperature: float = 0.0
    top_p: float = 1.0
    top_k: int = 0
    min_p: float = 0.0
    repetition_penalty: float = 1.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    penalize_prompt: bool = False
    seed: int | None = None
    stop_token_ids: frozenset[int] = field(default_factory=frozenset)
    ignore_eos: bool = False
    logprobs: int | None = None

    def __post_init__(self) -> None:
        # Ranges of engine/runtime/sampling.py:50-69; each failure is a ValueError.
        checks = (
            (0.0 <= self.temperature <= 2.0, "temperature must be in [0, 2]"),
            (0.0 < self.top_p <= 1.0, "top_p must be in (0, 1]"),
            (self.top_k >= 0, "top_k must be non-negative (0 disables it)"),
            (0.0 <= self.min_p <= 1.0, "min_p must be in [0, 1]"),
            (0.0 < self.repetition_penalty <= 2.0, "repetition_penalty must be in (0, 2]"),
            (-2.0 <= self.presence_penalty <= 2.0, "presence_penalty must be in [-2, 2]"),
            (-2.0 <= self.frequency_penalty <= 2.0, "frequency_penalty must be in [-2, 2]"),
            (self.logprobs is None or 0 <= self.logprobs <= 20, "logprobs must be in [0, 20]"),
            (self.seed is None or 0 <= self.seed < 2**63,
             "seed must be a non-negative 63-bit integer"),
        )
        for ok, message in checks:
            if not ok:
                raise ValueError(message)
        object.__setattr__(self, "stop_token_ids", frozenset(self.stop_token_ids))

    @property
    def greedy(self) -> bool:
        """Argmax whatever the other fields say (sampling.py:71-74)."""
        return self.temperature == 0.0 or self.top_k == 1

    @property
    def has_penalties(self) -> bool:
        """Any of the three history penalties is active (sampling.py:76-79)."""
        return (self.repetition_penalty != 1.0 or self.presence_penalty != 0.0
                or self.frequency_penalty != 0.0)

    @property
    def deterministic(self) -> bool:
        """Repeating the request reproduces its tokens (sampling.py:81-84)."""
        return self.greedy or self.seed is not None

    @property
    def can_reuse_cached_prediction(self) -> bool:
        """A prompt-only cache entry fixes the next token (sampling.py:86-94)."""
        return self.greedy and not self.has_penalties and self.logprobs is None


GREEDY = SamplingParams()
