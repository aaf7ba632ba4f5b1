"""Speculative-decoding counters (ne/engine/metrics.py:66-75) and the prefix-cache
hit gauge (metrics.py:61-65) in a per-engine registry.

Uses prometheus_client when it is importable, with the same metric names; the
benchmark definitions (ne/benchmarks/speculative.py:104-114) are
acceptance = accepted / proposed and tokens per target pass = tokens / (tokens - accepted).
"""

from __future__ import annotations

try:
    from prometheus_client import CollectorRegistry, Counter, Gauge
except ImportError:  # pragma: no cover - the image ships prometheus_client
    CollectorRegistry = None
    Counter = None
    Gauge = None


class _PlainCounter:
    def __init__(self) -> None:
        self.value = 0.0

    def inc(self, amount: float = 1.0) -> None:
        self.value += amount

    def set(self, value: float) -> None:
        self.value = value


class EngineMetrics:
    def __init__(self) -> None:
        if CollectorRegistry is not None:
            self.registry = CollectorRegistry()
            self.speculative_proposed_tokens = Counter(
                "nanoengine_speculative_proposed_tokens", "Tokens guessed by the speculative proposer",
                registry=self.registry)
            self.speculative_accepted_tokens = Counter(
                "nanoengine_speculative_accepted_tokens",
                "Guessed tokens the target model kept; accepted / proposed is the acceptance rate",
                registry=self.registry)
            self.prefix_cache_hit_tokens = Gauge(
                "nanoengine_prefix_cache_hit_tokens",
                "Prompt tokens taken from the prefix cache instead of computed, since start",
                registry=self.registry)
        else:
            self.registry = None
            self.speculative_proposed_tokens = _PlainCounter()
            self.speculative_accepted_tokens = _PlainCounter()
            self.prefix_cache_hit_tokens = _PlainCounter()

    def _value(self, counter, name: str) -> float:
        if self.registry is not None:
            return float(self.registry.get_sample_value(name) or 0.0)
        return counter.value

    @property
    def proposed(self) -> float:
        return self._value(self.speculative_proposed_tokens, "nanoengine_speculative_proposed_tokens_total")

    @property
    def accepted(self) -> float:
        return self._value(self.speculative_accepted_tokens, "nanoengine_speculative_accepted_tokens_total")

    @property
    def prefix_hit_tokens(self) -> float:
        return self._value(self.prefix_cache_hit_tokens, "nanoengine_prefix_cache_hit_tokens")


def acceptance_rate(proposed: float, accepted: float) -> float:
    return accepted / proposed if proposed else 0.0


def tokens_per_target_pass(tokens: float, accepted: float) -> float:
    return tokens / max(tokens - accepted, 1)
