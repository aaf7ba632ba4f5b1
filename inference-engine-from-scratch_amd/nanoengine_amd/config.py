"""Engine settings from ``NANOENGINE_*`` variables (ne/config.py:23-108, ne/constants.py:6-7).

Same field names, defaults and cross-field checks as the reference's
EngineSettings, restated without pydantic-settings.  Two deliberate widenings of
ne/config.py:91-97:

* the reference refuses speculation with a batched scheduler because its verify
  step handles one sequence; the HIP path verifies a whole batch per step, so
  ``scheduler=static|continuous`` with ``speculative=ngram`` is accepted;
* the reference refuses speculation with the prefix cache because its verify
  step registers blocks while the guesses are still part of the sequence
  (model_runner.py:60-61); the HIP runner registers only verified blocks after
  acceptance, so ``prefix_cache=true`` with ``speculative=ngram`` is accepted.
"""

from __future__ import annotations

import os
from dataclasses import dataclass, fields
from pathlib import Path

import torch

ENV_PREFIX = "NANOENGINE_"
ENV_FILE_VARIABLE = "NANOENGINE_ENV_FILE"
TORCH_DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}

_CHOICES = {
    "dtype": ("float32", "float16", "bfloat16"),
    "kv_cache": ("none", "contiguous", "paged"),
    "scheduler": ("serial", "static", "continuous"),
    "quantization": ("none", "int8"),
    "kv_cache_dtype": ("auto", "int8"),
    "speculative": ("none", "ngram", "draft"),
}
_MINIMUM_ONE = ("max_num_seqs", "kv_cache_memory_mb", "kv_block_size", "max_prefill_tokens",
                "max_num_batched_tokens", "cuda_graph_max_context", "cuda_graph_max_batch",
                "num_speculative_tokens", "ngram_max_size")


@dataclass
class EngineSettings:
    model_id: str = "Qwen/Qwen3-0.6B"
    served_model_name: str | None = None
    model_cache_dir: Path | None = None
    device: str = "cpu"
    dtype: str = "float32"
    max_model_len: int = 4096
    max_waiting_requests: int = 256
    kv_cache: str = "none"
    scheduler: str = "serial"
    max_num_seqs: int = 64
    kv_cache_memory_mb: int = 1024
    kv_block_size: int = 16
    max_prefill_tokens: int = 4096
    batch_fill_timeout_ms: int = 50
    prefix_cache: bool = False
    chunked_prefill: bool = False
    max_num_batched_tokens: int = 512
    quantization: str = "none"
    kv_cache_dtype: str = "auto"
    cuda_graphs: bool = False
    cuda_graph_max_context: int = 1024
    cuda_graph_max_batch: int = 8
    speculative: str = "none"
    num_speculative_tokens: int = 4
    draft_model_id: str = "Qwen/Qwen3-0.6B"
    ngram_max_size: int = 3
    host: str = "0.0.0.0"
    port: int = 8000
    log_level: str = "info"

    def __post_init__(self) -> None:
        for name, allowed in _CHOICES.items():
            if getattr(self, name) not in allowed:
                raise ValueError(f"{name}={getattr(self, name)!r} is not one of {allowed}")
        for name in _MINIMUM_ONE:
            if getattr(self, name) < 1:
                raise ValueError(f"{name} must be >= 1")
        self._check_combinations()

    @property
    def is_batched(self) -> bool:
        return self.scheduler != "serial"

    @property
    def is_int8_kv_cache(self) -> bool:
        return self.kv_cache_dtype == "int8"

    @property
    def public_model_name(self) -> str:
        return self.served_model_name or self.model_id

    def _check_combinations(self) -> None:
        """ne/config.py:81-98, with batched and prefix-cached speculation allowed (see module docstring)."""
        if self.is_batched and self.kv_cache == "none":
            raise ValueError(f"scheduler={self.scheduler} needs kv_cache=contiguous or paged")
        if self.prefix_cache and self.kv_cache != "paged":
            raise ValueError("prefix_cache needs kv_cache=paged (it shares blocks)")
        if self.chunked_prefill and self.scheduler != "continuous":
            raise ValueError("chunked_prefill needs scheduler=continuous")
        if self.kv_cache == "none" and (self.kv_cache_dtype == "int8" or self.cuda_graphs):
            raise ValueError("kv_cache_dtype=int8 and cuda_graphs need a KV cache")
        if self.speculative != "none" and self.kv_cache == "none":
            raise ValueError("speculative decoding needs a KV cache")
        if self.speculative == "draft" and self.prefix_cache:
            raise ValueError("draft-model speculation does not support the prefix cache")

    @classmethod
    def from_env(cls, environ: dict[str, str] | None = None) -> "EngineSettings":
        """Read ``NANOENGINE_*`` (real variables override ``NANOENGINE_ENV_FILE``)."""
        environ = dict(os.environ if environ is None else environ)
        values: dict[str, str] = {}
        env_file = environ.get(ENV_FILE_VARIABLE)
        if env_file:
            for line in Path(env_file).read_text().splitlines():
                line = line.strip()
                if line and not line.startswith("#") and "=" in line:
                    key, value = line.split("=", 1)
                    values[key.strip()] = value.strip().strip("'\"")
        values.update({k: v for k, v in environ.items() if k.startswith(ENV_PREFIX)})
        kwargs = {}
        for f in fields(cls):
            raw = values.get(ENV_PREFIX + f.name.upper())
            if raw is None:
                continue
            if f.type in ("bool", bool):
                kwargs[f.name] = raw.lower() in ("1", "true", "yes", "on")
            elif f.type in ("int", int):
                kwargs[f.name] = int(raw)
            elif f.name == "model_cache_dir":
                kwargs[f.name] = Path(raw)
            else:
                kwargs[f.name] = raw
        return cls(**kwargs)

    def hip_verify_path_error(self) -> str | None:
        """Why these settings cannot run the HIP verify path, or None when they can."""
        if not self.device.startswith("cuda"):
            return "device must be a ROCm GPU (cuda)"
        if self.dtype != "bfloat16":
            return "dtype must be bfloat16"
        if self.kv_cache != "paged":
            return "kv_cache must be paged"
        if self.quantization != "int8":
            return "quantization must be int8 (W8A16 projections)"
        if self.speculative not in ("ngram", "draft"):
            return "speculative must be ngram or draft"
        if self.kv_block_size % 16 != 0:
            return "kv_block_size must be a multiple of 16"
        return None
