"""int8 quantisation, restating ne/models/int8_quantization.py:17-73."""

from __future__ import annotations

import torch

INT8_MAX = 127
MIN_SCALE = 1e-8
QUANTIZED_PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def quantize_vectors(values: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """int8_quantization.py:30-34: symmetric absmax/127 per last-dim vector, round half even."""
    scales = values.abs().amax(dim=-1, keepdim=True).float().clamp(min=MIN_SCALE) / INT8_MAX
    quantized = torch.round(values.float() / scales).clamp(-INT8_MAX, INT8_MAX).to(torch.int8)
    return quantized, scales.to(values.dtype)


def int8_linear(inputs: torch.Tensor, weight_int8: torch.Tensor, weight_scale: torch.Tensor) -> torch.Tensor:
    """int8_quantization.py:55-57: dequantise the whole weight, then F.linear."""
    weight = weight_int8.to(inputs.dtype) * weight_scale[:, None]
    return torch.nn.functional.linear(inputs, weight)


def quantize_linear(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Int8Linear.from_linear (int8_quantization.py:50-53): per output row."""
    weight_int8, scale = quantize_vectors(weight.detach())
    return weight_int8, scale.squeeze(-1)
