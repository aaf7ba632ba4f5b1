"""int8 weight quantization and the weight-only int8 linear layer on the HIP GEMM.

Counterpart of ne/models/int8_quantization.py:17-73.  ``quantize_vectors`` is the
reference's per-vector symmetric formula (``scale = max|x| / 127`` in fp32, codes
``round(x / scale)`` clamped to +-127), so the codes and scales the kernels read are
the reference's.  ``Int8Linear.forward`` runs ``ne_w8a16_gemm``: the int8 rows become
bf16 in registers and the row scale multiplies the fp32 sum, where the reference first
materialises ``bf16(int8 * scale)`` for the whole weight (int8_quantization.py:55-57).
There is no other path: inputs off the GPU, or shapes the kernel does not take
(``k % 128``, ``n % 64``), raise.
"""

from __future__ import annotations

import torch
from torch import nn

from nanoengine_amd import kernels

INT8_MAX = 127
MIN_SCALE = 1e-8
QUANTIZED_PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def quantize_vectors(values: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """int8 codes and one scale per vector along the last dimension (the scale keeps that
    dimension, in the input dtype): int8_quantization.py:30-34."""
    scales = values.abs().amax(dim=-1, keepdim=True).float().clamp(min=MIN_SCALE) / INT8_MAX
    codes = torch.round(values.float() / scales).clamp(-INT8_MAX, INT8_MAX).to(torch.int8)
    return codes, scales.to(values.dtype)


class Int8Linear(nn.Module):
    """``y = x @ (int8 * scale)^T`` with bf16 activations, one scale per output row
    (int8_quantization.py:37-57), computed by the W8A16 kernel in one pass."""

    def __init__(self, weight_int8: torch.Tensor, weight_scale: torch.Tensor) -> None:
        super().__init__()
        self.register_buffer("weight_int8", weight_int8)
        self.register_buffer("weight_scale", weight_scale)

    @classmethod
    def from_linear(cls, linear: nn.Linear) -> "Int8Linear":
        """Codes and row scales computed on the host (IEEE fp32 division), so they do not
        depend on the device the layer sits on; then moved to that device."""
        weight = linear.weight.detach()
        weight_int8, weight_scale = quantize_vectors(weight.cpu())
        return cls(weight_int8.to(weight.device), weight_scale.squeeze(-1).to(weight.device))

    def forward(self, inputs: torch.Tensor) -> torch.Tensor:
        if not inputs.is_cuda:
            raise RuntimeError("Int8Linear runs on the HIP W8A16 kernel: inputs must be on the GPU")
        if inputs.dtype != torch.bfloat16:
            raise TypeError(f"the W8A16 kernel takes bf16 activations, got {inputs.dtype}")
        rows = inputs.reshape(-1, inputs.shape[-1])
        if rows.stride(-1) != 1 or rows.stride(0) % 8 != 0:
            rows = rows.contiguous()
        out = kernels.w8a16_gemm(rows, self.weight_int8, self.weight_scale)
        return out.reshape(*inputs.shape[:-1], self.weight_int8.shape[0])


def quantize_linear_layers(model: nn.Module) -> int:
    """Replace each attention and MLP projection of ``model.model.layers`` with
    ``Int8Linear``; returns how many (int8_quantization.py:60-73).  Embeddings, norms and
    the output head keep their dtype."""
    replaced = 0
    for layer in model.model.layers:
        for parent in (layer.self_attn, layer.mlp):
            for name in QUANTIZED_PROJECTIONS:
                projection = getattr(parent, name, None)
                if isinstance(projection, nn.Linear):
                    setattr(parent, name, Int8Linear.from_linear(projection))
                    replaced += 1
    return replaced
