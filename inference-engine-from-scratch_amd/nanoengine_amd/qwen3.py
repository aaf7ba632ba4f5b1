"""Qwen3 weights and the verify forward on the HIP kernels.

Host-side counterpart of ne/models/qwen3.py:13-203 and
ne/models/int8_quantization.py:37-73.  The 7 projections of every layer are
stored per-output-row int8 exactly as Int8Linear.from_linear quantises them;
q/k/v are concatenated into one [4096, 1024] weight and gate/up are interleaved
in groups of 16 rows so that one GEMM with a SwiGLU epilogue replaces
``down(silu(gate(x)) * up(x))``'s first two products.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, fields
from typing import Any

import torch

from nanoengine_amd import kernels
from nanoengine_amd._native import EPILOGUE_SWIGLU
from nanoengine_amd.int8_quantization import quantize_vectors


@dataclass(frozen=True)
class Qwen3Config:
    """ne/models/qwen3.py:13-28."""

    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    rms_norm_eps: float
    rope_theta: float
    tie_word_embeddings: bool

    @classmethod
    def from_dict(cls, values: dict[str, Any]) -> "Qwen3Config":
        return cls(**{f.name: values[f.name] for f in fields(cls)})


QWEN3_0_6B = Qwen3Config(151936, 1024, 3072, 28, 16, 8, 128, 1e-6, 1e6, True)


def parameter_specs(config: Qwen3Config) -> list[tuple[str, tuple[int, ...], str]]:
    """(name, shape, constructor init) in the reference's registration order
    (ne/models/qwen3.py:82-87, 123-125, 135-138, 157-162, 187-189)."""
    h, i = config.hidden_size, config.intermediate_size
    q = config.num_attention_heads * config.head_dim
    kv = config.num_key_value_heads * config.head_dim
    specs = [("model.embed_tokens.weight", (config.vocab_size, h), "embedding")]
    for layer in range(config.num_hidden_layers):
        p = f"model.layers.{layer}."
        specs += [
            (p + "self_attn.q_proj.weight", (q, h), "linear"),
            (p + "self_attn.k_proj.weight", (kv, h), "linear"),
            (p + "self_attn.v_proj.weight", (kv, h), "linear"),
            (p + "self_attn.o_proj.weight", (h, q), "linear"),
            (p + "self_attn.q_norm.weight", (config.head_dim,), "ones"),
            (p + "self_attn.k_norm.weight", (config.head_dim,), "ones"),
            (p + "mlp.gate_proj.weight", (i, h), "linear"),
            (p + "mlp.up_proj.weight", (i, h), "linear"),
            (p + "mlp.down_proj.weight", (h, i), "linear"),
            (p + "input_layernorm.weight", (h,), "ones"),
            (p + "post_attention_layernorm.weight", (h,), "ones"),
        ]
    specs.append(("model.norm.weight", (h,), "ones"))
    if not config.tie_word_embeddings:
        specs.append(("lm_head.weight", (config.vocab_size, h), "linear"))
    return specs


def random_state_dict(config: Qwen3Config, seed: int, std: float) -> dict[str, torch.Tensor]:
    """The reference's random initialisation: seed, construct the modules (whose own
    default initialisers draw from the generator), then draw every parameter from
    N(0, std^2) in registration order (tests/conftest.py pattern, nt/conftest.py:38-43).
    Returns fp32 CPU tensors."""
    torch.manual_seed(seed)
    state: dict[str, torch.Tensor] = {}
    for name, shape, init in parameter_specs(config):
        t = torch.empty(shape, dtype=torch.float32)
        if init == "embedding":
            torch.nn.init.normal_(t)
        elif init == "linear":
            torch.nn.init.kaiming_uniform_(t, a=math.sqrt(5))
        else:
            t.fill_(1.0)
        state[name] = t
    for name, _, _ in parameter_specs(config):
        torch.nn.init.normal_(state[name], std=std)
    return state


def quantize_rows(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-row symmetric int8, the codes and row scales of Int8Linear.from_linear
    (int8_quantization.py:50-53)."""
    q, scales = quantize_vectors(weight)
    return q, scales.squeeze(-1)


def pair_rows(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Interleave two [n, ...] tensors in groups of 16 rows: gate 0..15, up 0..15, gate 16..31, ..."""
    n = gate.shape[0]
    rest = gate.shape[1:]
    return torch.stack([gate.reshape(n // 16, 16, *rest), up.reshape(n // 16, 16, *rest)], dim=1).reshape(
        2 * n, *rest
    )


@dataclass
class LayerWeights:
    input_layernorm: torch.Tensor
    post_attention_layernorm: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    qkv_int8: torch.Tensor
    qkv_scale: torch.Tensor
    o_int8: torch.Tensor
    o_scale: torch.Tensor
    gate_up_int8: torch.Tensor  # gate/up rows paired per 16
    gate_up_scale: torch.Tensor
    down_int8: torch.Tensor
    down_scale: torch.Tensor


@dataclass
class Qwen3Weights:
    config: Qwen3Config
    embed: torch.Tensor  # [vocab, hidden] bf16, also the tied LM head
    norm: torch.Tensor
    layers: list[LayerWeights]
    lm_head: torch.Tensor | None = None

    @classmethod
    def from_state_dict(cls, config: Qwen3Config, state: dict[str, torch.Tensor], device: torch.device,
                        dtype: torch.dtype = torch.bfloat16) -> "Qwen3Weights":
        """Cast to ``dtype`` (the model dtype), quantise the 7 projections per layer to
        int8 as quantize_linear_layers does (int8_quantization.py:60-73), move to ``device``."""
        if dtype != torch.bfloat16:
            raise NotImplementedError("the HIP verify path runs bf16 activations (dtype=bfloat16)")

        def cast(name):
            return state[name].to(dtype)

        def dev(t):
            return t.contiguous().to(device)

        layers = []
        for i in range(config.num_hidden_layers):
            p = f"model.layers.{i}."
            qw, qs = quantize_rows(cast(p + "self_attn.q_proj.weight"))
            kw, ks = quantize_rows(cast(p + "self_attn.k_proj.weight"))
            vw, vs = quantize_rows(cast(p + "self_attn.v_proj.weight"))
            ow, os_ = quantize_rows(cast(p + "self_attn.o_proj.weight"))
            gw, gs = quantize_rows(cast(p + "mlp.gate_proj.weight"))
            uw, us = quantize_rows(cast(p + "mlp.up_proj.weight"))
            dw, ds = quantize_rows(cast(p + "mlp.down_proj.weight"))
            layers.append(LayerWeights(
                input_layernorm=dev(cast(p + "input_layernorm.weight")),
                post_attention_layernorm=dev(cast(p + "post_attention_layernorm.weight")),
                q_norm=dev(cast(p + "self_attn.q_norm.weight")),
                k_norm=dev(cast(p + "self_attn.k_norm.weight")),
                qkv_int8=dev(torch.cat([qw, kw, vw])),
                qkv_scale=dev(torch.cat([qs, ks, vs])),
                o_int8=dev(ow),
                o_scale=dev(os_),
                gate_up_int8=dev(pair_rows(gw, uw)),
                gate_up_scale=dev(pair_rows(gs, us)),
                down_int8=dev(dw),
                down_scale=dev(ds),
            ))
        lm_head = None if config.tie_word_embeddings else dev(cast("lm_head.weight"))
        return cls(config, dev(cast("model.embed_tokens.weight")), dev(cast("model.norm.weight")), layers,
                   lm_head)

    @property
    def output_weight(self) -> torch.Tensor:
        return self.embed if self.lm_head is None else self.lm_head


@dataclass
class AttentionBatch:
    """Device metadata of one step (the replacement of AttentionContext, attention_context.py:16-29)."""

    positions: torch.Tensor  # [rows] int32
    slot_mapping: torch.Tensor  # [rows] int32, pads -> scratch slot
    q_start: torch.Tensor  # [b] int32
    q_len: torch.Tensor  # [b] int32
    ctx_len: torch.Tensor  # [b] int32
    block_tables: torch.Tensor  # [b, max_blocks] int32
    max_q_len: int
    max_ctx_len: int


class Qwen3VerifyModel:
    """The verify forward (qwen3.py:164-203) as a chain of HIP kernels over packed rows."""

    def __init__(self, weights: Qwen3Weights, max_rows: int, device: torch.device) -> None:
        c = weights.config
        if c.head_dim != kernels.HEAD_DIM:
            raise NotImplementedError("the HIP kernels support head_dim 128")
        self.weights = weights
        self.config = c
        self.device = device
        self.max_rows = max_rows
        h = c.hidden_size
        q = c.num_attention_heads * c.head_dim
        qkv = (c.num_attention_heads + 2 * c.num_key_value_heads) * c.head_dim
        bf = dict(dtype=torch.bfloat16, device=device)
        self.residual = torch.empty(max_rows, h, **bf)
        self.normed = torch.empty(max_rows, h, **bf)
        self.delta = torch.empty(max_rows, h, **bf)
        self.qkv = torch.empty(max_rows, qkv, **bf)
        self.q = torch.empty(max_rows, c.num_attention_heads, c.head_dim, **bf)
        self.attn = torch.empty(max_rows, c.num_attention_heads, c.head_dim, **bf)
        self.act = torch.empty(max_rows, c.intermediate_size, **bf)
        # cos/sin per position (qwen3.py:47-57), computed once on the host as the
        # reference computes them per step; grown when a longer position appears
        self.rope_positions = 0
        self.rope = None
        self.graph_bound = False
        self.ensure_rope(4096)
        # attention scratch of the forwards a HIP graph captures (verify steps, graphed
        # draft decode rows) and, separately, of eager forwards (prefill, a draft's
        # catch-up): an eager forward of another shape must never move a buffer whose
        # address a graph holds
        self.workspace = kernels.AttentionWorkspace()
        self.eager_workspace = kernels.AttentionWorkspace()
        # QKV projection with QK-norm, RoPE and the KV write in its epilogue; False
        # runs the GEMM and the row kernel separately (the same bits, one more launch)
        self.fuse_qkv = True
        self.softmax_scale = 1.0 / math.sqrt(c.head_dim)
        # o_proj / down_proj (N = hidden) split K across work-groups when the rows alone
        # give too few output tiles; the fp32 partials feed the fused residual add + norm
        self.o_splits = [kernels.splitk_splits(r, h, q) for r in range(max_rows + 1)]
        self.down_splits = [kernels.splitk_splits(r, h, c.intermediate_size) for r in range(max_rows + 1)]
        most = max(max(a * r, b * r) for r, (a, b) in enumerate(zip(self.o_splits, self.down_splits)))
        self.partials = torch.empty(max(most, 1) * h, dtype=torch.float32, device=device)

    def bind_graph(self) -> None:
        """A HIP graph now holds this model's buffers (activations, RoPE table, the graph
        workspace): they must keep their addresses from here on."""
        self.graph_bound = True
        self.workspace.frozen = True

    def ensure_rope(self, positions: int) -> None:
        """Make the RoPE table cover positions 0 .. positions-1 (before any graph capture)."""
        if positions > self.rope_positions:
            if self.graph_bound:
                raise RuntimeError(f"RoPE table of {self.rope_positions} positions is held by a captured HIP "
                                   f"graph; {positions} positions must be reserved before capture")
            self.rope = kernels.rope_table(positions, self.config.rope_theta).to(self.device)
            self.rope_positions = positions

    def forward(self, rows: int, tokens: torch.Tensor, batch: AttentionBatch, pool,
                workspace: kernels.AttentionWorkspace | None = None) -> torch.Tensor:
        """Hidden states after the final norm for ``rows`` packed query rows; writes this
        step's keys/values into ``pool`` at ``batch.slot_mapping``.  ``workspace``: the
        attention scratch (default: the one graph-captured forwards use)."""
        if rows > self.max_rows:
            raise ValueError(f"{rows} rows exceed the model's capacity of {self.max_rows}")
        ws = self.workspace if workspace is None else workspace
        c = self.config
        w = self.weights
        eps = c.rms_norm_eps
        res, normed, delta = self.residual[:rows], self.normed[:rows], self.delta[:rows]
        qkv, q, attn, act = self.qkv[:rows], self.q[:rows], self.attn[:rows], self.act[:rows]
        kernels.embed_rmsnorm(tokens[:rows], w.embed, w.layers[0].input_layernorm, eps, residual=res, out=normed)
        # the attention work plan depends only on this step's metadata: made once, read by
        # every layer's attention call
        planned = kernels.plan_supported(c.num_attention_heads, c.num_key_value_heads, batch.max_q_len,
                                         batch.ctx_len.shape[0], pool.key_caches[0].dtype,
                                         pool.key_scale_2d(0).dtype if pool.key_scale_2d(0) is not None else None)
        if planned:
            kernels.paged_attention_plan(batch.block_tables, pool.block_size, batch.ctx_len, batch.q_start,
                                         batch.q_len, c.num_attention_heads, c.num_key_value_heads,
                                         batch.max_q_len, batch.max_ctx_len, ws)
        fuse = self.fuse_qkv and kernels.qkv_fusion_supported(pool.key_caches[0], pool.key_scale_2d(0))
        for i, layer in enumerate(w.layers):
            if fuse:  # QK-norm + RoPE + KV write in the QKV GEMM's epilogue (same bits)
                kernels.w8a16_qkv_norm_rope_kv(
                    normed, layer.qkv_int8, layer.qkv_scale, c.num_attention_heads, c.num_key_value_heads,
                    layer.q_norm, layer.k_norm, eps, batch.positions[:rows], self.rope,
                    batch.slot_mapping[:rows], pool.key_caches[i], pool.value_caches[i],
                    pool.key_scale_2d(i), pool.value_scale_2d(i), q_out=q,
                )
            else:
                kernels.w8a16_gemm(normed, layer.qkv_int8, layer.qkv_scale, out=qkv)
                kernels.qk_norm_rope_kv_write(
                    qkv, c.num_attention_heads, c.num_key_value_heads, layer.q_norm, layer.k_norm, eps,
                    batch.positions[:rows], self.rope, batch.slot_mapping[:rows],
                    pool.key_caches[i], pool.value_caches[i], pool.key_scale_2d(i), pool.value_scale_2d(i),
                    q_out=q,
                )
            kernels.paged_verify_attention(
                q, pool.key_caches[i], pool.value_caches[i], pool.key_scale_2d(i), pool.value_scale_2d(i),
                batch.block_tables, pool.block_size, batch.ctx_len, batch.q_start, batch.q_len,
                batch.max_q_len, batch.max_ctx_len, self.softmax_scale, out=attn, workspace=ws,
                planned=planned,
            )
            self._project_add_norm(attn.view(rows, -1), layer.o_int8, layer.o_scale, self.o_splits[rows],
                                   layer.post_attention_layernorm, res, delta, normed)
            kernels.w8a16_gemm(normed, layer.gate_up_int8, layer.gate_up_scale, epilogue=EPILOGUE_SWIGLU,
                               out=act)
            next_norm = w.layers[i + 1].input_layernorm if i + 1 < len(w.layers) else w.norm
            self._project_add_norm(act, layer.down_int8, layer.down_scale, self.down_splits[rows], next_norm,
                                   res, delta, normed)
        return normed

    def _project_add_norm(self, x, w_int8, w_scale, splits, norm_weight, res, delta, normed) -> None:
        """residual += bf16(x @ W^T); normed = RMSNorm(residual) (qwen3.py:145-149)."""
        eps = self.config.rms_norm_eps
        if splits > 1:
            rows = x.shape[0]
            parts = self.partials[: splits * rows * w_int8.shape[0]]
            kernels.w8a16_gemm_splitk(x, w_int8, w_scale, splits, out=parts)
            kernels.splitk_add_rmsnorm(res, parts, splits, norm_weight, eps, out=normed)
        else:
            kernels.w8a16_gemm(x, w_int8, w_scale, out=delta)
            kernels.add_rmsnorm(res, delta, norm_weight, eps, out=normed)

    def compute_logits(self, hidden: torch.Tensor, logits: bool = True, argmax: bool = False):
        """qwen3.py:197-203 on the bf16 LM-head kernel; optionally only argmax partials."""
        return kernels.lm_head(hidden, self.weights.output_weight, logits=logits, argmax_partials=argmax)
