"""Fused efficient ops of the gcu device.

``gcu_index`` keeps the reference's one efficient op
(torch_gcu/gcu/efficient/op.py:8-16 -> torch_gcu/csrc/efficient_ops/ops.cpp:335-342);
``rms_norm``, ``rope``, ``rope_`` and ``silu_mul`` are new fused kernels, and
``linear_residual`` / ``linear_silu_mul`` are matmuls with the residual add or
the SwiGLU product fused into their epilogue.
All are dispatcher ops (``torch.ops.torch_gcu.*``) with gcu kernels only.
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from ... import _C  # noqa: F401  (registers torch.ops.torch_gcu)


def rms_norm(x: torch.Tensor, weight: Optional[torch.Tensor], eps: float = 1e-6) -> torch.Tensor:
    """x * rsqrt(mean(x^2, -1) + eps) * weight, fp32 math, one rounding."""
    return torch.ops.torch_gcu.rms_norm(x, weight, eps)


def rope(q: torch.Tensor, k: torch.Tensor, positions: torch.Tensor,
         theta: float = 10000.0) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotate-half RoPE of [tokens, heads, head_dim] q and k."""
    return torch.ops.torch_gcu.rope(q, k, positions, theta)


def rope_(q: torch.Tensor, k: Optional[torch.Tensor], positions: torch.Tensor,
          theta: float = 10000.0) -> None:
    """In-place RoPE of q (and k)."""
    torch.ops.torch_gcu.rope_(q, k, positions, theta)


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up with one rounding."""
    return torch.ops.torch_gcu.silu_mul(gate, up)


def linear_residual(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
    """residual + F.linear(x, weight), bit for bit as the two ops (the product
    rounded to the input dtype first)."""
    return torch.ops.torch_gcu.linear_residual(x, weight, residual)


def linear_silu_mul(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor) -> torch.Tensor:
    """silu_mul(F.linear(x, w_gate), F.linear(x, w_up)), bit for bit as the
    three ops (both products rounded to the input dtype first)."""
    return torch.ops.torch_gcu.linear_silu_mul(x, w_gate, w_up)


def int8_linear(x: torch.Tensor, weight: torch.Tensor, scales: torch.Tensor,
                bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """(x @ weight^T) * scales (+ bias): int8 [N, K] weight, fp32 [N] scales,
    widened exactly to bf16/fp16 and multiplied on MFMA with fp32 accumulation."""
    return torch.ops.torch_gcu.int8_linear(x, weight, scales, bias)


def gcu_index(self: torch.Tensor, indices: Sequence[Optional[torch.Tensor]]) -> torch.Tensor:
    """self[indices] with int32 index tensors (no int64 upcast on device)."""
    return torch.ops.torch_gcu.int32_indices_index(self, list(indices))
