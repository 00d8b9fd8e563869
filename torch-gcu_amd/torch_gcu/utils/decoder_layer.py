"""The Llama-7B-shaped decoder layer of benchmark config 5, written as plain
torch code so that on a gcu tensor every op goes through the PrivateUse1
registrations: embedding (index_select), RMSNorm / RoPE (the fused efficient
ops), the q / k / v projections (mm on MFMA), causal
scaled_dot_product_attention (the flash kernel), and the o / down projections
with the residual add and the gate / up projections with the SiLU-mul fused
into the matmul epilogue (efficient ops that give what linear + add and
linear, linear + silu_mul give, bit for bit).

The same module runs on CPU tensors with the ATen compositions of the fused
ops, which is how the tests compare the two paths.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass
class LayerConfig:
    vocab: int = 32000
    hidden: int = 4096
    heads: int = 32
    head_dim: int = 128
    ffn: int = 11008
    theta: float = 10000.0
    eps: float = 1e-6


def init_weights(cfg: LayerConfig, seed: int = 20261205, dtype=torch.bfloat16) -> dict:
    """Random-init weights, normal(0, 0.02); norm weights are ones."""
    g = torch.Generator().manual_seed(seed)

    def w(*shape):
        return (torch.randn(shape, generator=g) * 0.02).to(dtype)

    h, f = cfg.hidden, cfg.ffn
    return {
        "embed": w(cfg.vocab, h),
        "attn_norm": torch.ones(h, dtype=dtype),
        "wq": w(h, h), "wk": w(h, h), "wv": w(h, h), "wo": w(h, h),
        "ffn_norm": torch.ones(h, dtype=dtype),
        "w_gate": w(f, h), "w_up": w(f, h), "w_down": w(h, f),
    }


def _rms_norm(x, w, eps):
    if x.device.type == "gcu":
        return torch.gcu.efficient.rms_norm(x, w, eps)
    return torch.rms_norm(x, [x.shape[-1]], w, eps)


def _rope_(q, k, pos, theta):
    """In-place rotate-half RoPE on [tokens, heads, head_dim]."""
    if q.device.type == "gcu":
        torch.gcu.efficient.rope_(q, k, pos, theta)
        return
    d = q.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
    ang = pos.float()[:, None] * inv[None, :]
    cos, sin = ang.cos()[:, None, :], ang.sin()[:, None, :]
    for t in (q, k):
        tf = t.float()
        x1, x2 = tf[..., : d // 2], tf[..., d // 2:]
        t.copy_(torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], -1))


def _silu_mul(gate, up):
    if gate.device.type == "gcu":
        return torch.gcu.efficient.silu_mul(gate, up)
    return (F.silu(gate.float()) * up.float()).to(gate.dtype)


def _linear_residual(x, w, residual):
    """residual + linear(x, w) (the product rounded first, as two ops)."""
    if x.device.type == "gcu":
        return torch.gcu.efficient.linear_residual(x, w, residual)
    return residual + F.linear(x, w)


def _linear_silu_mul(h, w_gate, w_up):
    """silu_mul(linear(h, w_gate), linear(h, w_up))."""
    if h.device.type == "gcu":
        return torch.gcu.efficient.linear_silu_mul(h, w_gate, w_up)
    return _silu_mul(F.linear(h, w_gate), F.linear(h, w_up))


def positions(batch: int, seq: int, device) -> torch.Tensor:
    """Token positions 0..seq-1 for each sequence, flattened (int64)."""
    return torch.arange(seq, dtype=torch.int64).repeat(batch).to(device)


def forward(weights: dict, ids: torch.Tensor, cfg: LayerConfig,
            pos: torch.Tensor | None = None, fused: bool = True) -> torch.Tensor:
    """One decoder layer over token ids [batch, seq]; returns [batch*seq, hidden].
    `pos` (from positions()) is passed in when the call is captured in a
    graph, so nothing inside the captured region is created on the host.
    fused=False runs the o / gate / up / down projections as plain linears
    followed by the adds and silu_mul (every projection then goes through the
    dispatcher's mm, which op_check compares op by op); the result is the
    same bit for bit."""
    B, S = ids.shape
    T = B * S
    H, D = cfg.heads, cfg.head_dim
    x = F.embedding(ids.reshape(-1), weights["embed"])  # [T, hidden]
    if pos is None:
        pos = positions(B, S, ids.device)
    h = _rms_norm(x, weights["attn_norm"], cfg.eps)
    q = F.linear(h, weights["wq"]).view(T, H, D)
    k = F.linear(h, weights["wk"]).view(T, H, D)
    v = F.linear(h, weights["wv"]).view(T, H, D)
    _rope_(q, k, pos, cfg.theta)
    qh = q.view(B, S, H, D).transpose(1, 2)
    kh = k.view(B, S, H, D).transpose(1, 2)
    vh = v.view(B, S, H, D).transpose(1, 2)
    a = F.scaled_dot_product_attention(qh, kh, vh, is_causal=True)
    a = a.transpose(1, 2).reshape(T, H * D)
    if not fused:
        x = x + F.linear(a, weights["wo"])
        h = _rms_norm(x, weights["ffn_norm"], cfg.eps)
        m = _silu_mul(F.linear(h, weights["w_gate"]), F.linear(h, weights["w_up"]))
        return x + F.linear(m, weights["w_down"])
    x = _linear_residual(a, weights["wo"], x)
    h = _rms_norm(x, weights["ffn_norm"], cfg.eps)
    m = _linear_silu_mul(h, weights["w_gate"], weights["w_up"])
    return _linear_residual(m, weights["w_down"], x)


def flops(cfg: LayerConfig, batch: int, seq: int) -> int:
    """Linear + causal attention FLOPs of one forward."""
    T = batch * seq
    params = 4 * cfg.hidden * cfg.hidden + 3 * cfg.hidden * cfg.ffn
    linear = 2 * T * params
    attn = 4 * batch * cfg.heads * cfg.head_dim * (seq * (seq + 1) // 2)
    return linear + attn
