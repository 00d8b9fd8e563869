"""Seeded synthetic inputs for the five benchmark configurations.

Every tensor is generated on the CPU from ``torch.Generator().manual_seed(
20261201 + config_index)`` so that the device path and the CPU ATen path see
identical bits after the copy.  ``rows`` arguments shrink the leading
dimension for quick parity runs while keeping the distributions.
"""
from __future__ import annotations

import torch

SEED_BASE = 20261201


def gen(config_index: int) -> torch.Generator:
    return torch.Generator().manual_seed(SEED_BASE + config_index)


def uniform(shape, lo, hi, g, dtype=torch.float32):
    return (torch.rand(shape, generator=g, dtype=torch.float32) * (hi - lo) + lo).to(dtype)


def normal(shape, mean, std, g, dtype=torch.float32):
    return (torch.randn(shape, generator=g, dtype=torch.float32) * std + mean).to(dtype)


def config1(rows: int = 4096, cols: int = 4096, table_rows: int = 1048576, n_idx: int = 262144):
    """out = a*b + c with b broadcast over rows; index_select on an int64 table."""
    g = gen(1)
    a = uniform((rows, cols), -1.0, 1.0, g)
    b = uniform((cols,), -1.0, 1.0, g)
    c = 0.5
    table = torch.randint(-2**63, 2**63 - 1, (table_rows, 8), generator=g, dtype=torch.int64)
    idx = torch.randint(0, table_rows, (n_idx,), generator=g, dtype=torch.int64)
    return {"a": a, "b": b, "c": c, "table": table, "idx": idx}


def config2(rows: int = 8192, vocab: int = 32000, mrows: int = 16384, mcols: int = 4096):
    """bf16 logits N(0, 4) for sum / amax / log_softmax; fp32 N(0, 1) for mean(0)."""
    g = gen(2)
    logits = normal((rows, vocab), 0.0, 4.0, g, torch.bfloat16)
    m = normal((mrows, mcols), 0.0, 1.0, g)
    return {"logits": logits, "m": m}


def config3(tokens: int = 16384, hidden: int = 4096, heads: int = 32, head_dim: int = 128,
            ffn: int = 11008, seq: int = 4096):
    """RMSNorm / RoPE / SiLU-mul inputs at the Llama-7B shape, bf16."""
    g = gen(3)
    x = normal((tokens, hidden), 0.0, 1.0, g, torch.bfloat16)
    w = normal((hidden,), 1.0, 0.02, g, torch.bfloat16)
    q = normal((tokens, heads, head_dim), 0.0, 1.0, g, torch.bfloat16)
    k = normal((tokens, heads, head_dim), 0.0, 1.0, g, torch.bfloat16)
    pos = torch.arange(tokens, dtype=torch.int64) % seq
    gate = normal((tokens, ffn), 0.0, 1.0, g, torch.bfloat16)
    up = normal((tokens, ffn), 0.0, 1.0, g, torch.bfloat16)
    return {"x": x, "w": w, "eps": 1e-6, "q": q, "k": k, "pos": pos, "theta": 10000.0,
            "gate": gate, "up": up}
