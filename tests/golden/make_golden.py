"""Writes the golden fixtures for the fused ops that have no reference
counterpart (RMSNorm, RoPE, SiLU-mul).

The reference holds no golden vectors for this path, so these are computed
here, in float64 numpy from the closed forms (independent of the torch code
in oracle/aten.py), and stored as float32.  Inputs are bf16-representable
values kept in float32 arrays.  Run from the repository root:

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import numpy_ref as npr  # noqa: E402


def main():
    rng = np.random.default_rng(20261201)
    x = npr.round_bf16(rng.standard_normal((6, 256)).astype(np.float32))
    w = npr.round_bf16((1.0 + 0.02 * rng.standard_normal(256)).astype(np.float32))
    np.savez(os.path.join(HERE, "rms_norm.npz"), x=x, w=w, eps=np.float64(1e-6),
             expected=npr.rms_norm64(x, w, 1e-6).astype(np.float32))
    q = npr.round_bf16(rng.standard_normal((5, 3, 32)).astype(np.float32))
    pos = np.array([0, 1, 7, 100, 4095], dtype=np.int64)
    np.savez(os.path.join(HERE, "rope.npz"), x=q, pos=pos, theta=np.float64(10000.0),
             expected=npr.rope64(q, pos, 10000.0).astype(np.float32))
    gt = npr.round_bf16(rng.standard_normal((4, 96)).astype(np.float32))
    up = npr.round_bf16(rng.standard_normal((4, 96)).astype(np.float32))
    np.savez(os.path.join(HERE, "silu_mul.npz"), gate=gt, up=up,
             expected=npr.silu_mul64(gt, up).astype(np.float32))


if __name__ == "__main__":
    main()
