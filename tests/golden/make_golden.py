"""Writes the golden fixtures for the fused ops that have no reference
counterpart (RMSNorm, RoPE, SiLU-mul) and for the training-side ops
(AdamW step, layer-norm forward and backward, log_softmax backward, cat).

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
    # one AdamW step (float64 closed form) with weight decay and grad scaling
    p = rng.standard_normal((3, 40)).astype(np.float32)
    g = (rng.standard_normal((3, 40)) * 16.0).astype(np.float32)
    m = (0.01 * rng.standard_normal((3, 40))).astype(np.float32)
    v = (1e-4 * rng.random((3, 40))).astype(np.float32)
    hp = np.array([2e-3, 0.9, 0.99, 0.05, 1e-8, 3.0, 16.0])  # lr b1 b2 wd eps step scale
    ep, eg, em, ev, _ = npr.adamw64(p, g, m, v, None, hp[5], hp[0], hp[1], hp[2], hp[3], hp[4],
                                    False, False, hp[6])
    np.savez(os.path.join(HERE, "adamw.npz"), p=p, g=g, m=m, v=v, hp=hp,
             expected=np.stack([ep, eg, em, ev]).astype(np.float32))
    # layer norm over rows of 48: forward and the three gradients
    x = (rng.standard_normal((5, 48)) * 2.0 + 0.5).astype(np.float32)
    w = rng.standard_normal(48).astype(np.float32)
    b = rng.standard_normal(48).astype(np.float32)
    dy = rng.standard_normal((5, 48)).astype(np.float32)
    out, mu, rs = npr.layer_norm64(x, w, b, 1e-5)
    dx, dw, db = npr.layer_norm_backward64(dy, x, mu, rs, w)
    np.savez(os.path.join(HERE, "layer_norm.npz"), x=x, w=w, b=b, dy=dy, eps=np.float64(1e-5),
             out=out.astype(np.float32), mean=mu.astype(np.float32), rstd=rs.astype(np.float32),
             dx=dx.astype(np.float32), dw=dw.astype(np.float32), db=db.astype(np.float32))
    # log_softmax backward from a float64 log_softmax
    z = rng.standard_normal((4, 70))
    y = z - z.max(-1, keepdims=True)
    y = y - np.log(np.exp(y).sum(-1, keepdims=True))
    gy = rng.standard_normal((4, 70))
    np.savez(os.path.join(HERE, "log_softmax_backward.npz"), dy=gy.astype(np.float32),
             y=y.astype(np.float32),
             expected=npr.log_softmax_backward64(gy.astype(np.float32), y.astype(np.float32)).astype(np.float32))
    # cat of three int64 blocks along dim 1 (the brute-force walk)
    parts = [rng.integers(-2**62, 2**62, size=(3, k, 2)) for k in (2, 5, 1)]
    np.savez(os.path.join(HERE, "cat.npz"), a=parts[0], b=parts[1], c=parts[2],
             expected=npr.cat_brute(parts, 1))


if __name__ == "__main__":
    main()
