"""numpy restatements of the path's arithmetic, used to pin ``oracle.aten``.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

bfloat16 values are carried as float32 arrays holding exactly representable
bf16 numbers; ``round_bf16`` applies round-to-nearest-even to 8 mantissa bits
(the rounding c10::BFloat16 uses).
"""
from __future__ import annotations

import numpy as np


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bfloat16, returned as float32 (NaN -> qNaN)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    out = (r.astype(np.uint32) << 16).view(np.float32)
    return np.where(np.isnan(x), np.float32(np.nan), out)


def mul(a, b):
    return np.multiply(a, b, dtype=np.float32)


def add(a, b, alpha=1.0):
    if alpha == 1.0:
        return np.add(a, b, dtype=np.float32)
    return np.add(a, np.float32(alpha) * np.asarray(b, dtype=np.float32), dtype=np.float32)


def index_select(table: np.ndarray, dim: int, idx: np.ndarray) -> np.ndarray:
    return np.take(table, idx, axis=dim)


def index_select_brute(table: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """Row gather by explicit loops (tiny inputs only)."""
    out = np.empty((len(idx),) + table.shape[1:], dtype=table.dtype)
    for i, j in enumerate(idx):
        out[i] = table[j]
    return out


def cat_brute(arrays, dim: int) -> np.ndarray:
    """Concatenation by an explicit walk over output positions along dim (tiny
    inputs only): position j of out comes from the input whose range holds j."""
    nd = arrays[0].ndim
    dim = dim % nd
    total = sum(a.shape[dim] for a in arrays)
    shape = list(arrays[0].shape)
    shape[dim] = total
    out = np.empty(shape, dtype=np.result_type(*arrays))
    for j in range(total):
        k, base = 0, 0
        while j >= base + arrays[k].shape[dim]:
            base += arrays[k].shape[dim]
            k += 1
        src = [slice(None)] * nd
        dst = [slice(None)] * nd
        src[dim] = j - base
        dst[dim] = j
        out[tuple(dst)] = arrays[k][tuple(src)]
    return out


def sum64(x, axis):
    return np.sum(np.asarray(x, dtype=np.float64), axis=axis)


def mean64(x, axis):
    return np.mean(np.asarray(x, dtype=np.float64), axis=axis)


def log_softmax64(x, axis=-1):
    x = np.asarray(x, dtype=np.float64)
    m = np.max(x, axis=axis, keepdims=True)
    return x - m - np.log(np.sum(np.exp(x - m), axis=axis, keepdims=True))


def softmax64(x, axis=-1):
    return np.exp(log_softmax64(x, axis))


def rms_norm64(x, w, eps):
    x = np.asarray(x, dtype=np.float64)
    y = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    if w is not None:
        y = y * np.asarray(w, dtype=np.float64)
    return y


def rope64(x, positions, theta):
    x = np.asarray(x, dtype=np.float64)
    d = x.shape[-1]
    h = d // 2
    inv = 1.0 / (theta ** (np.arange(0, d, 2, dtype=np.float64) / d))
    ang = np.asarray(positions, dtype=np.float64)[:, None] * inv[None, :]
    c = np.cos(ang)[:, None, :]
    s = np.sin(ang)[:, None, :]
    x1, x2 = x[..., :h], x[..., h:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)


def silu_mul64(g, u):
    g = np.asarray(g, dtype=np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(u, dtype=np.float64)


def matmul64(a, b):
    return np.asarray(a, dtype=np.float64) @ np.asarray(b, dtype=np.float64)


def attention64(q, k, v, causal, scale=None):
    """softmax(scale q k^T + mask) v in float64 for [B, H, Sq, D] q and
    [B, Hk, Sk, D] k/v (query head h reads kv head h * Hk // H); the causal
    mask is top-left aligned (key j visible to query i when j <= i).
    Returns (out, lse) with lse the natural-log row log-sum-exp."""
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    H, Hk = q.shape[1], k.shape[1]
    idx = np.arange(H) * Hk // H
    k, v = k[:, idx], v[:, idx]
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    s = np.einsum("bhqd,bhkd->bhqk", q, k) * scale
    if causal:
        Sq, Sk = s.shape[-2:]
        s = np.where(np.arange(Sk)[None, :] > np.arange(Sq)[:, None], -np.inf, s)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    z = e.sum(-1, keepdims=True)
    return np.einsum("bhqk,bhkd->bhqd", e / z, v), (m + np.log(z))[..., 0]


def adamw64(p, g, m, v, vmax, step, lr, beta1, beta2, wd, eps, amsgrad, maximize,
            grad_scale=None, found_inf=None):
    """One AdamW step in float64 (Loshchilov and Hutter's decoupled weight
    decay with Adam's bias corrections, as torch.optim.AdamW documents it).
    Returns (p, g, m, v, vmax); g comes back unscaled when grad_scale is given."""
    p, g, m, v = (np.asarray(x, dtype=np.float64).copy() for x in (p, g, m, v))
    vmax = None if vmax is None else np.asarray(vmax, dtype=np.float64).copy()
    if found_inf is not None and found_inf == 1.0:
        return p, g, m, v, vmax
    if grad_scale is not None:
        g = g / grad_scale
    d = -g if maximize else g
    p = p * (1.0 - lr * wd)
    m = beta1 * m + (1.0 - beta1) * d
    v = beta2 * v + (1.0 - beta2) * d * d
    bc1 = 1.0 - beta1 ** step
    bc2 = 1.0 - beta2 ** step
    if amsgrad:
        vmax = np.maximum(vmax, v)
        den = np.sqrt(vmax) / np.sqrt(bc2) + eps
    else:
        den = np.sqrt(v) / np.sqrt(bc2) + eps
    p = p - (lr / bc1) * m / den
    return p, g, m, v, vmax


def silu_backward64(dy, x):
    x = np.asarray(x, dtype=np.float64)
    s = 1.0 / (1.0 + np.exp(-x))
    return np.asarray(dy, dtype=np.float64) * s * (1.0 + x * (1.0 - s))


def log_softmax_backward64(dy, y, axis=-1):
    dy = np.asarray(dy, dtype=np.float64)
    return dy - np.exp(np.asarray(y, dtype=np.float64)) * dy.sum(axis=axis, keepdims=True)


def softmax_backward64(dy, y, axis=-1):
    dy, y = np.asarray(dy, dtype=np.float64), np.asarray(y, dtype=np.float64)
    return y * (dy - (dy * y).sum(axis=axis, keepdims=True))


def layer_norm64(x, w, b, eps):
    """Rows of the last axis: (out, mean, rstd)."""
    x = np.asarray(x, dtype=np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=-1, keepdims=True)
    rs = 1.0 / np.sqrt(var + eps)
    out = (x - mu) * rs
    if w is not None:
        out = out * np.asarray(w, dtype=np.float64)
    if b is not None:
        out = out + np.asarray(b, dtype=np.float64)
    return out, mu, rs


def layer_norm_backward64(dy, x, mu, rs, w):
    """Closed form of the layer-norm gradient over the last axis (float64):
    returns (dx, dgamma, dbeta) with dgamma / dbeta summed over all rows."""
    dy = np.asarray(dy, dtype=np.float64)
    x = np.asarray(x, dtype=np.float64)
    n = x.shape[-1]
    xh = (x - mu) * rs
    gw = dy * (np.asarray(w, dtype=np.float64) if w is not None else 1.0)
    dx = rs * (gw - gw.sum(-1, keepdims=True) / n - xh * (gw * xh).sum(-1, keepdims=True) / n)
    rows = dy.reshape(-1, n)
    return dx, (rows * xh.reshape(-1, n)).sum(0), rows.sum(0)


def central_difference(f, x, eps=1e-6):
    """d(sum(f(x) * c)) / dx for a fixed random c, by central differences
    (float64, tiny inputs only); returns (grad, c)."""
    x = np.asarray(x, dtype=np.float64)
    c = np.random.default_rng(7).standard_normal(np.shape(f(x)))
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        xp, xm = x.copy(), x.copy()
        xp[i] += eps
        xm[i] -= eps
        g[i] = ((f(xp) * c).sum() - (f(xm) * c).sum()) / (2 * eps)
    return g, c


def round_to(x: np.ndarray, kind: str) -> np.ndarray:
    """float32 values rounded once to 'f32', 'bf16' or 'f16' (as float32)."""
    x = np.asarray(x, dtype=np.float32)
    if kind == "bf16":
        return round_bf16(x)
    if kind == "f16":
        return x.astype(np.float16).astype(np.float32)
    return x


def foreach_binary32(x, value, op: str, kind: str, round_scalar: bool = True) -> np.ndarray:
    """x (op) value in float32, rounded once to `kind`: the foreach add / mul
    of 16- and 32-bit floats.  A Python-number operand is first rounded to
    the list's dtype (round_scalar); a 0-dim float32 tensor operand is not."""
    a = np.asarray(x, dtype=np.float32)
    v = round_to(np.float32(value), kind) if round_scalar else np.float32(value)
    r = a + v if op == "add" else a * v
    return round_to(r, kind)


def amp_unscale_ref(grads, inv_scale: float, kind: str):
    """(grads * inv_scale in float32 rounded to `kind`, 1.0 if any element of
    the input grads is inf or NaN else 0.0); inv_scale == 1 leaves values as
    they are."""
    found = 0.0
    out = []
    for g in grads:
        g = np.asarray(g, dtype=np.float32)
        if not np.all(np.isfinite(g)):
            found = 1.0
        out.append(g.copy() if inv_scale == 1.0 else round_to(g * np.float32(inv_scale), kind))
    return out, found


def amp_update_scale_ref(scale: float, tracker: int, found_inf: float, growth: float,
                         backoff: float, interval: int):
    """One GradScaler update (torch.amp.GradScaler's documented rule): on inf
    the scale backs off and the count restarts; otherwise the count grows and,
    at `interval`, the scale grows (kept only if the float32 result is
    finite) and the count restarts.  Products in float64, rounded to float32."""
    if found_inf:
        return float(np.float32(scale * backoff)), 0
    tracker += 1
    if tracker == interval:
        grown = np.float32(scale * growth)
        if np.isfinite(grown):
            scale = float(grown)
        return scale, 0
    return scale, tracker


def adv_index(arr: np.ndarray, indices) -> np.ndarray:
    """numpy advanced indexing: arr[i0, :, i2, ...] with None for ':'."""
    key = tuple(slice(None) if i is None else np.asarray(i) for i in indices)
    return arr[key]


def adv_index_brute(arr: np.ndarray, indices) -> np.ndarray:
    """The same by explicit loops over output positions: the defined indices
    broadcast to one shape B; B replaces the indexed dims in place when they
    are adjacent, else comes first; negative indices count from the end."""
    import itertools

    idx = list(indices) + [None] * (arr.ndim - len(indices))
    kdims = [d for d, i in enumerate(idx) if i is not None]
    bs = np.broadcast_arrays(*[np.asarray(idx[d]) for d in kdims])
    bshape = bs[0].shape
    adjacent = kdims == list(range(kdims[0], kdims[-1] + 1))
    rest = [d for d in range(arr.ndim) if idx[d] is None]
    if adjacent:
        before = [d for d in rest if d < kdims[0]]
        after = [d for d in rest if d > kdims[-1]]
        layout = [("s", d) for d in before] + [("b", j) for j in range(len(bshape))] + \
                 [("s", d) for d in after]
    else:
        layout = [("b", j) for j in range(len(bshape))] + [("s", d) for d in rest]
    oshape = tuple(arr.shape[x] if kind == "s" else bshape[x] for kind, x in layout)
    out = np.empty(oshape, dtype=arr.dtype)
    for pos in itertools.product(*[range(n) for n in oshape]):
        src = [0] * arr.ndim
        bpos = [0] * len(bshape)
        for (kind, x), c in zip(layout, pos):
            if kind == "s":
                src[x] = c
            else:
                bpos[x] = c
        for k, d in enumerate(kdims):
            v = int(bs[k][tuple(bpos)])
            src[d] = v + arr.shape[d] if v < 0 else v
        out[pos] = arr[tuple(src)]
    return out
