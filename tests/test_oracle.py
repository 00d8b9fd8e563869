"""Pins the CPU oracle before it is trusted (CPU only).

Each oracle function is checked against something that does not share its
code: a numpy restatement, a closed form, an invariant, brute force on tiny
inputs, or a committed golden fixture.  A planted mistake (dropped term,
wrong sign, swapped half, transposed operand) fails at least one of them,
see test_planted_mistakes_are_caught.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import aten, numpy_ref as npr
from oracle.tolerance import assert_close, assert_exact, bar, bar_ratio

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def g(seed=0):
    return torch.Generator().manual_seed(seed)


# ---- config 1 -----------------------------------------------------------------

def test_mul_add_bit_exact_vs_numpy():
    a = torch.rand(257, 129, generator=g(1)) * 2 - 1
    b = torch.rand(129, generator=g(2)) * 2 - 1
    got = aten.add(aten.mul(a, b), 0.5)
    want = npr.add(npr.mul(a.numpy(), b.numpy()), np.float32(0.5))
    assert_exact(got, torch.from_numpy(want), "a*b+0.5")


def test_add_alpha_and_sub_vs_numpy():
    a = torch.randn(1000, generator=g(3))
    b = torch.randn(1000, generator=g(4))
    # alpha = 1 and -1 are single roundings
    assert_exact(aten.sub(a, b), torch.from_numpy(np.subtract(a.numpy(), b.numpy())), "sub")
    assert_exact(aten.div(a, b), torch.from_numpy(np.divide(a.numpy(), b.numpy())), "div")


def test_index_select_vs_numpy_and_brute_force():
    table = torch.randint(-2**63, 2**63 - 1, (1000, 8), generator=g(5), dtype=torch.int64)
    idx = torch.randint(0, 1000, (300,), generator=g(6), dtype=torch.int64)
    got = aten.index_select(table, 0, idx)
    assert_exact(got, torch.from_numpy(npr.index_select(table.numpy(), 0, idx.numpy())), "take")
    small = table[:7]
    sidx = torch.tensor([6, 0, 0, 3, 6], dtype=torch.int64)
    assert_exact(aten.index_select(small, 0, sidx),
                 torch.from_numpy(npr.index_select_brute(small.numpy(), sidx.numpy())), "brute")
    # dim 1 gather
    assert_exact(aten.index_select(table, 1, torch.tensor([7, 1])),
                 torch.from_numpy(table.numpy()[:, [7, 1]]), "dim1")


def test_cat_vs_numpy_and_brute_force():
    a = torch.randint(-2**63, 2**63 - 1, (3, 5, 4), generator=g(40), dtype=torch.int64)
    b = torch.randint(-2**63, 2**63 - 1, (3, 2, 4), generator=g(41), dtype=torch.int64)
    c = torch.randint(-2**63, 2**63 - 1, (3, 7, 4), generator=g(42), dtype=torch.int64)
    for dim in (1, -2):
        got = aten.cat([a, b, c], dim)
        assert_exact(got, torch.from_numpy(np.concatenate([a.numpy(), b.numpy(), c.numpy()], 1)),
                     "concatenate")
        assert_exact(got, torch.from_numpy(npr.cat_brute([a.numpy(), b.numpy(), c.numpy()], dim)),
                     "brute")
    x = torch.randn(4, 3, generator=g(43))
    y = torch.randn(4, 5, generator=g(44))
    assert_exact(aten.cat([x, y], 1), torch.from_numpy(npr.cat_brute([x.numpy(), y.numpy()], 1)),
                 "last dim")
    # legacy: a 1-D empty input is skipped whatever the rank of the others
    assert_exact(aten.cat([x, torch.empty(0), x], 0), torch.from_numpy(np.concatenate([x.numpy()] * 2)),
                 "skip 1-D empty")
    # promotion: int32 with float32 gives float32 holding the converted ints
    i = torch.arange(-6, 6, dtype=torch.int32).reshape(4, 3)
    got = aten.cat([i, x], 0)
    assert got.dtype == torch.float32
    assert_exact(got, torch.from_numpy(np.concatenate([i.numpy().astype(np.float32), x.numpy()])),
                 "promotion")


def test_copy_casts_vs_numpy():
    x = torch.randn(64, 33, generator=g(45)) * 300
    for dt, npdt in [(torch.float16, np.float16), (torch.int32, np.int32), (torch.float64, np.float64),
                     (torch.int8, None), (torch.bool, np.bool_)]:
        got = aten.copy(torch.empty(64, 33, dtype=dt), x)
        if npdt is None:  # float -> int8 goes through int64 in ATen (wraps)
            want = x.numpy().astype(np.int64).astype(np.int8)
        else:
            want = x.numpy().astype(npdt)
        assert_exact(got, torch.from_numpy(want), f"cast {dt}")
    row = torch.randn(33, generator=g(46))
    assert_exact(aten.copy(torch.empty(5, 33), row),
                 torch.from_numpy(np.broadcast_to(row.numpy(), (5, 33)).copy()), "broadcast")


@pytest.mark.parametrize("amsgrad,maximize,scaled", [(False, False, False), (True, True, False),
                                                      (False, False, True)])
def test_fused_adamw_vs_float64_closed_form(amsgrad, maximize, scaled):
    shapes = [(37,), (8, 9)]
    p = [torch.randn(s, generator=g(60 + i)) for i, s in enumerate(shapes)]
    m = [torch.zeros(s) for s in shapes]
    v = [torch.zeros(s) for s in shapes]
    vm = [torch.zeros(s) for s in shapes] if amsgrad else []
    hp = dict(lr=2e-3, beta1=0.9, beta2=0.99, weight_decay=0.05, eps=1e-8, amsgrad=amsgrad,
              maximize=maximize)
    gs = torch.tensor(8.0) if scaled else None
    for step in (1, 2, 3):
        grads = [torch.randn(s, generator=g(70 + 10 * step + i)) for i, s in enumerate(shapes)]
        out = aten.fused_adamw(p, grads, m, v, vm, [torch.tensor(float(step))] * len(shapes),
                               grad_scale=gs, **hp)
        for i in range(len(shapes)):
            want = npr.adamw64(p[i].numpy(), grads[i].numpy(), m[i].numpy(), v[i].numpy(),
                               vm[i].numpy() if amsgrad else None, step, hp["lr"], hp["beta1"],
                               hp["beta2"], hp["weight_decay"], hp["eps"], amsgrad, maximize,
                               8.0 if scaled else None)
            for k, name in [(0, "param"), (2, "exp_avg"), (3, "exp_avg_sq")] + \
                    ([(1, "grad")] if scaled else []) + ([(4, "max_exp_avg_sq")] if amsgrad else []):
                assert_close(out[k][i].double(), torch.from_numpy(want[k]), "fp32", f"{name} step {step}")
        p, m, v = out[0], out[2], out[3]
        vm = out[4] if amsgrad else []
    # found_inf = 1 leaves everything as it was
    grads = [torch.randn(s, generator=g(99)) for s in shapes]
    out = aten.fused_adamw(p, grads, m, v, vm, [torch.tensor(4.0)] * 2, found_inf=torch.tensor(1.0),
                           grad_scale=gs, **hp)
    assert all(torch.equal(a, b) for a, b in zip(out[0], p))
    assert all(torch.equal(a, b) for a, b in zip(out[1], grads))


def test_backward_closed_forms_match_central_differences():
    """The float64 closed forms the backward oracles are pinned to are the
    derivatives of their forward ops (central differences on tiny inputs)."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 6))
    silu = lambda t: t / (1.0 + np.exp(-t))  # noqa: E731
    num, c = npr.central_difference(silu, x)
    assert np.abs(num - npr.silu_backward64(c, x)).max() < 1e-7

    def log_softmax(t):
        m = t.max(-1, keepdims=True)
        return t - m - np.log(np.exp(t - m).sum(-1, keepdims=True))
    num, c = npr.central_difference(log_softmax, x)
    assert np.abs(num - npr.log_softmax_backward64(c, log_softmax(x))).max() < 1e-7
    softmax = lambda t: np.exp(log_softmax(t))  # noqa: E731
    num, c = npr.central_difference(softmax, x)
    assert np.abs(num - npr.softmax_backward64(c, softmax(x))).max() < 1e-7

    w, b = rng.standard_normal(6), rng.standard_normal(6)
    num, c = npr.central_difference(lambda t: npr.layer_norm64(t, w, b, 1e-5)[0], x)
    _, mu, rs = npr.layer_norm64(x, w, b, 1e-5)
    dx, dw, db = npr.layer_norm_backward64(c, x, mu, rs, w)
    assert np.abs(num - dx).max() < 1e-6
    numw, _ = npr.central_difference(lambda ww: npr.layer_norm64(x, ww, b, 1e-5)[0], w)
    numb, _ = npr.central_difference(lambda bb: npr.layer_norm64(x, w, bb, 1e-5)[0], b)
    # the same random cotangent c (seeded) is used for every difference
    assert np.abs(numw - dw).max() < 1e-6 and np.abs(numb - db).max() < 1e-6


def test_backward_oracles_vs_float64():
    x = torch.randn(64, 333, generator=g(80))
    dy = torch.randn(64, 333, generator=g(81))
    assert_close(aten.silu_backward(dy, x).double(),
                 torch.from_numpy(npr.silu_backward64(dy.numpy(), x.numpy())), "fp32", "silu_backward")
    y = torch.log_softmax(x, -1)
    assert_close(aten.log_softmax_backward(dy, y, -1, torch.float32).double(),
                 torch.from_numpy(npr.log_softmax_backward64(dy.numpy(), y.numpy())), "fp32",
                 "log_softmax_backward")
    p = torch.softmax(x, 0)
    assert_close(aten.softmax_backward(dy, p, 0, torch.float32).double(),
                 torch.from_numpy(npr.softmax_backward64(dy.numpy(), p.numpy(), 0)), "fp32",
                 "softmax_backward dim 0")
    w, b = torch.randn(333, generator=g(82)), torch.randn(333, generator=g(83))
    out, mean, rstd = aten.layer_norm_forward(x, [333], w, b, 1e-5)
    dx, dw, db = aten.layer_norm_backward(dy, x, [333], mean, rstd, w, b, [True, True, True])
    rdx, rdw, rdb = npr.layer_norm_backward64(dy.numpy(), x.numpy(), mean.double().numpy(),
                                              rstd.double().numpy(), w.numpy())
    assert_close(dx.double(), torch.from_numpy(rdx), "fp32", "layer_norm dx")
    assert_close(dw.double(), torch.from_numpy(rdw), "fp32", "layer_norm dgamma")
    assert_close(db.double(), torch.from_numpy(rdb), "fp32", "layer_norm dbeta")


# ---- config 2 -------------------------------------------------------------------

def test_sum_amax_bf16_vs_float64():
    x = (torch.randn(64, 3000, generator=g(7)) * 4).bfloat16()
    s = aten.sum_(x, -1)
    assert s.dtype == torch.bfloat16
    ref = torch.from_numpy(npr.sum64(x.float().numpy(), -1)).bfloat16()
    assert_close(s, ref, "bf16", "sum")
    assert_exact(aten.amax(x, -1), torch.from_numpy(x.float().numpy().max(-1)).bfloat16(), "amax")


def test_sum_constant_row_closed_form_and_spike():
    x = torch.full((4, 32000), 0.25, dtype=torch.bfloat16)
    assert_exact(aten.sum_(x, -1), torch.full((4,), 8000.0, dtype=torch.bfloat16), "N*c")
    y = torch.zeros(3, 32000, dtype=torch.bfloat16)
    y[1, 12345] = 7.5
    assert_exact(aten.amax(y, -1), torch.tensor([0.0, 7.5, 0.0], dtype=torch.bfloat16), "spike")


def test_mean_dim0_vs_float64():
    m = torch.randn(2048, 256, generator=g(8))
    got = aten.mean(m, 0)
    ref = torch.from_numpy(npr.mean64(m.numpy(), 0)).float()
    assert_close(got, ref, "fp32", "mean0")


def test_log_softmax_vs_float64_and_invariants():
    x = (torch.randn(16, 32000, generator=g(9)) * 4).bfloat16()
    got = aten.log_softmax(x, -1)
    ref = torch.from_numpy(npr.log_softmax64(x.float().numpy())).bfloat16()
    assert_close(got, ref, "bf16", "log_softmax")
    # constant row: every entry is -ln(N)
    c = torch.full((2, 32000), 3.0)
    assert torch.allclose(aten.log_softmax(c, -1), torch.full((2, 32000), -math.log(32000.0)))
    # logsumexp of each output row is 0
    lse = torch.logsumexp(aten.log_softmax(x.float(), -1).double(), -1)
    assert lse.abs().max().item() < 1e-5
    sm = aten.softmax(x.float(), -1)
    assert (sm.double().sum(-1) - 1).abs().max().item() < 1e-5
    assert_close(sm, torch.from_numpy(npr.softmax64(x.float().numpy())).float(), "fp32", "softmax")


# ---- config 3 ------------------------------------------------------------------

def test_rms_norm_matches_torch_rms_norm_exactly():
    x = torch.randn(32, 4096, generator=g(10)).bfloat16()
    w = (torch.randn(4096, generator=g(11)) * 0.02 + 1).bfloat16()
    assert_exact(aten.rms_norm(x, w, 1e-6), torch.rms_norm(x, [4096], w, 1e-6), "rms_norm")
    ref = torch.from_numpy(npr.rms_norm64(x.float().numpy(), w.float().numpy(), 1e-6)).bfloat16()
    assert_close(aten.rms_norm(x, w, 1e-6), ref, "bf16", "rms_norm64")


def test_rope_invariants_and_float64():
    q = torch.randn(64, 4, 128, generator=g(12))
    pos = torch.arange(64) * 61
    out = aten.rope(q, pos, 10000.0)
    # position 0 is the identity
    assert torch.equal(out[0], q[0])
    # each (i, i + d/2) pair keeps its norm
    h = 64
    n_in = q[..., :h] ** 2 + q[..., h:] ** 2
    n_out = out[..., :h] ** 2 + out[..., h:] ** 2
    assert torch.allclose(n_in, n_out, rtol=1e-4, atol=1e-5)
    # fp32 angles at positions up to ~3900 carry ~1e-4 absolute error
    ref = torch.from_numpy(npr.rope64(q.numpy(), pos.numpy(), 10000.0)).float()
    assert (out.double() - ref.double()).abs().max().item() < 2e-3
    # rotating by p then by -p is the identity (composition law)
    back = aten.rope(out, -pos, 10000.0)
    assert torch.allclose(back, q, atol=1e-4)


def test_silu_mul_vs_float64():
    gt = torch.randn(64, 1000, generator=g(13)).bfloat16()
    up = torch.randn(64, 1000, generator=g(14)).bfloat16()
    ref = torch.from_numpy(npr.silu_mul64(gt.float().numpy(), up.float().numpy())).bfloat16()
    assert_close(aten.silu_mul(gt, up), ref, "bf16", "silu_mul")
    # silu(0) = 0, silu(x) -> x for large x
    z = torch.tensor([0.0, 20.0, -20.0])
    assert torch.allclose(aten.silu_mul(z, torch.ones(3)), torch.tensor([0.0, 20.0, -20.0 * math.exp(-20)]),
                          atol=1e-6)


# ---- config 4/5: contractions and attention ---------------------------------------

def test_addmm_bmm_vs_float64():
    a = torch.randn(64, 96, generator=g(20)).bfloat16()
    b = torch.randn(96, 48, generator=g(21)).bfloat16()
    bias = torch.randn(48, generator=g(22)).bfloat16()
    ref = npr.matmul64(a.float().numpy(), b.float().numpy()) * 0.5 + 2.0 * bias.double().numpy()
    assert_close(aten.addmm(bias, a, b, beta=2.0, alpha=0.5), torch.from_numpy(ref).bfloat16(),
                 "bf16", "addmm")
    a3 = torch.randn(3, 32, 40, generator=g(23)).bfloat16()
    b3 = torch.randn(3, 40, 24, generator=g(24)).bfloat16()
    ref3 = np.stack([npr.matmul64(a3[i].float().numpy(), b3[i].float().numpy()) for i in range(3)])
    assert_close(aten.bmm(a3, b3), torch.from_numpy(ref3).bfloat16(), "bf16", "bmm")
    # row sampling identity: rows of the product are products of rows
    assert_exact(aten.addmm(None, a[5:9], b), aten.addmm(None, a, b)[5:9], "addmm rows")


def test_addmv_vs_float64_and_ignored_operands():
    mat = torch.randn(70, 300, generator=g(90)).bfloat16()
    vec = torch.randn(300, generator=g(91)).bfloat16()
    bias = torch.randn(70, generator=g(92)).bfloat16()
    ref = npr.matmul64(mat.float().numpy(), vec.double().numpy()[:, None])[:, 0] * 0.5 \
        + 2.0 * bias.double().numpy()
    assert_close(aten.addmv(bias, mat, vec, beta=2.0, alpha=0.5), torch.from_numpy(ref).bfloat16(),
                 "bf16", "addmv")
    m32, v32 = mat.float(), vec.float()
    ref32 = npr.matmul64(m32.numpy(), v32.double().numpy()[:, None])[:, 0]
    assert_close(aten.addmv(None, m32, v32), torch.from_numpy(ref32).float(), "fp32", "mv")
    # beta = 0 ignores a NaN bias; alpha = 0 ignores NaN in mat
    nan_b = torch.full((70,), float("nan")).bfloat16()
    assert torch.isfinite(aten.addmv(nan_b, mat, vec, beta=0.0).float()).all()
    nan_m = mat.clone()
    nan_m[3, 7] = float("nan")
    assert_exact(aten.addmv(bias, nan_m, vec, beta=1.0, alpha=0.0), bias, "addmv alpha 0")


def test_int8_linear_vs_float64_and_weight_int8pack_mm():
    x = torch.randn(16, 128, generator=g(25)).bfloat16()
    w = torch.randint(-128, 128, (64, 128), generator=g(26), dtype=torch.int8)
    s = (torch.rand(64, generator=g(27)) * 0.01 + 1e-3).bfloat16()
    got = aten.int8_linear(x, w, s)
    ref = npr.matmul64(x.float().numpy(), w.float().numpy().T) * s.double().numpy()
    assert_close(got, torch.from_numpy(ref).bfloat16(), "bf16", "int8_linear")
    lib = torch.ops.aten._weight_int8pack_mm(x, w, s)
    assert_close(got, lib, "bf16", "int8_linear vs _weight_int8pack_mm")


@pytest.mark.parametrize("H,Hk,Sq,Sk,causal", [(4, 4, 64, 64, True), (4, 2, 64, 80, False),
                                               (2, 1, 33, 33, True), (2, 2, 1, 40, False)])
def test_sdpa_vs_float64(H, Hk, Sq, Sk, causal):
    q = torch.randn(2, H, Sq, 64, generator=g(28)).bfloat16()
    k = torch.randn(2, Hk, Sk, 64, generator=g(29)).bfloat16()
    v = torch.randn(2, Hk, Sk, 64, generator=g(30)).bfloat16()
    out, lse = aten.sdpa(q, k, v, causal)
    ro, rl = npr.attention64(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal)
    assert_close(out, torch.from_numpy(ro).bfloat16(), "bf16", "sdpa out")
    assert (lse.double() - torch.from_numpy(rl)).abs().max().item() < 1e-3
    if causal:  # query 0 sees key 0 only: out = v[0], lse = scale * q0.k0
        assert_exact(out[:, :, 0], v[:, torch.arange(H) * Hk // H, 0], "causal row 0")


@pytest.mark.parametrize("name", ["rms_norm", "rope", "silu_mul"])
def test_golden_fixtures(name):
    path = os.path.join(GOLDEN, f"{name}.npz")
    data = np.load(path)
    if name == "rms_norm":
        got = aten.rms_norm(torch.from_numpy(data["x"]), torch.from_numpy(data["w"]),
                            float(data["eps"]))
    elif name == "rope":
        got = aten.rope(torch.from_numpy(data["x"]), torch.from_numpy(data["pos"]),
                        float(data["theta"]))
    else:
        got = aten.silu_mul(torch.from_numpy(data["gate"]), torch.from_numpy(data["up"]))
    want = torch.from_numpy(data["expected"])
    if name == "rope":
        # the fp32 closed form rounds pos * inv_freq to fp32: at pos 4095 the
        # angle is off by up to 4095 * 2^-24 rad, so compare absolutely
        assert (got.double() - want.double()).abs().max().item() < 1e-3
    else:
        assert_close(got, want, "fp32", name)


def test_golden_training_fixtures():
    """CPU ATen on the committed float64 fixtures of the training-side ops and
    cat (tests/golden/make_golden.py)."""
    d = np.load(os.path.join(GOLDEN, "adamw.npz"))
    hp = d["hp"]
    t = lambda k: torch.from_numpy(d[k])  # noqa: E731
    out = aten.fused_adamw([t("p")], [t("g")], [t("m")], [t("v")], [], [torch.tensor(float(hp[5]))],
                           lr=float(hp[0]), beta1=float(hp[1]), beta2=float(hp[2]),
                           weight_decay=float(hp[3]), eps=float(hp[4]), amsgrad=False,
                           maximize=False, grad_scale=torch.tensor(float(hp[6])))
    for k, name in enumerate(("param", "grad", "exp_avg", "exp_avg_sq")):
        assert_close(out[k][0], torch.from_numpy(d["expected"][k]), "fp32", f"adamw {name}")
    d = np.load(os.path.join(GOLDEN, "layer_norm.npz"))
    x, w, b, dy = (torch.from_numpy(d[k]) for k in ("x", "w", "b", "dy"))
    y, mean, rstd = aten.layer_norm_forward(x, [48], w, b, float(d["eps"]))
    assert_close(y, torch.from_numpy(d["out"]), "fp32", "layer_norm out")
    assert_close(mean, torch.from_numpy(d["mean"]), "fp32", "layer_norm mean")
    assert_close(rstd, torch.from_numpy(d["rstd"]), "fp32", "layer_norm rstd")
    dx, dw, db = aten.layer_norm_backward(dy, x, [48], mean, rstd, w, b, [True, True, True])
    for got, k in ((dx, "dx"), (dw, "dw"), (db, "db")):
        assert_close(got, torch.from_numpy(d[k]), "fp32", f"layer_norm {k}")
    d = np.load(os.path.join(GOLDEN, "log_softmax_backward.npz"))
    assert_close(aten.log_softmax_backward(torch.from_numpy(d["dy"]), torch.from_numpy(d["y"]), -1,
                                           torch.float32),
                 torch.from_numpy(d["expected"]), "fp32", "log_softmax_backward")
    d = np.load(os.path.join(GOLDEN, "cat.npz"))
    assert_exact(aten.cat([torch.from_numpy(d[k]) for k in ("a", "b", "c")], 1),
                 torch.from_numpy(d["expected"]), "cat")


def test_planted_mistakes_are_caught():
    """Mutated oracles must fail the same pins."""
    q = torch.randn(8, 2, 16, generator=g(15))
    pos = torch.arange(8)
    ref = torch.from_numpy(npr.rope64(q.numpy(), pos.numpy(), 10000.0)).float()

    def rope_wrong_sign(x, p, th):
        d = x.shape[-1]
        h = d // 2
        cos, sin = aten.rope_tables(p, d, th)
        x1, x2 = x[..., :h], x[..., h:]
        return torch.cat([x1 * cos[:, None] + x2 * sin[:, None], x2 * cos[:, None] + x1 * sin[:, None]], -1)

    assert (rope_wrong_sign(q, pos, 10000.0) - ref).abs().max() > 1e-2
    x = torch.randn(4, 64, generator=g(16))
    ref_rms = torch.from_numpy(npr.rms_norm64(x.numpy(), None, 1e-6)).float()
    dropped_mean = x * torch.rsqrt(x.pow(2).sum(-1, keepdim=True) + 1e-6)
    assert (dropped_mean - ref_rms).abs().max() > 1e-2
    table = torch.arange(36).reshape(6, 6)
    idx = torch.tensor([3, 1, 5])
    want = torch.from_numpy(npr.index_select(table.numpy(), 0, idx.numpy()))
    assert not torch.equal(aten.index_select(table, 1, idx), want)  # transposed gather
    q = torch.randn(1, 2, 16, 32, generator=g(17))
    ro, _ = npr.attention64(q.numpy(), q.numpy(), q.numpy(), True)
    unscaled = torch.softmax((q @ q.transpose(-1, -2)).masked_fill(
        torch.ones(16, 16, dtype=torch.bool).triu(1), float("-inf")), -1) @ q
    assert (unscaled.double() - torch.from_numpy(ro)).abs().max() > 1e-2  # dropped 1/sqrt(d)
    p1, p2 = torch.arange(6).reshape(2, 3), torch.arange(6, 10).reshape(2, 2)
    want = torch.from_numpy(npr.cat_brute([p1.numpy(), p2.numpy()], 1))
    assert not torch.equal(aten.cat([p2, p1], 1), want)  # inputs in the wrong order
    # AdamW without the first-moment bias correction misses the closed form
    pa, ga = torch.randn(16, generator=g(18)), torch.randn(16, generator=g(19))
    want = npr.adamw64(pa.numpy(), ga.numpy(), np.zeros(16), np.zeros(16), None, 1, 1e-2, 0.9,
                       0.999, 0.0, 1e-8, False, False)[0]
    no_bc1 = pa.double() - 1e-2 * (0.1 * ga.double()) / (
        (0.001 * ga.double() ** 2).sqrt() / math.sqrt(0.001) + 1e-8)
    assert (no_bc1 - torch.from_numpy(want)).abs().max() > 1e-3
    # a layer-norm gradient without the xh * mean(gw * xh) term misses its central difference
    rng = np.random.default_rng(4)
    xs = rng.standard_normal((2, 5))
    num, c = npr.central_difference(lambda t: npr.layer_norm64(t, None, None, 1e-5)[0], xs)
    _, mu, rs = npr.layer_norm64(xs, None, None, 1e-5)
    dropped = rs * (c - c.sum(-1, keepdims=True) / 5)
    assert np.abs(num - dropped).max() > 1e-2


# ---- foreach and mixed-precision grad scaling ------------------------------------------

KIND = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_foreach_add_mul_vs_float32_closed_form(dtype):
    ts = [torch.randn(s, generator=g(60 + i)).to(dtype) for i, s in enumerate([(7,), (33, 5), ()])]
    for value in (0.3, -1.75, 1e-3):
        got = aten.foreach_add_scalar(ts, value)
        for a, t in zip(got, ts):
            want = npr.foreach_binary32(t.float().numpy(), value, "add", KIND[dtype])
            assert_exact(a.float(), torch.from_numpy(np.asarray(want)).reshape(t.shape),
                         f"foreach_add {dtype} {value}")
        got = aten.foreach_mul(ts, value)
        for a, t in zip(got, ts):
            want = npr.foreach_binary32(t.float().numpy(), value, "mul", KIND[dtype])
            assert_exact(a.float(), torch.from_numpy(np.asarray(want)).reshape(t.shape),
                         f"foreach_mul {dtype} {value}")
    # a 0-dim float32 tensor factor keeps its float value (not rounded to the
    # list's dtype as a Python number is)
    for a, t in zip(aten.foreach_mul(ts, torch.tensor(0.37)), ts):
        want = npr.foreach_binary32(t.float().numpy(), 0.37, "mul", KIND[dtype], round_scalar=False)
        assert_exact(a.float(), torch.from_numpy(np.asarray(want)).reshape(t.shape),
                     f"foreach_mul tensor factor {dtype}")
    # identities
    for a, t in zip(aten.foreach_add_scalar(ts, 0.0), ts):
        assert_exact(a, t, "x + 0")
    for a, t in zip(aten.foreach_mul(ts, -1.0), ts):
        assert_exact(a, -t, "x * -1")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_amp_unscale_vs_float32_closed_form(dtype):
    grads = [(torch.randn(s, generator=g(70 + i)) * 512).to(dtype)
             for i, s in enumerate([(9,), (4, 6), ()])]
    for inv, poison in ((1.0 / 512, None), (1.0 / 3, float("inf")), (1.0, float("nan")),
                        (0.25, float("-inf"))):
        gs = [t.clone() for t in grads]
        if poison is not None:
            gs[1].view(-1)[5] = poison
        got, fi = aten.amp_unscale(gs, torch.zeros(1), torch.tensor([inv]))
        want, found = npr.amp_unscale_ref([t.float().numpy() for t in gs], inv, KIND[dtype])
        assert float(fi) == found == (0.0 if poison is None else 1.0)
        for a, w in zip(got, want):
            a32, w32 = a.float(), torch.from_numpy(np.asarray(w, dtype=np.float32)).reshape(a.shape)
            same = (a32 == w32) | (torch.isnan(a32) & torch.isnan(w32))
            assert bool(same.all()), f"unscale {dtype} inv={inv}"
        if inv == 1.0:
            for a, t in zip(got, gs):
                assert_exact(a, t, "inv_scale 1 leaves values")


def test_amp_update_scale_vs_state_machine_and_worked_steps():
    # hand-worked: growth 2, backoff 0.5, interval 3 from 65536
    steps = [0, 0, 0, 1, 0, 0, 0, 0, 1, 1]
    worked = [(65536.0, 1), (65536.0, 2), (131072.0, 0), (65536.0, 0), (65536.0, 1),
              (65536.0, 2), (131072.0, 0), (131072.0, 1), (65536.0, 0), (32768.0, 0)]
    for start, table in ((65536.0, worked), (3.0e38, None), (1.0, None)):
        s, t = torch.tensor([start]), torch.tensor([0], dtype=torch.int32)
        rs, rt = float(np.float32(start)), 0
        for k, bad in enumerate(steps):
            s, t = aten.amp_update_scale(s, t, torch.tensor([float(bad)]), 2.0, 0.5, 3)
            rs, rt = npr.amp_update_scale_ref(rs, rt, float(bad), 2.0, 0.5, 3)
            assert (float(s), int(t)) == (rs, rt), (start, k)
            if table is not None:
                assert (float(s), int(t)) == table[k], (start, k)
    # a growth that overflows float32 is not taken, but the count restarts
    s, t = aten.amp_update_scale(torch.tensor([3.0e38]), torch.tensor([2], dtype=torch.int32),
                                 torch.tensor([0.0]), 2.0, 0.5, 3)
    assert float(s) == float(np.float32(3.0e38)) and int(t) == 0


def test_planted_mistakes_in_grad_scaling_are_caught():
    # a back-off that forgets to reset the count, and a growth taken even
    # when it overflows, each leave the worked sequence
    def forgetful(scale, tracker, found, growth, backoff, interval):
        if found:
            return float(np.float32(scale * backoff)), tracker
        return npr.amp_update_scale_ref(scale, tracker, found, growth, backoff, interval)

    s, t, s2, t2 = 65536.0, 0, 65536.0, 0
    diverged = False
    for bad in [0, 0, 1, 0, 0, 0]:
        s, t = npr.amp_update_scale_ref(s, t, bad, 2.0, 0.5, 3)
        s2, t2 = forgetful(s2, t2, bad, 2.0, 0.5, 3)
        diverged |= (s, t) != (s2, t2)
    assert diverged
    grown = float(np.float32(3.0e38) * np.float32(2.0))
    assert not math.isfinite(grown)
    assert npr.amp_update_scale_ref(3.0e38, 2, 0.0, 2.0, 0.5, 3)[0] != grown
    # unscaling with the scale instead of its inverse misses the closed form
    g0 = [np.array([512.0, -1024.0], dtype=np.float32)]
    assert not np.array_equal(npr.amp_unscale_ref(g0, 1 / 512, "f32")[0][0], g0[0] * 512)


# ---- int32 advanced index ------------------------------------------------------------

INDEX_CASES = [
    ("rows", (7, 5), lambda r: [r.integers(-7, 7, (4,))]),
    ("2-D index", (6, 4, 3), lambda r: [r.integers(0, 6, (2, 3))]),
    ("middle dim", (3, 8, 2), lambda r: [None, r.integers(-8, 8, (5,))]),
    ("two broadcast", (5, 6, 2), lambda r: [r.integers(0, 5, (3, 1)), r.integers(0, 6, (4,))]),
    ("non-adjacent", (4, 3, 5, 2), lambda r: [r.integers(0, 4, (2, 2)), None, r.integers(0, 5, (2,))]),
    ("0-dim index", (5, 3), lambda r: [np.array(3)]),
    ("last dim", (2, 3, 9), lambda r: [None, None, r.integers(0, 9, (4,))]),
]


@pytest.mark.parametrize("name", [c[0] for c in INDEX_CASES])
def test_int32_indices_index_vs_numpy_and_brute_force(name):
    _, shape, mk = next(c for c in INDEX_CASES if c[0] == name)
    rng = np.random.default_rng(abs(hash(name)) % 1000)
    arr = rng.integers(-2**62, 2**62, shape)
    idx = mk(rng)
    t_idx = [None if i is None else torch.from_numpy(np.asarray(i, dtype=np.int32)) for i in idx]
    got = aten.int32_indices_index(torch.from_numpy(arr), t_idx)
    assert np.array_equal(got.numpy(), npr.adv_index(arr, idx)), name
    assert np.array_equal(got.numpy(), npr.adv_index_brute(arr, idx)), name


def test_int32_indices_index_planted_mistake_non_adjacent_order():
    # placing B in the position of the first indexed dim even when the
    # indexed dims are not adjacent gives another shape than the brute force
    arr = np.arange(4 * 3 * 5).reshape(4, 3, 5)
    idx = [np.array([0, 1]), None, np.array([2, 4])]
    want = npr.adv_index_brute(arr, idx)
    assert want.shape == (2, 3)
    wrong = np.stack([arr[idx[0][j], :, idx[2][j]] for j in range(2)], 0)  # same here...
    wrong_layout = np.moveaxis(wrong, 0, 1)  # ...but B placed second
    assert wrong_layout.shape != want.shape or not np.array_equal(wrong_layout, want)


# ---- the CPU fallback widened to float ------------------------------------------------

@pytest.mark.parametrize("low", [torch.float16, torch.bfloat16])
def test_widened_fallback_vs_float64_closed_forms(low):
    import scipy.special

    # integer-valued matrix: the diagonal sum is exact in every precision
    m = torch.randint(-8, 9, (12, 12), generator=g(80)).to(low)
    t = aten.widened_fallback(torch.trace, m)
    assert t.dtype == low and t.dim() == 0
    assert float(t) == float(np.trace(m.double().numpy()))
    x = (torch.rand(500, generator=g(81)) * 6 - 2).to(low)
    got = aten.widened_fallback(torch.special.erfcx, x)
    assert got.dtype == low
    ref = torch.from_numpy(scipy.special.erfcx(x.double().numpy())).to(low)
    # float32 erfcx rounded to 16 bits vs float64 rounded to 16 bits: at most
    # one unit in the last place apart
    ulp = (ref.double().abs() * (2.0 ** -10 if low == torch.float16 else 2.0 ** -7)).clamp_min(1e-30)
    assert bool(((got.double() - ref.double()).abs() <= ulp).all())
    # a planted mistake: forgetting to round the result back leaves float32
    assert torch.special.erfcx(x.float()).dtype != low


def test_bar_ratio_agrees_with_assert_close():
    """bar_ratio <= 1 exactly when assert_close passes: an error of k times
    the bar at one element gives ratio k (hand-computed bar: rtol 1e-2 and
    atol 1e-2 * rms of the reference)."""
    e = torch.tensor([3.0, -4.0, 0.0, 0.5], dtype=torch.float64)
    rms = math.sqrt((9 + 16 + 0 + 0.25) / 4)
    assert bar(e, "bf16") == (1e-2, pytest.approx(1e-2 * rms))
    for k in (0.5, 0.99, 1.01, 3.0):
        a = e.clone()
        a[2] = k * 1e-2 * rms  # error at the zero element is k times the floor
        assert bar_ratio(a, e, "bf16") == pytest.approx(k)
        if k <= 1:
            assert_close(a, e, "bf16")
        else:
            with pytest.raises(AssertionError):
                assert_close(a, e, "bf16")
    a = e.clone()
    a[1] = -4.0 * (1 + 2 * 1e-2) - 1e-2 * rms  # past rtol|ref| + atol by 4e-2
    assert bar_ratio(a, e, "bf16") == pytest.approx((8e-2 + 1e-2 * rms) / (4e-2 + 1e-2 * rms))
