"""torch._fused_adamw_ and torch.optim.AdamW(fused=True) on the gcu device,
against CPU ATen's fused AdamW (oracle.aten.fused_adamw) on the same inputs:
fp32 / fp64 within the fp32 bar, bf16 / fp16 within the bf16 bar (a stored
value may differ by one rounding of the fp32 result)."""
import pytest
import torch

import torch_gcu
from oracle import aten
from oracle.tolerance import assert_close, assert_exact

pytestmark = pytest.mark.gpu

C = torch_gcu._C

SHAPES = [(1000,), (33, 65), (4096, 130), (7,), (0,), (3, 5, 17), (8,)]


def g(seed):
    return torch.Generator().manual_seed(seed)


def make_lists(dtype, amsgrad, seed, shapes=SHAPES):
    p = [torch.randn(s, generator=g(seed + i)).to(dtype) for i, s in enumerate(shapes)]
    m = [(torch.randn(s, generator=g(seed + 100 + i)) * 0.01).to(dtype) for i, s in enumerate(shapes)]
    v = [(torch.rand(s, generator=g(seed + 200 + i)) * 1e-4).to(dtype) for i, s in enumerate(shapes)]
    vm = [(torch.rand(s, generator=g(seed + 300 + i)) * 1e-4).to(dtype) for i, s in enumerate(shapes)] \
        if amsgrad else []
    return p, m, v, vm


def bar_of(dtype):
    return "fp32" if dtype in (torch.float32, torch.float64) else "bf16"


CONFIGS = {
    "plain": dict(amsgrad=False, maximize=False, wd=0.01, scaled=False, lr="float"),
    "amsgrad_maximize": dict(amsgrad=True, maximize=True, wd=0.1, scaled=False, lr="float"),
    "grad_scale": dict(amsgrad=False, maximize=False, wd=0.01, scaled=True, lr="float"),
    "no_decay_lr_on_gcu": dict(amsgrad=False, maximize=False, wd=0.0, scaled=False, lr="gcu"),
    "lr_on_cpu": dict(amsgrad=True, maximize=False, wd=0.01, scaled=True, lr="cpu"),
}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
@pytest.mark.parametrize("cfg", list(CONFIGS))
def test_fused_adamw_parity(dtype, cfg):
    c = CONFIGS[cfg]
    p, m, v, vm = make_lists(dtype, c["amsgrad"], 10)
    dev = [[t.to("gcu") for t in lst] for lst in (p, m, v, vm)]
    hp = dict(beta1=0.9, beta2=0.999, weight_decay=c["wd"], eps=1e-8, amsgrad=c["amsgrad"],
              maximize=c["maximize"])
    lr = 1e-3
    gs = torch.tensor(1024.0) if c["scaled"] else None
    for step in (1, 2, 3):
        grads = [(torch.randn(s, generator=g(50 + 10 * step + i)) * (1024.0 if c["scaled"] else 1.0)).to(dtype)
                 for i, s in enumerate(SHAPES)]
        dgrads = [t.to("gcu") for t in grads]
        steps = [torch.tensor(float(step)) for _ in SHAPES]
        want = aten.fused_adamw(p, grads, m, v, vm, steps, lr=lr, grad_scale=gs, **hp)
        lr_arg = {"float": lr, "gcu": torch.tensor(lr, device="gcu"), "cpu": torch.tensor(lr)}[c["lr"]]
        torch._fused_adamw_(dev[0], dgrads, dev[1], dev[2], dev[3], [s.to("gcu") for s in steps],
                            lr=lr_arg, grad_scale=None if gs is None else gs.to("gcu"), **hp)
        torch.gcu.synchronize()
        for k, name, lst in [(0, "param", dev[0]), (2, "exp_avg", dev[1]), (3, "exp_avg_sq", dev[2])] + \
                ([(1, "grad", dgrads)] if c["scaled"] else []) + \
                ([(4, "max_exp_avg_sq", dev[3])] if c["amsgrad"] else []):
            for i, s in enumerate(SHAPES):
                assert_close(lst[i].cpu(), want[k][i], bar_of(dtype), f"{cfg} {name} {s} step {step}")
        if not c["scaled"]:
            for i in range(len(SHAPES)):  # grads untouched without grad_scale
                assert torch.equal(dgrads[i].cpu(), grads[i])
        p, m, v = want[0], want[2], want[3]
        vm = want[4] if c["amsgrad"] else []


def test_fused_adamw_found_inf_many_tensors_and_misaligned():
    """found_inf = 1 leaves every tensor untouched; 40 tensors span two
    launches; a tensor at an address that is not 16-byte aligned takes the
    element path."""
    shapes = [(17 + 3 * i,) for i in range(40)]
    p, m, v, _ = make_lists(torch.float32, False, 30, shapes)
    base = torch.randn(1 + 4096, generator=g(31))
    p.append(base[1:])  # 4-byte offset
    m.append(torch.zeros(4096))
    v.append(torch.zeros(4096))
    shapes.append((4096,))
    grads = [torch.randn(s, generator=g(400 + i)) for i, s in enumerate(shapes)]
    hp = dict(lr=1e-2, beta1=0.8, beta2=0.95, weight_decay=0.02, eps=1e-6, amsgrad=False, maximize=False)
    dbase = base.to("gcu")
    dp = [t.to("gcu") for t in p[:-1]] + [dbase[1:]]
    dm, dv, dg = ([t.to("gcu") for t in lst] for lst in (m, v, grads))
    steps = [torch.tensor(1.0, device="gcu") for _ in shapes]
    torch._fused_adamw_(dp, dg, dm, dv, [], steps, found_inf=torch.tensor(1.0, device="gcu"), **hp)
    torch.gcu.synchronize()
    assert all(torch.equal(a.cpu(), b) for a, b in zip(dp, p))
    torch._fused_adamw_(dp, dg, dm, dv, [], steps, found_inf=torch.tensor(0.0, device="gcu"), **hp)
    want = aten.fused_adamw(p, grads, m, v, [], [torch.tensor(1.0)] * len(shapes), **hp)
    for i in range(len(shapes)):
        assert_close(dp[i].cpu(), want[0][i], "fp32", f"param {i}")
        assert_close(dm[i].cpu(), want[2][i], "fp32", f"exp_avg {i}")
    assert float(dbase[0].cpu()) == float(base[0])  # the element before the view is untouched


def test_optim_adamw_fused_trains_on_gcu():
    """torch.optim.AdamW(fused=True) over a small model's gcu parameters runs
    the native kernel (no CPU fallback) and follows the same optimizer on CPU."""
    torch.manual_seed(0)
    model = torch.nn.Sequential(torch.nn.Linear(64, 128), torch.nn.SiLU(), torch.nn.Linear(128, 10))
    ref = [t.detach().clone() for t in model.parameters()]
    dparams = [torch.nn.Parameter(t.to("gcu")) for t in ref]
    cparams = [torch.nn.Parameter(t.clone()) for t in ref]
    dopt = torch.optim.AdamW(dparams, lr=1e-2, weight_decay=0.1, fused=True)
    copt = torch.optim.AdamW(cparams, lr=1e-2, weight_decay=0.1, fused=True)
    C._set_op_debug_config("op_statistics=true")
    C._clear_op_statistics()
    try:
        for it in range(4):
            grads = [torch.randn(t.shape, generator=g(500 + 10 * it + i)) for i, t in enumerate(ref)]
            for dp_, cp_, gr in zip(dparams, cparams, grads):
                dp_.grad = gr.to("gcu")
                cp_.grad = gr.clone()
            dopt.step()
            copt.step()
        torch.gcu.synchronize()
        stats = C._op_statistics()
    finally:
        C._set_op_debug_config("")
    for dp_, cp_ in zip(dparams, cparams):
        assert_close(dp_.detach().cpu(), cp_.detach(), "fp32", "AdamW(fused=True) params")
    assert stats.get("_fused_adamw_", (0, 0))[0] == 4, stats
    # the step-count advance is native too: nothing of the step falls back to CPU
    assert stats.get("_foreach_add_.Scalar", (0, 0))[0] == 4, stats
    assert all(v[1] == 0 for v in stats.values()), stats


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
def test_foreach_add_scalar_parity(dtype):
    """_foreach_add_.Scalar over 70 tensors (two launches) of several sizes,
    including an empty one and a misaligned view, equals CPU ATen's."""
    shapes = [(7,), (), (0,), (33, 65), (5000,)] * 14
    base = torch.randn(1 + 513, generator=g(600)).to(dtype)
    ts = [torch.randn(s, generator=g(601 + i)).to(dtype) for i, s in enumerate(shapes)] + [base[1:]]
    dbase = base.to("gcu")
    dts = [t.to("gcu") for t in ts[:-1]] + [dbase[1:]]
    torch._foreach_add_(dts, 0.3)
    want = aten.foreach_add_scalar(ts, 0.3)
    for a, b in zip(dts, want):
        assert_exact(a.cpu(), b, "foreach_add_")
    assert float(dbase[0].cpu()) == float(base[0])
    # an integer list takes the per-tensor path
    ints = [torch.arange(5).to("gcu"), torch.arange(3).to("gcu")]
    torch._foreach_add_(ints, 2)
    assert torch.equal(ints[0].cpu(), torch.arange(5) + 2) and torch.equal(ints[1].cpu(), torch.arange(3) + 2)



@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_amp_unscale_parity(dtype):
    """_amp_foreach_non_finite_check_and_unscale_ over 70 tensors: the grads
    are multiplied by inv_scale as CPU ATen does, found_inf stays 0 for finite
    grads, becomes 1 with an inf or a NaN anywhere, and inv_scale = 1 leaves
    the values as they are."""
    shapes = [(7,), (0,), (33, 65), (5000,), ()] * 14
    grads = [(torch.randn(s, generator=g(700 + i)) * 512).to(dtype) for i, s in enumerate(shapes)]
    for inv, poison in ((1.0 / 512, None), (1.0 / 512, float("inf")), (1.0, float("nan"))):
        cg = [t.clone() for t in grads]
        if poison is not None:
            cg[23].view(-1)[17] = poison
        dg = [t.to("gcu") for t in cg]
        fi, dfi = torch.zeros(1), torch.zeros(1, device="gcu")
        cg, fi = aten.amp_unscale(cg, fi, torch.tensor([inv]))
        torch._amp_foreach_non_finite_check_and_unscale_(dg, dfi, torch.tensor([inv], device="gcu"))
        assert float(dfi.cpu()) == float(fi) == (0.0 if poison is None else 1.0)
        for a, b in zip(dg, cg):
            assert_exact(a.cpu(), b, f"unscale {inv}")


def test_amp_update_scale_parity():
    """_amp_update_scale_ follows CPU ATen's over a sequence of clean and
    overflowing steps: growth after growth_interval clean steps, back-off and
    a restarted count on inf, and a growth that would overflow fp32 is not
    taken."""
    for start in (65536.0, 3.0e38):
        cs, ct = torch.tensor([start]), torch.tensor([0], dtype=torch.int32)
        ds, dt = cs.to("gcu"), ct.to("gcu")
        for k, bad in enumerate([0, 0, 0, 1, 0, 0, 0, 0, 1, 1, 0, 0, 0]):
            cf = torch.tensor([float(bad)])
            cs, ct = aten.amp_update_scale(cs, ct, cf, 2.0, 0.5, 3)
            torch._amp_update_scale_(ds, dt, cf.to("gcu"), 2.0, 0.5, 3)
            assert float(ds.cpu()) == float(cs) and int(dt.cpu()) == int(ct), (start, k)


def test_grad_scaler_with_fused_adamw_on_gcu():
    """torch.amp.GradScaler over AdamW(fused=True): the unscale check, the
    fused step with grad_scale / found_inf and the scale update all run
    natively, an overflowing step is skipped, and the parameters and scale
    follow the same loop on CPU."""
    torch.manual_seed(0)
    ref = [torch.randn(64, 32) * 0.1, torch.randn(64) * 0.1]
    res = {}
    C._set_op_debug_config("op_statistics=true")
    C._clear_op_statistics()
    try:
        for dev in ("gcu", "cpu"):
            ps = [torch.nn.Parameter(t.clone().to(dev)) for t in ref]
            opt = torch.optim.AdamW(ps, lr=1e-2, fused=True)
            scaler = torch.amp.GradScaler(dev, init_scale=1024.0, growth_interval=2)
            for it in range(5):
                x = torch.randn(16, 32, generator=g(800 + it)).to(dev)
                loss = torch.nn.functional.linear(x, ps[0], ps[1]).pow(2).mean()
                if it == 2:
                    loss = loss * float("inf")
                opt.zero_grad()
                scaler.scale(loss).backward()
                scaler.step(opt)
                scaler.update()
            res[dev] = ([p.detach().cpu() for p in ps], float(scaler.get_scale()))
            if dev == "gcu":
                torch.gcu.synchronize()
                stats = C._op_statistics()
    finally:
        C._set_op_debug_config("")
    for a, b in zip(res["gcu"][0], res["cpu"][0]):
        assert_close(a, b, "fp32", "GradScaler + AdamW(fused=True) params")
    assert res["gcu"][1] == res["cpu"][1]
    for op in ("_amp_foreach_non_finite_check_and_unscale_", "_amp_update_scale_", "_fused_adamw_"):
        assert stats.get(op, (0, 0))[0] >= 4 and stats[op][1] == 0, (op, stats.get(op))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
def test_foreach_mul_parity(dtype):
    """_foreach_mul_ by a Python scalar, by a 0-dim fp32 scalar on the device
    (read by the kernel, as gradient clipping passes it) and by a CPU scalar
    tensor, over 70 tensors with an empty one and a misaligned view, equals
    CPU ATen's; an integer list takes the per-tensor path."""
    shapes = [(7,), (), (0,), (33, 65), (5000,)] * 14
    for k, other in enumerate((0.37, torch.tensor(0.37), torch.tensor(-1.75))):
        base = torch.randn(1 + 513, generator=g(900 + k)).to(dtype)
        ts = [torch.randn(s, generator=g(910 + k * 100 + i)).to(dtype) for i, s in enumerate(shapes)]
        ts.append(base[1:])
        dbase = base.to("gcu")
        dts = [t.to("gcu") for t in ts[:-1]] + [dbase[1:]]
        want = aten.foreach_mul(ts, other)
        dother = other.to("gcu") if (isinstance(other, torch.Tensor) and k == 1) else other
        torch._foreach_mul_(dts, dother)
        for a, b in zip(dts, want):
            assert_exact(a.cpu(), b, f"foreach_mul_ {k}")
        assert float(dbase[0].cpu()) == float(base[0])
    ints = [torch.arange(5).to("gcu")]
    torch._foreach_mul_(ints, 3)
    assert torch.equal(ints[0].cpu(), torch.arange(5) * 3)


def test_clip_grad_norm_foreach_on_gcu():
    """torch.nn.utils.clip_grad_norm_(foreach=True) scales gcu gradients with
    the native _foreach_mul_.Tensor and matches the CPU result."""
    grads = [torch.randn(s, generator=g(990 + i)) * 3 for i, s in enumerate([(64, 32), (64,), (7, 5)])]
    cps = [torch.nn.Parameter(torch.zeros(gr.shape)) for gr in grads]
    dps = [torch.nn.Parameter(torch.zeros(gr.shape, device="gcu")) for gr in grads]
    for c, d, gr in zip(cps, dps, grads):
        c.grad, d.grad = gr.clone(), gr.to("gcu")
    C._set_op_debug_config("op_statistics=true")
    C._clear_op_statistics()
    try:
        dn = torch.nn.utils.clip_grad_norm_(dps, 1.0, foreach=True)
        torch.gcu.synchronize()
        stats = C._op_statistics()
    finally:
        C._set_op_debug_config("")
    cn = torch.nn.utils.clip_grad_norm_(cps, 1.0, foreach=True)
    assert_close(dn.cpu(), cn, "fp32", "total norm")
    for c, d in zip(cps, dps):
        assert_close(d.grad.cpu(), c.grad, "fp32", "clipped grad")
    st = stats.get("_foreach_mul_.Tensor", (0, 0))
    assert st[0] == 1 and st[1] == 0, stats
