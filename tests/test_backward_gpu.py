"""The training-side backward ops on the gcu device (silu_backward,
_log_softmax_backward_data / _softmax_backward_data, native_layer_norm_backward)
against CPU ATen on the same inputs, and end to end through autograd.
fp32 results within the fp32 bar, bf16 / fp16 results within the bf16 bar."""
import pytest
import torch
import torch.nn.functional as F

import torch_gcu
from oracle import aten
from oracle import numpy_ref as npr
from oracle.tolerance import assert_close

pytestmark = pytest.mark.gpu

C = torch_gcu._C


def g(seed):
    return torch.Generator().manual_seed(seed)


def rn(shape, dtype, seed, scale=1.0):
    return (torch.randn(shape, generator=g(seed)) * scale).to(dtype)


def bar(dtype):
    return "fp32" if dtype == torch.float32 else "bf16"


@pytest.fixture(autouse=True)
def _clean():
    C._set_op_debug_config("")
    yield
    C._set_op_debug_config("")
    torch.gcu.synchronize()


# ---- silu_backward ----------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(2048, 11008), (3, 7), (1, 1001)])
def test_silu_backward_parity(dtype, shape):
    dy, x = rn(shape, dtype, 1), rn(shape, dtype, 2, 3.0)
    got = torch.ops.aten.silu_backward(dy.to("gcu"), x.to("gcu"))
    assert got.dtype == dtype and got.shape == x.shape
    assert_close(got.cpu(), aten.silu_backward(dy, x), bar(dtype), f"silu_backward {shape}")


def test_silu_backward_layouts_promotion_and_out():
    x = rn((64, 96), torch.float32, 3, 3.0)
    dy = rn((64, 96), torch.float32, 4)
    dyt = rn((96, 64), torch.float32, 5).to("gcu").t()  # strided grad
    got = torch.ops.aten.silu_backward(dyt, x.to("gcu"))
    assert_close(got.cpu(), aten.silu_backward(dyt.cpu(), x), "fp32", "silu_backward transposed grad")
    # broadcast grad row, bf16 input promoted with a float grad
    row = rn((96,), torch.float32, 6)
    xb = x.bfloat16()
    got = torch.ops.aten.silu_backward(row.to("gcu"), xb.to("gcu"))
    want = aten.silu_backward(row, xb)
    assert got.dtype == want.dtype == torch.float32
    assert_close(got.cpu(), want, "fp32", "silu_backward broadcast + promotion")
    out = torch.empty(0, dtype=torch.float32, device="gcu")
    torch.ops.aten.silu_backward.grad_input(dy.contiguous().to("gcu"), x.to("gcu"), grad_input=out)
    assert_close(out.cpu(), aten.silu_backward(dy, x), "fp32", "silu_backward out=")


# ---- softmax family -----------------------------------------------------------------------

_SM_CASES = [
    ((8192, 32000), -1, torch.bfloat16, torch.bfloat16),   # config 2's shape, register rows
    ((64, 1000), -1, torch.float32, torch.float32),
    ((33, 65), 0, torch.float32, torch.float32),            # non-last dim: one lane per column
    ((7, 33), 1, torch.bfloat16, torch.bfloat16),           # unaligned rows: two-read row kernel
    ((16, 4096), -1, torch.float32, torch.float16),          # half_to_float: grads float, out half
    ((2, 3, 40), 1, torch.float16, torch.float16),
]


@pytest.mark.parametrize("shape,dim,dt,input_dtype", _SM_CASES)
@pytest.mark.parametrize("log", [True, False])
def test_softmax_backward_parity(shape, dim, dt, input_dtype, log):
    x = rn(shape, torch.float32, 10, 2.0)
    y = (torch.log_softmax(x, dim) if log else torch.softmax(x, dim)).to(dt)
    dy = rn(shape, dt, 11)
    # CPU ATen has no half_to_float backward (float grads into a half result):
    # its float result rounded once to half is the reference there
    h2f = dt == torch.float32 and input_dtype == torch.float16
    cpu_dtype = torch.float32 if h2f else input_dtype
    if log:
        got = torch.ops.aten._log_softmax_backward_data(dy.to("gcu"), y.to("gcu"), dim, input_dtype)
        want = aten.log_softmax_backward(dy, y, dim, cpu_dtype)
    else:
        got = torch.ops.aten._softmax_backward_data(dy.to("gcu"), y.to("gcu"), dim, input_dtype)
        want = aten.softmax_backward(dy, y, dim, cpu_dtype)
    if h2f:
        want = want.half()
    assert got.dtype == want.dtype, (got.dtype, want.dtype)
    assert_close(got.cpu(), want, bar(want.dtype if want.dtype != torch.float16 else torch.bfloat16),
                 f"{'log_' if log else ''}softmax_backward {shape} dim {dim}")


def test_softmax_backward_out_and_strided_operands():
    x = rn((40, 100), torch.float32, 12)
    y = torch.log_softmax(x, -1)
    dy = rn((100, 40), torch.float32, 13).t()
    out = torch.empty(0, device="gcu")
    torch.ops.aten._log_softmax_backward_data.out(dy.to("gcu"), y.to("gcu"), -1, torch.float32, out=out)
    assert_close(out.cpu(), aten.log_softmax_backward(dy, y, -1, torch.float32), "fp32", "out=")
    dyt = rn((100, 40), torch.float32, 14).to("gcu").t()
    got = torch.ops.aten._log_softmax_backward_data(dyt, y.to("gcu"), -1, torch.float32)
    assert_close(got.cpu(), aten.log_softmax_backward(dyt.cpu(), y, -1, torch.float32), "fp32",
                 "strided grad")


# ---- native_layer_norm_backward -----------------------------------------------------------

_LN_CASES = [
    ((16384, 4096), torch.bfloat16, torch.bfloat16),   # fused path, bf16 mean / rstd
    ((512, 1000), torch.float32, torch.float32),        # fused, 250 vectors per row
    ((64, 12288), torch.bfloat16, torch.float32),       # fused, 3 vectors per lane, fp32 weight
    ((8, 20000), torch.bfloat16, torch.bfloat16),       # rows too long for the fused path
    ((3, 5, 7), torch.float32, torch.float32),          # odd rows: row and column kernels
    ((4500, 256), torch.float16, torch.float16),        # more blocks than partial rows
]


@pytest.mark.parametrize("shape,dt,wdt", _LN_CASES)
@pytest.mark.parametrize("affine", [True, False])
def test_layer_norm_backward_parity(shape, dt, wdt, affine):
    n = shape[-1]
    x = rn(shape, dt, 20, 2.0) + 0.5
    w = rn((n,), wdt, 21) if affine else None
    b = rn((n,), wdt, 22) if affine else None
    _, mean, rstd = aten.layer_norm_forward(x, [n], w, b, 1e-5)
    dy = rn(shape, dt, 23)
    mask = [True, affine, affine]
    want = aten.layer_norm_backward(dy, x, [n], mean, rstd, w, b, mask)
    dev = lambda t: None if t is None else t.to("gcu")  # noqa: E731
    got = torch.ops.aten.native_layer_norm_backward(dev(dy), dev(x), [n], dev(mean), dev(rstd),
                                                    dev(w), dev(b), mask)
    assert_close(got[0].cpu(), want[0], bar(dt), f"dx {shape}")
    if affine:
        if dt == torch.float32:
            assert_close(got[1].cpu(), want[1], "fp32", f"dgamma {shape}")
            assert_close(got[2].cpu(), want[2], "fp32", f"dbeta {shape}")
        else:
            # CPU ATen adds 16-bit dgamma / dbeta columns in 16-bit arithmetic
            # (about 5 % off at 16384 rows); the float64 closed form on the same
            # inputs, rounded once to the output dtype, is the reference
            _, rdw, rdb = npr.layer_norm_backward64(dy.float().numpy(), x.float().numpy(),
                                                    mean.double().numpy(), rstd.double().numpy(),
                                                    w.float().numpy())
            assert_close(got[1].cpu(), torch.from_numpy(rdw).to(wdt), "bf16", f"dgamma {shape}")
            assert_close(got[2].cpu(), torch.from_numpy(rdb).to(wdt), "bf16", f"dbeta {shape}")


_LNF_CASES = [
    ((16384, 4096), [4096], torch.bfloat16, torch.bfloat16),  # register rows, bf16 statistics
    ((512, 1000), [1000], torch.float32, torch.float32),
    ((64, 12288), [12288], torch.bfloat16, torch.float32),   # fp32 parameters: fp32 statistics
    ((8, 20000), [20000], torch.bfloat16, torch.bfloat16),   # rows read three times
    ((6, 5, 7), [5, 7], torch.float32, None),                 # two normalized dims, no affine
]


@pytest.mark.parametrize("shape,nshape,dt,wdt", _LNF_CASES)
def test_layer_norm_forward_parity(shape, nshape, dt, wdt):
    n = 1
    for d in nshape:
        n *= d
    x = rn(shape, dt, 50, 2.0) + 0.3
    w = rn(nshape, wdt, 51) if wdt is not None else None
    b = rn(nshape, wdt, 52) if wdt is not None else None
    want = aten.layer_norm_forward(x, nshape, w, b, 1e-5)
    dev = lambda t: None if t is None else t.to("gcu")  # noqa: E731
    got = torch.native_layer_norm(dev(x), nshape, dev(w), dev(b), 1e-5)
    for i, name in enumerate(("out", "mean", "rstd")):
        assert got[i].shape == want[i].shape and got[i].dtype == want[i].dtype, (name, got[i].dtype)
        assert_close(got[i].cpu(), want[i], bar(want[i].dtype if want[i].dtype != torch.float16
                                                else torch.bfloat16), f"{name} {shape}")


def test_layer_norm_backward_masks_and_no_rows():
    x = rn((256, 512), torch.float32, 30)
    w, b = rn((512,), torch.float32, 31), rn((512,), torch.float32, 32)
    _, mean, rstd = aten.layer_norm_forward(x, [512], w, b, 1e-5)
    dy = rn((256, 512), torch.float32, 33)
    for mask in ([False, True, True], [True, False, False], [False, False, True]):
        want = aten.layer_norm_backward(dy, x, [512], mean, rstd, w, b, mask)
        got = torch.ops.aten.native_layer_norm_backward(dy.to("gcu"), x.to("gcu"), [512], mean.to("gcu"),
                                                        rstd.to("gcu"), w.to("gcu"), b.to("gcu"), mask)
        for i in range(3):
            if mask[i]:
                assert_close(got[i].cpu(), want[i], "fp32", f"mask {mask} output {i}")
            else:
                assert got[i] is None and want[i] is None
    # no rows: dgamma and dbeta are zeros
    e = torch.empty(0, 512, device="gcu")
    got = torch.ops.aten.native_layer_norm_backward(e, e, [512], torch.empty(0, 1, device="gcu"),
                                                    torch.empty(0, 1, device="gcu"), w.to("gcu"),
                                                    b.to("gcu"), [True, True, True])
    assert got[0].shape == (0, 512)
    assert float(got[1].abs().sum()) == 0.0 and float(got[2].abs().sum()) == 0.0


@pytest.mark.parametrize("rows", [64, 61])
def test_layer_norm_backward_16bit_statistics(rows):
    """mean / rstd in the input's 16-bit dtype (what a bf16 forward on gcu
    stores), through the fused kernel, with a last block of fewer rows than
    a step when rows is odd; CPU ATen given the same statistics (its bf16
    forward stores them in bf16 too)."""
    n = 1024
    x = rn((rows, n), torch.bfloat16, 34, 2.0) + 0.5
    w, b = rn((n,), torch.bfloat16, 35), rn((n,), torch.bfloat16, 36)
    _, mean, rstd = aten.layer_norm_forward(x, [n], w, b, 1e-5)
    mean, rstd = mean.bfloat16(), rstd.bfloat16()
    dy = rn((rows, n), torch.bfloat16, 37)
    want = aten.layer_norm_backward(dy, x, [n], mean, rstd, w, b, [True, False, False])
    got = torch.ops.aten.native_layer_norm_backward(dy.to("gcu"), x.to("gcu"), [n], mean.to("gcu"),
                                                    rstd.to("gcu"), w.to("gcu"), b.to("gcu"),
                                                    [True, True, True])
    assert_close(got[0].cpu(), want[0], "bf16", f"dx, bf16 statistics, {rows} rows")
    _, rdw, rdb = npr.layer_norm_backward64(dy.float().numpy(), x.float().numpy(),
                                            mean.double().numpy(), rstd.double().numpy(),
                                            w.float().numpy())
    assert_close(got[1].cpu(), torch.from_numpy(rdw).bfloat16(), "bf16", "dgamma, bf16 statistics")
    assert_close(got[2].cpu(), torch.from_numpy(rdb).bfloat16(), "bf16", "dbeta, bf16 statistics")


# ---- autograd end to end ---------------------------------------------------------------------

def test_autograd_layer_norm_silu_log_softmax_on_gcu():
    """A small network's backward on gcu tensors reaches the native backward
    kernels (no CPU fallback for them) and matches the same backward on CPU."""
    torch.manual_seed(0)
    H, V = 256, 1000
    xc = torch.randn(128, H, generator=g(40))
    wc, bc = torch.randn(H, generator=g(41)), torch.randn(H, generator=g(42))
    pc = torch.randn(H, V, generator=g(43)) * 0.05
    tgt = torch.randint(0, V, (128,), generator=g(44))

    def run(dev):
        x = xc.to(dev).requires_grad_()
        w, b = wc.to(dev).requires_grad_(), bc.to(dev).requires_grad_()
        h = F.silu(F.layer_norm(x, [H], w, b, 1e-5))
        logp = torch.log_softmax(h @ pc.to(dev), -1)
        loss = -logp[torch.arange(128, device=dev), tgt.to(dev)].sum()
        loss.backward()
        return x.grad, w.grad, b.grad

    C._set_op_debug_config("op_statistics=true")
    C._clear_op_statistics()
    try:
        gx, gw, gb = run("gcu")
        torch.gcu.synchronize()
        stats = C._op_statistics()
    finally:
        C._set_op_debug_config("")
    rx, rw, rb = run("cpu")
    assert_close(gx.cpu(), rx, "fp32", "dx")
    assert_close(gw.cpu(), rw, "fp32", "dgamma")
    assert_close(gb.cpu(), rb, "fp32", "dbeta")
    for op in ("native_layer_norm", "native_layer_norm_backward", "silu_backward",
               "_log_softmax_backward_data"):
        assert stats.get(op, (0, 0))[0] >= 1 and stats.get(op, (0, 0))[1] == 0, (op, stats)
