"""GPU parity of the gfx950 kernels, called through the C ABI.

Every case runs the same seeded CPU inputs through CPU ATen (the reference's
own fallback path, via ``oracle.aten``) and through the kernel library, then
compares: bit-exact for integer/index/amax and single-rounding elementwise
ops, fp32 rel 1e-5 (+1e-5*max|ref|) for fp32 reductions, bf16 rel 1e-2
(+1e-2*rms(ref)) for bf16 outputs with fp32 accumulation.
"""
import math

import pytest
import torch

from oracle import aten
from oracle.tolerance import assert_close, assert_exact
from torch_gcu import _abi
from torch_gcu.utils import synthetic

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _setup():
    torch.cuda.init()
    _abi.install_workspace()
    yield
    torch.cuda.synchronize()


def g(seed):
    return torch.Generator().manual_seed(seed)


def dev(t):
    return t.to(DEV)


def empty_like_ref(ref):
    return torch.empty(ref.shape, dtype=ref.dtype, device=DEV)


def rand(shape, dtype, seed):
    if dtype.is_floating_point:
        return torch.randn(shape, generator=g(seed)).to(dtype)
    if dtype == torch.bool:
        return torch.randint(0, 2, shape, generator=g(seed)).bool()
    lo, hi = (-1000, 1000) if dtype != torch.uint8 else (0, 255)
    return torch.randint(lo, hi, shape, generator=g(seed)).to(dtype)


# ---- elementwise -------------------------------------------------------------------

def test_config1_mul_add_full_size_bit_exact():
    c = synthetic.config1()
    a, b = dev(c["a"]), dev(c["b"])
    t = torch.empty_like(a)
    out = torch.empty_like(a)
    _abi.mul(t, a, b)
    _abi.add(out, t, c["c"])
    ref = aten.add(aten.mul(c["a"], c["b"]), c["c"])
    assert_exact(out, ref, "a*b+0.5")


BIN_DTYPES = [torch.float32, torch.bfloat16, torch.float16, torch.float64, torch.int32,
              torch.int64]


@pytest.mark.parametrize("dtype", BIN_DTYPES)
@pytest.mark.parametrize("layout", ["full", "row", "col", "scalar0d", "transposed", "odd"])
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
def test_binary_parity(dtype, layout, op):
    if op == "div" and not dtype.is_floating_point:
        pass  # true division promotes to float32
    shape = (67, 130) if layout != "odd" else (13, 7, 5)
    a = rand(shape, dtype, 1)
    if layout == "full" or layout == "odd":
        b = rand(shape, dtype, 2)
    elif layout == "row":
        b = rand(shape[-1:], dtype, 2)
    elif layout == "col":
        b = rand((shape[0], 1), dtype, 2)
    elif layout == "scalar0d":
        b = rand((), dtype, 2)
    else:
        b = rand(shape[::-1], dtype, 2).t()
    if op == "div" and not dtype.is_floating_point:
        b = torch.where(b == 0, torch.ones_like(b), b)
    ref = getattr(aten, op)(a, b)
    out = empty_like_ref(ref)
    getattr(_abi, op)(out, dev(a), dev(b))
    assert_exact(out, ref, f"{op} {dtype} {layout}")


# The typed 2-D path (dense rows of whole 16-byte vectors): a lane finds the
# row and column of its vectors by one division and then steps when a row
# holds at least 256 vectors, else divides each; ragged last blocks.
@pytest.mark.parametrize("shape,dtype", [
    ((33, 2048), torch.float32),    # 512 vectors a row: stepped
    ((1031, 2048), torch.float32),  # stepped, last block ragged
    ((7, 8192), torch.bfloat16),    # 1024 vectors a row, fewer vectors than one block
    ((5, 1000), torch.float32),     # 250 vectors a row: divided
    ((300, 1024), torch.bfloat16),  # 128 vectors a row: divided
    ((1, 4096), torch.float32),     # one row
])
@pytest.mark.parametrize("layout", ["row", "col", "full", "scalar"])
@pytest.mark.parametrize("op", ["add", "mul"])
def test_binary_2d_path_parity(shape, dtype, layout, op):
    a = rand(shape, dtype, 11)
    if layout == "row":
        b = rand(shape[-1:], dtype, 12)
    elif layout == "col":
        b = rand((shape[0], 1), dtype, 12)
    elif layout == "full":
        b = rand(shape, dtype, 12)
    else:
        b = 0.5
    ref = getattr(aten, op)(a, b)
    out = empty_like_ref(ref)
    getattr(_abi, op)(out, dev(a), b if layout == "scalar" else dev(b))
    assert_exact(out, ref, f"{op} {shape} {dtype} {layout}")
    # the operand order swapped: the broadcast one first
    if layout in ("row", "col"):
        ref2 = getattr(aten, op)(b, a)
        out2 = empty_like_ref(ref2)
        getattr(_abi, op)(out2, dev(b), dev(a))
        assert_exact(out2, ref2, f"{op} {shape} {dtype} {layout} swapped")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.int64,
                                   torch.int32, torch.uint8])
@pytest.mark.parametrize("value", [0.5, 0.1, 3, -2])
def test_scalar_operand_parity(dtype, value):
    a = rand((129, 33), dtype, 3)
    ref_add = aten.add(a, value)
    out = empty_like_ref(ref_add)
    _abi.add(out, dev(a), value)
    assert_exact(out, ref_add, f"add {dtype} {value}")
    ref_mul = aten.mul(a, value)
    out = empty_like_ref(ref_mul)
    _abi.mul(out, dev(a), value)
    assert_exact(out, ref_mul, f"mul {dtype} {value}")


def test_mixed_dtype_promotion():
    a = rand((40, 50), torch.bfloat16, 4)
    b = rand((40, 50), torch.float32, 5)
    s32 = rand((), torch.float32, 6) * 0.3
    cases = [(a, b), (b, a), (a, s32), (s32, a), (rand((40, 50), torch.int32, 7), rand((), torch.float64, 8))]
    for op in ["mul", "add", "div"]:
        for x, y in cases:
            ref = getattr(aten, op)(x, y)
            out = empty_like_ref(ref)
            getattr(_abi, op)(out, dev(x), dev(y))
            assert_exact(out, ref, f"{op} {x.dtype}[{x.dim()}]x{y.dtype}[{y.dim()}]")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.int32])
@pytest.mark.parametrize("value", [0.1, 0.3, 7.0, 3])
def test_div_by_scalar(dtype, value):
    a = rand((70, 30), dtype, 35)
    ref = aten.div(a, value)
    out = empty_like_ref(ref)
    _abi.div(out, dev(a), value)
    assert_exact(out, ref, f"div {dtype} {value}")


def test_add_alpha():
    a = rand((1000,), torch.float32, 9)
    b = rand((1000,), torch.float32, 10)
    ref = aten.add(a, b, alpha=2)
    out = empty_like_ref(ref)
    _abi.add(out, dev(a), dev(b), alpha=2)
    assert_exact(out, ref, "alpha=2")
    ref = aten.sub(a, b, alpha=0.3)
    out = empty_like_ref(ref)
    _abi.sub(out, dev(a), dev(b), alpha=0.3)
    assert_close(out, ref, "fp32", "alpha=0.3")


def test_empty_and_single_element():
    for shape in [(0,), (0, 5), (1,), ()]:
        a = rand(shape, torch.float32, 11)
        ref = aten.add(a, a)
        out = empty_like_ref(ref)
        _abi.add(out, dev(a), dev(a))
        assert_exact(out, ref, f"add {shape}")


@pytest.mark.parametrize("src,dst", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32),
                                     (torch.float32, torch.float16), (torch.int64, torch.float32),
                                     (torch.float64, torch.float16), (torch.float32, torch.int32),
                                     (torch.float32, torch.uint8), (torch.int32, torch.bool),
                                     (torch.float64, torch.float64), (torch.bfloat16, torch.bfloat16)])
def test_copy_conversions(src, dst):
    x = rand((33, 65), src, 12) * (3 if src.is_floating_point else 1)
    for view in [x, x.t(), x[:, ::2]]:
        ref = view.to(dst)
        out = torch.empty(ref.shape, dtype=dst, device=DEV)
        _abi.copy_(out, _strided_on_device(view))
        assert_exact(out, ref, f"copy {src}->{dst}")


def _strided_on_device(view):
    """Device tensor with the same (possibly non-contiguous) view."""
    base = view
    while base._base is not None:
        base = base._base
    d = dev(base)
    return d.as_strided(view.shape, view.stride(), view.storage_offset())


def test_copy_broadcast_and_fill():
    src = rand((1, 17), torch.float32, 13)
    out = torch.empty(9, 17, device=DEV)
    _abi.copy_(out, dev(src))
    assert_exact(out, src.expand(9, 17).contiguous(), "broadcast copy")
    for dtype, v in [(torch.float32, 1.5), (torch.bfloat16, 0.1), (torch.int64, -7), (torch.bool, 1),
                     (torch.float16, 65504.0), (torch.uint8, 255)]:
        o = torch.empty(1001, dtype=dtype, device=DEV)
        _abi.fill_(o, v)
        assert_exact(o, torch.full((1001,), v, dtype=dtype), f"fill {dtype}")
    o = torch.zeros(10, 10, device=DEV)
    _abi.fill_(o[:, 3], 2.0)
    ref = torch.zeros(10, 10)
    ref[:, 3] = 2.0
    assert_exact(o, ref, "strided fill")


# ---- index_select -----------------------------------------------------------------

def test_config1_index_select_full_size_bit_exact():
    c = synthetic.config1()
    ref = aten.index_select(c["table"], 0, c["idx"])
    out = empty_like_ref(ref)
    _abi.index_select(out, dev(c["table"]), 0, dev(c["idx"]))
    assert_exact(out, ref, "index_select int64")


@pytest.mark.parametrize("dtype", [torch.int64, torch.bfloat16, torch.float32, torch.uint8])
@pytest.mark.parametrize("dim", [0, 1, 2])
@pytest.mark.parametrize("idx_dtype", [torch.int64, torch.int32])
def test_index_select_parity(dtype, dim, idx_dtype):
    x = rand((11, 6, 9), dtype, 14)
    idx = torch.randint(0, x.shape[dim], (13,), generator=g(15)).to(idx_dtype)
    ref = aten.index_select(x, dim, idx)
    out = empty_like_ref(ref)
    _abi.index_select(out, dev(x), dim, dev(idx))
    assert_exact(out, ref, f"index_select {dtype} dim{dim}")
    # non-contiguous self
    xt = x.transpose(0, 2)
    ref = aten.index_select(xt, dim, idx.clamp(max=xt.shape[dim] - 1))
    out = empty_like_ref(ref)
    _abi.index_select(out, _strided_on_device(xt), dim, dev(idx.clamp(max=xt.shape[dim] - 1)))
    assert_exact(out, ref, "index_select transposed")


def test_index_select_embedding_rows_and_edges():
    emb = rand((320, 4096), torch.bfloat16, 16)
    ids = torch.randint(0, 320, (1000,), generator=g(17))
    ref = aten.index_select(emb, 0, ids)
    out = empty_like_ref(ref)
    _abi.index_select(out, dev(emb), 0, dev(ids))
    assert_exact(out, ref, "embedding")
    # empty index
    e = torch.empty(0, dtype=torch.int64)
    ref = aten.index_select(emb, 0, e)
    out = empty_like_ref(ref)
    _abi.index_select(out, dev(emb), 0, dev(e))
    assert out.shape == (0, 4096)
    # out-of-range rows are written as zeros, never read, and recorded for
    # mi_index_fault_take (one of the bad indices, with the dim size)
    assert _abi.index_fault_take(0) is None
    bad = torch.tensor([0, 320, -1, 5])
    out = torch.full((4, 4096), 7.0, dtype=torch.bfloat16, device=DEV)
    _abi.index_select(out, dev(emb), 0, dev(bad))
    o = out.cpu()
    assert torch.equal(o[0], emb[0]) and torch.equal(o[3], emb[5])
    assert (o[1] == 0).all() and (o[2] == 0).all()
    fault = _abi.index_fault_take(0)
    assert fault is not None and fault[0] in (320, -1) and fault[1] == emb.shape[0], fault
    assert _abi.index_fault_take(0) is None  # the record was cleared


# ---- reductions -------------------------------------------------------------------

def test_config2_sum_amax_log_softmax_reduced_rows():
    c = synthetic.config2(rows=512, mrows=2048)
    x = dev(c["logits"])
    ref = aten.sum_(c["logits"], -1)
    out = empty_like_ref(ref)
    _abi.sum_(out, x, [-1])
    assert_close(out, ref, "bf16", "sum")
    ref = aten.amax(c["logits"], -1)
    out = empty_like_ref(ref)
    _abi.amax(out, x, [-1])
    assert_exact(out, ref, "amax")
    ref = aten.log_softmax(c["logits"], -1)
    out = empty_like_ref(ref)
    _abi.log_softmax(out, x, -1)
    assert_close(out, ref, "bf16", "log_softmax")
    ref = aten.mean(c["m"], 0)
    out = empty_like_ref(ref)
    _abi.mean(out, dev(c["m"]), [0])
    assert_close(out, ref, "fp32", "mean0")


def test_config2_full_size():
    c = synthetic.config2()
    x = dev(c["logits"])
    out = torch.empty(8192, dtype=torch.bfloat16, device=DEV)
    _abi.amax(out, x, [-1])
    assert_exact(out, aten.amax(c["logits"], -1), "amax full")
    _abi.sum_(out, x, [-1])
    assert_close(out, aten.sum_(c["logits"], -1), "bf16", "sum full")
    ls = torch.empty_like(x)
    _abi.log_softmax(ls, x, -1)
    assert_close(ls, aten.log_softmax(c["logits"], -1), "bf16", "log_softmax full")
    # size-independent property: every row's log-sum-exp is 0 (bf16 output)
    lse = torch.logsumexp(ls.float(), -1)
    assert lse.abs().max().item() < 0.05
    m = torch.empty(4096, device=DEV)
    _abi.mean(m, dev(c["m"]), [0])
    assert_close(m, aten.mean(c["m"], 0), "fp32", "mean0 full")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64, torch.int32, torch.int64])
@pytest.mark.parametrize("dims,keepdim", [((-1,), False), ((0,), True), ((1,), False), ((0, 2), False),
                                          ((), False), ((1, 2), True)])
def test_reduce_parity(dtype, dims, keepdim):
    x = rand((37, 19, 45), dtype, 18)
    ref = aten.sum_(x, list(dims) if dims else None, keepdim) if dims else torch.sum(x)
    out = empty_like_ref(ref)
    _abi.sum_(out, dev(x), dims, keepdim)
    if dtype.is_floating_point:
        assert_close(out, ref, "bf16" if dtype == torch.bfloat16 else "fp32", f"sum {dims}")
    else:
        assert_exact(out, ref, f"sum {dims}")
    ref = aten.amax(x, dims, keepdim)
    out = empty_like_ref(ref)
    _abi.amax(out, dev(x), dims, keepdim)
    assert_exact(out, ref, f"amax {dims}")
    if dtype.is_floating_point:
        ref = aten.mean(x, list(dims), keepdim) if dims else torch.mean(x)
        out = empty_like_ref(ref)
        _abi.mean(out, dev(x), dims, keepdim)
        assert_close(out, ref, "bf16" if dtype == torch.bfloat16 else "fp32", f"mean {dims}")


def test_reduce_long_rows_and_noncontiguous():
    x = rand((3, 1 << 20), torch.float32, 19)
    ref = aten.sum_(x, -1)
    out = empty_like_ref(ref)
    _abi.sum_(out, dev(x), [-1])
    assert_close(out, ref, "fp32", "long rows")
    ref = torch.sum(x)
    out = empty_like_ref(ref)
    _abi.sum_(out, dev(x), [])
    assert_close(out, ref, "fp32", "reduce all")
    xt = rand((64, 48), torch.float32, 20).t()
    ref = aten.amax(xt, 1)
    out = empty_like_ref(ref)
    _abi.amax(out, _strided_on_device(xt), [1])
    assert_exact(out, ref, "transposed amax")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64, torch.int64,
                                   torch.int32, torch.uint8])
@pytest.mark.parametrize("shape,dims", [((3000, 257), (0,)), ((2, 1500, 1024), (1,)),
                                        ((1024, 4099), (0,)), ((700, 8, 3), (0,)),
                                        ((2, 600, 4096), (1,)), ((600, 2052), (0,))])
def test_column_reduce_split_pass(dtype, shape, dims):
    """Column reductions long enough to be split over blocks and finished by
    the second pass over partials, with aligned (vector) and odd widths; the
    last two shapes take 1024-lane column blocks (two outer slices; a row of
    513 column vectors, half a block idle) and, in fp32 accumulation, the
    float4 finish over several outer slices and a ragged last block."""
    x = rand(shape, dtype, 29)
    ref = aten.sum_(x, list(dims))
    out = empty_like_ref(ref)
    _abi.sum_(out, dev(x), dims)
    if dtype.is_floating_point:
        assert_close(out, ref, "bf16" if dtype == torch.bfloat16 else "fp32", "split sum")
    else:
        assert_exact(out, ref, "split sum")
    if dtype.is_floating_point:
        x.view(-1)[777] = float("nan")
    ref = aten.amax(x, list(dims))
    out = empty_like_ref(ref)
    _abi.amax(out, dev(x), dims)
    assert_exact(out, ref, "split amax")
    if dtype.is_floating_point:
        x = rand(shape, dtype, 30)
        ref = aten.mean(x, list(dims))
        out = empty_like_ref(ref)
        _abi.mean(out, dev(x), dims)
        assert_close(out, ref, "bf16" if dtype == torch.bfloat16 else "fp32", "split mean")


def test_amax_nan_and_empty_sum():
    x = torch.randn(4, 100)
    x[2, 17] = float("nan")
    out = torch.empty(4, device=DEV)
    _abi.amax(out, dev(x), [1])
    assert_exact(out, aten.amax(x, 1), "nan amax")
    e = torch.empty(5, 0)
    out = torch.empty(5, device=DEV)
    _abi.sum_(out, dev(e), [1])
    assert_exact(out, torch.zeros(5), "empty sum")


# ---- softmax ----------------------------------------------------------------------

@pytest.mark.parametrize("log", [True, False])
@pytest.mark.parametrize("case", ["bf16", "f32", "bf16_to_f32", "long_f32", "odd", "dim0"])
def test_softmax_parity(log, case):
    if case == "bf16":
        x, dim, h2f = rand((33, 32000), torch.bfloat16, 21) * 4, -1, False
    elif case == "f32":
        x, dim, h2f = rand((20, 1000), torch.float32, 22), -1, False
    elif case == "bf16_to_f32":
        x, dim, h2f = rand((20, 5000), torch.bfloat16, 23), -1, True
    elif case == "long_f32":
        x, dim, h2f = rand((3, 100003), torch.float32, 24), -1, False
    elif case == "odd":
        x, dim, h2f = rand((7, 1001), torch.bfloat16, 25), 1, False
    else:
        x, dim, h2f = rand((50, 6, 7), torch.float32, 26), 0, False
    ref = (aten.log_softmax if log else aten.softmax)(x, dim, h2f)
    out = empty_like_ref(ref)
    (_abi.log_softmax if log else _abi.softmax)(out, dev(x), dim)
    kind = "bf16" if ref.dtype == torch.bfloat16 else "fp32"
    assert_close(out, ref, kind, f"softmax {case}")


# row widths that select each register-resident block shape (256 x 1 ..
# 1024 x 16 vectors) and the two-read fallback just past it
@pytest.mark.parametrize("width,dtype", [(2048, torch.bfloat16), (4096, torch.bfloat16),
                                         (8192, torch.bfloat16), (16384, torch.bfloat16),
                                         (65536, torch.bfloat16), (131072, torch.bfloat16),
                                         (131080, torch.bfloat16), (60000, torch.float32),
                                         (65540, torch.float32)])
def test_softmax_row_shapes(width, dtype):
    x = rand((9, width), dtype, 27) * 3
    for log in (True, False):
        ref = (aten.log_softmax if log else aten.softmax)(x, -1)
        out = empty_like_ref(ref)
        (_abi.log_softmax if log else _abi.softmax)(out, dev(x), -1)
        kind = "bf16" if dtype == torch.bfloat16 else "fp32"
        assert_close(out, ref, kind, f"softmax log={log} width={width}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_softmax_nan_inf_rows(dtype):
    """A NaN anywhere in a row makes the whole row NaN (ATen's max propagates
    it); +inf makes the row NaN; an all -inf row is NaN; -inf elements give
    probability 0 (log -inf)."""
    x = rand((6, 32000), dtype, 28) * 4
    x[0, 17] = float("nan")
    x[1, 31999] = float("inf")
    x[2, :] = float("-inf")
    x[3, ::3] = float("-inf")
    x[4, 0] = float("nan")
    x[4, 1] = float("inf")
    for log in (True, False):
        ref = (aten.log_softmax if log else aten.softmax)(x, -1)
        out = empty_like_ref(ref)
        (_abi.log_softmax if log else _abi.softmax)(out, dev(x), -1)
        o = out.cpu()
        assert torch.equal(torch.isnan(o), torch.isnan(ref)), f"NaN pattern log={log}"
        assert_close(out, ref, "bf16" if dtype == torch.bfloat16 else "fp32",
                     f"softmax special log={log}")


# ---- fused efficient ops ----------------------------------------------------------

def test_config3_rms_norm_rope_silu_mul_reduced_tokens():
    c = synthetic.config3(tokens=1024)
    ref = aten.rms_norm(c["x"], c["w"], c["eps"])
    out = empty_like_ref(ref)
    _abi.rms_norm(out, dev(c["x"]), dev(c["w"]), c["eps"])
    assert_close(out, ref, "bf16", "rms_norm")
    # torch.rms_norm itself (identical on CPU)
    assert_close(out, torch.rms_norm(c["x"], [4096], c["w"], c["eps"]), "bf16", "torch.rms_norm")
    qo = torch.empty_like(dev(c["q"]))
    ko = torch.empty_like(qo)
    _abi.rope(qo, ko, dev(c["q"]), dev(c["k"]), dev(c["pos"]), c["theta"])
    assert_close(qo, aten.rope(c["q"], c["pos"], c["theta"]), "bf16", "rope q")
    assert_close(ko, aten.rope(c["k"], c["pos"], c["theta"]), "bf16", "rope k")
    ref = aten.silu_mul(c["gate"], c["up"])
    out = empty_like_ref(ref)
    _abi.silu_mul(out, dev(c["gate"]), dev(c["up"]))
    assert_close(out, ref, "bf16", "silu_mul")


def test_config3_full_size():
    c = synthetic.config3()
    out = torch.empty(c["x"].shape, dtype=torch.bfloat16, device=DEV)
    _abi.rms_norm(out, dev(c["x"]), dev(c["w"]), c["eps"])
    assert_close(out, aten.rms_norm(c["x"], c["w"], c["eps"]), "bf16", "rms_norm full")
    q = dev(c["q"])
    _abi.rope(q, None, q, None, dev(c["pos"]), c["theta"])  # in place, q only
    assert_close(q, aten.rope(c["q"], c["pos"], c["theta"]), "bf16", "rope full")
    out = torch.empty(c["gate"].shape, dtype=torch.bfloat16, device=DEV)
    _abi.silu_mul(out, dev(c["gate"]), dev(c["up"]))
    assert_close(out, aten.silu_mul(c["gate"], c["up"]), "bf16", "silu_mul full")


@pytest.mark.parametrize("tokens,hq,hk,d,dtype,with_k", [
    (37, 32, 32, 128, torch.bfloat16, True),    # ragged last block of 16 tokens
    (16, 5, 3, 64, torch.float16, True),
    (23, 4, 0, 32, torch.float32, False),        # q only
    (3, 2, 1, 4096, torch.bfloat16, True),       # one token per block (LDS-bound)
    (129, 1, 1, 16, torch.float32, True),
])
def test_rope_shapes(tokens, hq, hk, d, dtype, with_k):
    q = rand((tokens, hq, d), dtype, 34)
    pos = torch.randint(0, 8192, (tokens,), generator=g(35))
    qo = torch.empty_like(dev(q))
    if with_k:
        k = rand((tokens, hk, d), dtype, 36)
        ko = torch.empty_like(dev(k))
        _abi.rope(qo, ko, dev(q), dev(k), dev(pos), 10000.0)
        # the bf16 bar for every dtype: at positions near 8192 one ulp of the
        # fp32 angle (from powf / sincosf differing by an ulp between the
        # device and CPU libm) moves cos/sin by ~5e-4
        assert_close(ko, aten.rope(k, pos, 10000.0), "bf16", "rope k")
    else:
        _abi.rope(qo, None, dev(q), None, dev(pos), 10000.0)
    assert_close(qo, aten.rope(q, pos, 10000.0), "bf16", "rope q")


def test_fused_edge_cases():
    # rms_norm without weight, fp32, odd width (block path), strided rows
    x = rand((9, 1000), torch.float32, 27)
    out = torch.empty(9, 1000, device=DEV)
    _abi.rms_norm(out, dev(x), None, 1e-5)
    assert_close(out, aten.rms_norm(x, None, 1e-5), "fp32", "rms_norm no weight")
    big = rand((9, 2048), torch.bfloat16, 28)
    view = big[:, :1024]
    w = rand((1024,), torch.bfloat16, 29)
    out = torch.empty(9, 1024, dtype=torch.bfloat16, device=DEV)
    _abi.rms_norm(out, _strided_on_device(view), dev(w), 1e-6)
    assert_close(out, aten.rms_norm(view, w, 1e-6), "bf16", "rms_norm strided rows")
    # rope: position 0 is the identity; GQA k with fewer heads
    q = rand((4, 8, 64), torch.bfloat16, 30)
    k = rand((4, 2, 64), torch.bfloat16, 31)
    pos = torch.tensor([0, 1, 2, 4095])
    qo, ko = torch.empty_like(dev(q)), torch.empty_like(dev(k))
    _abi.rope(qo, ko, dev(q), dev(k), dev(pos.int()), 10000.0)
    assert torch.equal(qo[0].cpu(), q[0])
    assert_close(ko, aten.rope(k, pos, 10000.0), "bf16", "rope gqa k")
    # silu_mul: ragged tail and strided gate
    gt = rand((3, 1001), torch.bfloat16, 32)
    up = rand((3, 1001), torch.bfloat16, 33)
    out = torch.empty(3, 1001, dtype=torch.bfloat16, device=DEV)
    _abi.silu_mul(out, dev(gt), dev(up))
    assert_close(out, aten.silu_mul(gt, up), "bf16", "silu_mul ragged")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.int16])
@pytest.mark.parametrize("shape", [(1000, 777), (64, 64), (3, 130, 70), (1000, 776), (3, 136, 72),
                                   (8, 2048)])
def test_transpose_copy(dtype, shape):
    """copy_ of a transposed view (the tiled-transpose path) is bit-exact."""
    x = rand(shape, dtype, 40)
    view = x.transpose(-1, -2)
    out = torch.empty(view.shape, dtype=dtype, device=DEV)
    _abi.copy_(out, _strided_on_device(view))
    assert_exact(out, view.contiguous(), f"transpose copy {shape}")


# ---- cat ------------------------------------------------------------------------------

_CAT_CASES = [
    ([(4, 5, 8), (4, 3, 8), (4, 1, 8)], 1),      # 16-byte rows of several lengths
    ([(7, 33), (7, 31)], 1),                      # odd row lengths: narrower words
    ([(1000, 128), (24, 128)], 0),                # outer == 1: one run per input
    ([(2, 8, 64, 64), (2, 8, 64, 64)], 3),        # halves of a head (rotate-half pattern)
    ([(3, 4, 5)], 2),                             # one input
    ([(0, 5), (3, 5), (0, 5)], 0),                # empty inputs
    ([(2, 3)] * 40, 0),                           # more inputs than one launch takes
    ([(5, 7, 3), (5, 1, 3), (5, 12, 3)], -2),     # negative dim
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.int64, torch.uint8])
@pytest.mark.parametrize("shapes,dim", _CAT_CASES)
def test_cat_parity(dtype, shapes, dim):
    """mi_cat on dense inputs (the batched row copy) is bit-exact with CPU ATen's cat."""
    xs = [rand(s, dtype, 50 + i) for i, s in enumerate(shapes)]
    ref = aten.cat(xs, dim)
    out = torch.empty(ref.shape, dtype=dtype, device=DEV)
    _abi.cat(out, [dev(x) for x in xs], dim % ref.dim())
    assert_exact(out, ref, f"cat {shapes} dim {dim}")


def test_cat_layouts_casts_and_alignment():
    """The other paths of mi_cat: channels-last inputs and out (row copy in
    memory order), strided inputs and dtype casts (copy per input), inputs at
    addresses that are not 16-byte aligned (byte words), a strided out."""
    a = rand((2, 3, 5, 6), torch.bfloat16, 60).contiguous(memory_format=torch.channels_last)
    b = rand((2, 4, 5, 6), torch.bfloat16, 61).contiguous(memory_format=torch.channels_last)
    ref = aten.cat([a, b], 1)
    out = torch.empty(ref.shape, dtype=torch.bfloat16, device=DEV).contiguous(
        memory_format=torch.channels_last)
    _abi.cat(out, [dev(a), dev(b)], 1)
    assert_exact(out, ref, "channels-last")
    # a transposed input and an int32 input cast into a float32 out
    t = rand((6, 9), torch.float32, 62).t()
    i = rand((4, 6), torch.int32, 63)
    ref = aten.cat([t, i.float()], 0)
    out = torch.empty(ref.shape, dtype=torch.float32, device=DEV)
    _abi.cat(out, [_strided_on_device(t), dev(i)], 0)
    assert_exact(out, ref, "strided + cast")
    # uint8 inputs one byte off alignment
    base = rand((1 + 5 * 17,), torch.uint8, 64)
    x = base[1:].view(5, 17)
    y = rand((5, 3), torch.uint8, 65)
    ref = aten.cat([x, y], 1)
    out = torch.empty(ref.shape, dtype=torch.uint8, device=DEV)
    _abi.cat(out, [_strided_on_device(x), dev(y)], 1)
    assert_exact(out, ref, "misaligned bytes")
    # out is a column slice of a wider buffer
    wide = torch.zeros(5, 30, dtype=torch.uint8, device=DEV)
    _abi.cat(wide[:, 4:24], [_strided_on_device(x), dev(y)], 1)
    assert_exact(wide[:, 4:24], ref, "strided out")
    assert int(wide[:, :4].sum()) == 0 and int(wide[:, 24:].sum()) == 0


def test_cat_rejects_bad_shapes():
    x = dev(rand((4, 5), torch.float32, 66))
    y = dev(rand((3, 5), torch.float32, 67))
    with pytest.raises(_abi.MiError, match="size"):
        _abi.cat(torch.empty(7, 6, device=DEV), [x, y], 0)
    with pytest.raises(_abi.MiError, match="add up"):
        _abi.cat(torch.empty(8, 5, device=DEV), [x, y], 0)
    with pytest.raises(_abi.MiError, match="dims"):
        _abi.cat(torch.empty(7, 5, device=DEV), [x, y[0]], 0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_transpose_copy_partial_tiles(dtype):
    """Transposes whose rows or columns end inside a 16-byte piece (views cut
    from wider, aligned tensors): the edge lanes copy element by element."""
    x = rand((200, 136), dtype, 41)
    for view in [x[:, :130].t(), x[:195, :].t(), x[:3, :9].t(), x[:197, :133].t()]:
        out = torch.empty(view.shape, dtype=dtype, device=DEV)
        _abi.copy_(out, _strided_on_device(view))
        assert_exact(out, view.contiguous(), f"transpose copy {tuple(view.shape)}")


# ---- fused AdamW ----------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("amsgrad", [False, True])
def test_fused_adamw_abi(dtype, amsgrad):
    """mi_fused_adamw through the C ABI, lr read from a device tensor."""
    shapes = [(4097,), (64, 33), (1,)]
    p = [rand(s, dtype, 70 + i) for i, s in enumerate(shapes)]
    grads = [rand(s, dtype, 80 + i) for i, s in enumerate(shapes)]
    m = [(rand(s, torch.float32, 90 + i) * 0.01).to(dtype) for i, s in enumerate(shapes)]
    v = [(torch.rand(s, generator=g(95 + i)) * 1e-3).to(dtype) for i, s in enumerate(shapes)]
    vm = [t.clone() for t in v] if amsgrad else []
    steps = [torch.tensor(5.0) for _ in shapes]
    hp = dict(beta1=0.9, beta2=0.999, weight_decay=0.01, eps=1e-8, amsgrad=amsgrad, maximize=False)
    want = aten.fused_adamw(p, grads, m, v, vm, steps, lr=3e-4, **hp)
    dp, dg, dm, dv, dvm, ds = ([dev(t) for t in lst] for lst in (p, grads, m, v, vm, steps))
    _abi.fused_adamw(dp, dg, dm, dv, dvm, ds, lr=dev(torch.tensor(3e-4)), **hp)
    kind = "fp32" if dtype == torch.float32 else "bf16"
    for i in range(len(shapes)):
        assert_close(dp[i], want[0][i], kind, f"param {i}")
        assert_close(dm[i], want[2][i], kind, f"exp_avg {i}")
        assert_close(dv[i], want[3][i], kind, f"exp_avg_sq {i}")
        if amsgrad:
            assert_close(dvm[i], want[4][i], kind, f"max_exp_avg_sq {i}")


def test_fused_adamw_abi_rejects_mismatched_lists():
    p = [dev(rand((8,), torch.float32, 1))]
    with pytest.raises(_abi.MiError, match="exp_avg"):
        _abi.fused_adamw(p, [dev(rand((8,), torch.float32, 2))], [dev(rand((9,), torch.float32, 3))],
                         [dev(rand((8,), torch.float32, 4))], [], [dev(torch.tensor(1.0))],
                         lr=1e-3, beta1=0.9, beta2=0.999, weight_decay=0.0, eps=1e-8)
    with pytest.raises(_abi.MiError, match="state_step"):
        _abi.fused_adamw(p, [dev(rand((8,), torch.float32, 2))], [dev(rand((8,), torch.float32, 3))],
                         [dev(rand((8,), torch.float32, 4))], [], [dev(torch.tensor([1.0, 2.0]))],
                         lr=1e-3, beta1=0.9, beta2=0.999, weight_decay=0.0, eps=1e-8)


# ---- backward ops -----------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_backward_ops_abi(dtype):
    """mi_silu_backward, mi_log_softmax_backward / mi_softmax_backward and
    mi_layer_norm_backward through the C ABI (16-bit layer-norm column sums
    against the float64 closed form: CPU ATen adds them in 16-bit)."""
    from oracle import numpy_ref as npr
    kind = "fp32" if dtype == torch.float32 else "bf16"
    dy = rand((300, 1024), dtype, 90)
    x = rand((300, 1024), dtype, 91) * 2
    out = torch.empty(300, 1024, dtype=dtype, device=DEV)
    _abi.silu_backward(out, dev(dy), dev(x))
    assert_close(out, aten.silu_backward(dy, x), kind, "silu_backward")
    y = torch.log_softmax(x.float(), -1).to(dtype)
    _abi.log_softmax_backward(out, dev(dy), dev(y), -1)
    assert_close(out, aten.log_softmax_backward(dy, y, -1, dtype), kind, "log_softmax_backward")
    p = torch.softmax(x.float(), -1).to(dtype)
    _abi.softmax_backward(out, dev(dy), dev(p), -1)
    assert_close(out, aten.softmax_backward(dy, p, -1, dtype), kind, "softmax_backward")
    w, b = rand((1024,), dtype, 92), rand((1024,), dtype, 93)
    y_ref, mean, rstd = aten.layer_norm_forward(x, [1024], w, b, 1e-5)
    m_dev, r_dev = torch.empty(300, 1, dtype=dtype, device=DEV), torch.empty(300, 1, dtype=dtype, device=DEV)
    _abi.layer_norm(out, m_dev, r_dev, dev(x), dev(w), dev(b), 1024, 1e-5)
    assert_close(out, y_ref, kind, "layer_norm")
    assert_close(m_dev, mean, kind, "layer_norm mean")
    assert_close(r_dev, rstd, kind, "layer_norm rstd")
    want = aten.layer_norm_backward(dy, x, [1024], mean, rstd, w, b, [True, True, True])
    dw, db = torch.empty(1024, dtype=dtype, device=DEV), torch.empty(1024, dtype=dtype, device=DEV)
    _abi.layer_norm_backward(out, dw, db, dev(dy), dev(x), dev(mean), dev(rstd), dev(w), 1024)
    assert_close(out, want[0], kind, "layer_norm dx")
    _, rdw, rdb = npr.layer_norm_backward64(dy.float().numpy(), x.float().numpy(),
                                            mean.double().numpy(), rstd.double().numpy(),
                                            w.float().numpy())
    assert_close(dw, torch.from_numpy(rdw).to(dtype), kind, "layer_norm dgamma")
    assert_close(db, torch.from_numpy(rdb).to(dtype), kind, "layer_norm dbeta")
    # only the column sums, no weight
    _abi.layer_norm_backward(None, None, db, dev(dy), dev(x), dev(mean), dev(rstd), None, 1024)
    assert_close(db, torch.from_numpy(rdb).to(dtype), kind, "layer_norm dbeta alone")
