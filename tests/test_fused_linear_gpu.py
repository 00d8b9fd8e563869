"""GPU parity of the fused matmul epilogues through the C ABI:
mi_linear_residual (residual + x @ W^T) and mi_linear_silu_mul
(silu(x @ Wg^T) * (x @ Wu^T)).

Each must equal, bit for bit, the unfused gcu ops it replaces (the matmul,
rounded to the input dtype, then add or silu_mul), and match the CPU ATen
composition at the bf16 bar.  The shapes take both paths: the large-tile
kernel with the epilogue (at least 256 output tiles of 256 x 256, or of 128
output columns for silu_mul; exact and ragged edges) and the unfused
fallback (K not a multiple of 64, or too few tiles)."""
import pytest
import torch

from oracle import aten
from oracle.tolerance import assert_close
from torch_gcu import _abi

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _setup():
    torch.cuda.init()
    _abi.install_workspace()
    yield
    torch.cuda.synchronize()


def rn(shape, seed, dtype, std):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(dtype)


def assert_equal_bits(a, b, what):
    a, b = a.cpu(), b.cpu()
    same = a.view(torch.int16) == b.view(torch.int16)
    assert bool(same.all()), f"{what}: {int((~same).sum())} of {a.numel()} elements differ"


# (M, N, K): fused with exact tiles, fused with ragged M and N, and the fallback
# for K % 64 != 0 and for too few tiles.  The fused shapes have at least 256
# tiles of 256 x 256, so the unfused matmul they are compared with runs the
# same large-tile kernel (the decoder layer's projections all do); kernels
# with other MFMA shapes round the same products differently.
RESID_SHAPES = [(2048, 8192, 128), (4000, 4100, 64), (64, 200, 96), (300, 500, 128)]
SILU_SHAPES = [(4096, 4096, 128), (4000, 4100, 64), (64, 200, 96), (300, 500, 128)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", RESID_SHAPES)
def test_linear_residual_equals_unfused_and_cpu(dtype, M, N, K):
    x, w = rn((M, K), 1, dtype, 1.0), rn((N, K), 2, dtype, 0.2)
    r = rn((M, N), 3, dtype, 1.0)
    xd, wd, rd = x.cuda(), w.cuda(), r.cuda()
    out = torch.empty(M, N, dtype=dtype, device="cuda")
    _abi.linear_residual(out, xd, wd, rd)
    prod = torch.empty(M, N, dtype=dtype, device="cuda")
    _abi.mm(prod, xd, wd.t())
    unfused = torch.empty(M, N, dtype=dtype, device="cuda")
    _abi.add(unfused, rd, prod)
    torch.cuda.synchronize()
    assert_equal_bits(out, unfused, f"linear_residual {M}x{N}x{K}")
    ref = aten.add(r, aten.addmm(None, x, w.t(), beta=0.0))
    assert_close(out, ref, "bf16", f"linear_residual vs CPU {M}x{N}x{K}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", SILU_SHAPES)
def test_linear_silu_mul_equals_unfused_and_cpu(dtype, M, N, K):
    x = rn((M, K), 4, dtype, 1.0)
    wg, wu = rn((N, K), 5, dtype, 0.3), rn((N, K), 6, dtype, 0.3)
    xd, gd, ud = x.cuda(), wg.cuda(), wu.cuda()
    out = torch.empty(M, N, dtype=dtype, device="cuda")
    _abi.linear_silu_mul(out, xd, gd, ud)
    g_ = torch.empty(M, N, dtype=dtype, device="cuda")
    u_ = torch.empty(M, N, dtype=dtype, device="cuda")
    _abi.mm(g_, xd, gd.t())
    _abi.mm(u_, xd, ud.t())
    unfused = torch.empty(M, N, dtype=dtype, device="cuda")
    _abi.silu_mul(unfused, g_, u_)
    torch.cuda.synchronize()
    assert_equal_bits(out, unfused, f"linear_silu_mul {M}x{N}x{K}")
    ref = aten.silu_mul(aten.addmm(None, x, wg.t(), beta=0.0), aten.addmm(None, x, wu.t(), beta=0.0))
    assert_close(out, ref, "bf16", f"linear_silu_mul vs CPU {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(2048, 8192, 128), (64, 200, 96)])
def test_linear_residual_in_place_and_strided(M, N, K):
    """out may be the residual itself; a residual with a padded row stride
    and a view of x with a padded row stride give the same bits."""
    dtype = torch.bfloat16
    x, w, r = rn((M, K), 7, dtype, 1.0), rn((N, K), 8, dtype, 0.2), rn((M, N), 9, dtype, 1.0)
    want = torch.empty(M, N, dtype=dtype, device="cuda")
    _abi.linear_residual(want, x.cuda(), w.cuda(), r.cuda())
    inplace = r.cuda()
    _abi.linear_residual(inplace, x.cuda(), w.cuda(), inplace)
    xpad = torch.zeros(M, K + 64, dtype=dtype, device="cuda")
    xpad[:, :K] = x.cuda()
    rpad = torch.zeros(M, N + 8, dtype=dtype, device="cuda")
    rpad[:, :N] = r.cuda()
    strided = torch.empty(M, N, dtype=dtype, device="cuda")
    _abi.linear_residual(strided, xpad[:, :K], w.cuda(), rpad[:, :N])
    torch.cuda.synchronize()
    assert_equal_bits(inplace, want, "in place")
    assert_equal_bits(strided, want, "padded row strides")


def test_fused_linear_argument_checks():
    dtype = torch.bfloat16
    x = torch.zeros(64, 128, dtype=dtype, device="cuda")
    w = torch.zeros(32, 128, dtype=dtype, device="cuda")
    out = torch.empty(64, 32, dtype=dtype, device="cuda")
    with pytest.raises(RuntimeError, match="residual has the wrong shape"):
        _abi.linear_residual(out, x, w, torch.zeros(64, 31, dtype=dtype, device="cuda"))
    with pytest.raises(RuntimeError, match="share a dtype"):
        _abi.linear_residual(out, x, w, torch.zeros(64, 32, dtype=torch.float16, device="cuda"))
    with pytest.raises(RuntimeError, match="w_up has the wrong shape"):
        _abi.linear_silu_mul(out, x, w, torch.zeros(32, 64, dtype=dtype, device="cuda"))
    with pytest.raises(RuntimeError, match="features"):
        _abi.linear_silu_mul(out, x, torch.zeros(32, 96, dtype=dtype, device="cuda"),
                             torch.zeros(32, 96, dtype=dtype, device="cuda"))


def test_efficient_ops_on_gcu_tensors():
    """torch.gcu.efficient.linear_residual / linear_silu_mul on gcu tensors
    (leading dims flattened) equal the ops they fuse, run on gcu."""
    import torch.nn.functional as F
    import torch_gcu  # noqa: F401

    dtype = torch.bfloat16
    x = rn((4, 1024, 128), 10, dtype, 1.0).to("gcu")
    w = rn((4096, 128), 11, dtype, 0.2).to("gcu")
    wu = rn((4096, 128), 12, dtype, 0.2).to("gcu")
    r = rn((4, 1024, 4096), 13, dtype, 1.0).to("gcu")
    got = torch.gcu.efficient.linear_residual(x, w, r)
    want = r + F.linear(x, w)
    assert got.shape == want.shape
    assert_equal_bits(got, want, "efficient.linear_residual")
    got = torch.gcu.efficient.linear_silu_mul(x, w, wu)
    want = torch.gcu.efficient.silu_mul(F.linear(x, w), F.linear(x, wu))
    assert got.shape == want.shape
    assert_equal_bits(got, want, "efficient.linear_silu_mul")
