"""GPU parity of the MFMA contractions (addmm / mm / bmm / baddbmm and the
int8 weight-only linear) through the C ABI, against the fp32 closed form on
CPU (bf16 outputs: |d| <= 1e-2*|ref| + 1e-2*rms(ref); fp32: 1e-5 bars scaled
by the K-term sum)."""
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


def g(seed):
    return torch.Generator().manual_seed(seed)


def rn(shape, seed, dtype=torch.bfloat16, std=0.02):
    return (torch.randn(shape, generator=g(seed)) * std).to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(256, 256, 64), (512, 768, 1024), (300, 200, 136),
                                   (37, 1000, 72), (1, 512, 256), (1024, 64, 4096), (77, 77, 8)])
@pytest.mark.parametrize("b_layout", ["kn", "nk"])
def test_mm_parity(dtype, M, N, K, b_layout):
    a = rn((M, K), 1, dtype, 1.0)
    b = rn((K, N), 2, dtype, 1.0) if b_layout == "kn" else rn((N, K), 2, dtype, 1.0).t()
    ref = aten.addmm(None, a, b, beta=0.0)
    out = torch.empty(M, N, dtype=dtype, device="cuda")
    _abi.mm(out, a.cuda(), b.cuda() if b_layout == "kn" else b.t().contiguous().cuda().t())
    assert_close(out, ref, "bf16", f"mm {M}x{N}x{K} {b_layout}")


@pytest.mark.parametrize("bias_shape", ["row", "full", "col"])
def test_addmm_bias_alpha_beta(bias_shape):
    M, N, K = 384, 640, 512
    a, b = rn((M, K), 3), rn((K, N), 4)
    bias = {"row": rn((N,), 5), "full": rn((M, N), 5), "col": rn((M, 1), 5)}[bias_shape]
    for alpha, beta in [(1.0, 1.0), (0.5, 2.0), (1.0, 0.0)]:
        ref = aten.addmm(bias, a, b, beta=beta, alpha=alpha)
        out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        _abi.addmm(out, bias.cuda(), a.cuda(), b.cuda(), beta=beta, alpha=alpha)
        assert_close(out, ref, "bf16", f"addmm {bias_shape} a={alpha} b={beta}")
    # fp32 bias with bf16 operands
    bf = torch.randn(N, generator=g(6))
    ref = aten.addmm(bf, a, b)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    _abi.addmm(out, bf.cuda(), a.cuda(), b.cuda())
    assert_close(out, ref, "bf16", "addmm fp32 bias")


def test_config4_addmm_full_size():
    """M8192 N4096 K4096 with a row bias: the whole output against the fp32
    closed form (275 GFLOP of CPU work, about a second on the box's cores),
    plus a column checksum that is independent of the oracle's product."""
    M, N, K = 8192, 4096, 4096
    a, b, bias = rn((M, K), 7), rn((K, N), 8), rn((N,), 9)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    _abi.addmm(out, bias.cuda(), a.cuda(), b.cuda())
    got = out.cpu()
    assert_close(got, aten.addmm(bias, a, b), "bf16", "addmm config 4, every output")
    # checksum: sum over rows of C equals (sum of A rows) @ B + M * bias
    colsum = got.float().sum(0)
    want = (a.float().sum(0) @ b.float()) + M * bias.float()
    rel = ((colsum - want).norm() / want.norm()).item()
    assert rel < 2e-2, rel


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_bmm_and_baddbmm(dtype):
    B, M, N, K = 6, 130, 96, 200
    a, b = rn((B, M, K), 11, dtype, 1.0), rn((B, K, N), 12, dtype, 1.0)
    ref = aten.bmm(a, b)
    out = torch.empty(B, M, N, dtype=dtype, device="cuda")
    _abi.bmm(out, a.cuda(), b.cuda())
    assert_close(out, ref, "bf16" if dtype == torch.bfloat16 else "fp32", "bmm")
    # transposed second operand as attention uses it (q @ k^T)
    kt = rn((B, N, K), 13, dtype, 1.0)
    out2 = torch.empty(B, M, N, dtype=dtype, device="cuda")
    _abi.bmm(out2, a.cuda(), kt.cuda().transpose(1, 2))
    assert_close(out2, aten.bmm(a, kt.transpose(1, 2).contiguous()),
                 "bf16" if dtype == torch.bfloat16 else "fp32", "bmm kt")
    bias = rn((B, M, N), 14, dtype, 1.0)
    out3 = torch.empty(B, M, N, dtype=dtype, device="cuda")
    _abi.baddbmm(out3, bias.cuda(), a.cuda(), b.cuda(), beta=0.5, alpha=2.0)
    ref3 = (0.5 * bias.float() + 2.0 * torch.bmm(a.float(), b.float())).to(dtype)
    assert_close(out3, ref3, "bf16" if dtype == torch.bfloat16 else "fp32", "baddbmm")


def test_fp32_mm_and_empty_k():
    a, b = torch.randn(70, 33, generator=g(15)), torch.randn(33, 45, generator=g(16))
    out = torch.empty(70, 45, device="cuda")
    _abi.mm(out, a.cuda(), b.cuda())
    assert_close(out, a @ b, "fp32", "fp32 mm")
    z = torch.empty(5, 0, dtype=torch.bfloat16)
    w = torch.empty(0, 7, dtype=torch.bfloat16)
    out = torch.full((5, 7), 3.0, dtype=torch.bfloat16, device="cuda")
    _abi.mm(out, z.cuda(), w.cuda())
    assert (out.cpu() == 0).all()


def int8_inputs(M, N=11008, K=4096, seed=20):
    w = torch.randint(-127, 128, (N, K), generator=g(seed), dtype=torch.int8)
    scales = torch.rand(N, generator=g(seed + 1)) * 0.009 + 0.001
    x = torch.randn(M, K, generator=g(seed + 2)).to(torch.bfloat16)
    return x, w, scales


@pytest.mark.parametrize("M", [16, 256])
def test_config4_int8_linear(M):
    x, w, scales = int8_inputs(M)
    out = torch.empty(M, w.shape[0], dtype=torch.bfloat16, device="cuda")
    _abi.int8_linear(out, x.cuda(), w.cuda(), scales.cuda())
    assert_close(out, aten.int8_linear(x, w, scales), "bf16", f"int8 linear M={M}")


def test_config4_int8_linear_m4096_full():
    """M=4096: the whole [4096, 11008] output against the fp32 closed form
    (369 GFLOP of CPU work)."""
    x, w, scales = int8_inputs(4096)
    out = torch.empty(4096, w.shape[0], dtype=torch.bfloat16, device="cuda")
    _abi.int8_linear(out, x.cuda(), w.cuda(), scales.cuda())
    assert_close(out, aten.int8_linear(x, w, scales), "bf16", "int8 M=4096, every output")


def test_int8_linear_edges_and_bias():
    x, w, scales = int8_inputs(33, N=300, K=200, seed=40)
    bias = torch.randn(300, generator=g(41)).to(torch.bfloat16)
    out = torch.empty(33, 300, dtype=torch.bfloat16, device="cuda")
    _abi.int8_linear(out, x.cuda(), w.cuda(), scales.cuda(), bias.cuda())
    assert_close(out, aten.int8_linear(x, w, scales, bias), "bf16", "int8 ragged + bias")


# ---- the 256 x 256 direct-to-LDS kernel (K % 64 == 0, >= 256 tiles) ------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(4100, 4200, 128), (4096, 4096, 64), (8192, 2049, 192)])
def test_dl_kernel_ragged_tiles(dtype, M, N, K):
    a = rn((M, K), 50, dtype, 1.0)
    w = rn((N, K), 51, dtype, 1.0)  # F.linear weight, K contiguous
    ref = aten.addmm(None, a, w.t(), beta=0.0)
    out = torch.empty(M, N, dtype=dtype, device="cuda")
    _abi.mm(out, a.cuda(), w.cuda().t())
    assert_close(out, ref, "bf16", f"dl mm {M}x{N}x{K}")


@pytest.mark.parametrize("bias_shape", ["row", "full", "col", "f32row"])
def test_dl_kernel_bias_alpha_beta(bias_shape):
    M, N, K = 4160, 4096, 256
    a, w = rn((M, K), 52, std=1.0), rn((N, K), 53, std=1.0)
    bias = {"row": rn((N,), 54, std=1.0), "full": rn((M, N), 54, std=1.0),
            "col": rn((M, 1), 54, std=1.0),
            "f32row": torch.randn(N, generator=g(54))}[bias_shape]
    for alpha, beta in [(1.0, 1.0), (0.5, 2.0)]:
        ref = aten.addmm(bias, a, w.t(), beta=beta, alpha=alpha)
        out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        _abi.addmm(out, bias.cuda(), a.cuda(), w.cuda().t(), beta=beta, alpha=alpha)
        assert_close(out, ref, "bf16", f"dl addmm {bias_shape} a={alpha} b={beta}")


@pytest.mark.parametrize("kind", ["strided", "misaligned", "ragged_n", "f32_misaligned"])
def test_dl_kernel_row_bias_layouts(kind):
    """Row-broadcast bias through the epilogue's four-column loads: a strided
    view (stride 2: per-element loads), an offset view (not 8-byte aligned:
    per-element loads), an N that is not a multiple of 4 (the last run of a
    tile clamps its columns) and an fp32 bias one element into its buffer."""
    M, N, K = 4160, 4096, 128
    if kind == "ragged_n":
        N = 4098
    a, w = rn((M, K), 62, std=1.0), rn((N, K), 63, std=1.0)
    if kind == "strided":
        base = rn((2 * N,), 64, std=1.0)
        bias_cpu, bias_dev = base[::2], base.cuda()[::2]
    elif kind == "misaligned":
        base = rn((N + 1,), 64, std=1.0)
        bias_cpu, bias_dev = base[1:], base.cuda()[1:]
    elif kind == "f32_misaligned":
        base = torch.randn(N + 1, generator=g(64))
        bias_cpu, bias_dev = base[1:], base.cuda()[1:]
    else:
        bias_cpu = rn((N,), 64, std=1.0)
        bias_dev = bias_cpu.cuda()
    ref = aten.addmm(bias_cpu, a, w.t(), beta=0.75, alpha=1.25)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    _abi.addmm(out, bias_dev, a.cuda(), w.cuda().t(), beta=0.75, alpha=1.25)
    assert_close(out, ref, "bf16", f"dl addmm row bias {kind}")


def test_dl_kernel_batched_strided_and_odd_ldc():
    # bmm with enough batches to select the large-tile kernel
    B, M, N, K = 64, 512, 512, 128
    a, bt = rn((B, M, K), 55, std=1.0), rn((B, N, K), 56, std=1.0)
    out = torch.empty(B, M, N, dtype=torch.bfloat16, device="cuda")
    _abi.bmm(out, a.cuda(), bt.cuda().transpose(1, 2))
    assert_close(out, aten.bmm(a, bt.transpose(1, 2).contiguous()), "bf16", "dl bmm")
    # A rows inside a wider buffer (lda > K), output rows with an odd stride
    M, N, K = 4096, 4096, 192
    wide = rn((M, K + 64), 57, std=1.0)
    a = wide[:, 32:32 + K]
    w = rn((N, K), 58, std=1.0)
    big = torch.zeros(M, N + 3, dtype=torch.bfloat16, device="cuda")
    out = big[:, :N]
    _abi.mm(out, wide.cuda()[:, 32:32 + K], w.cuda().t())
    assert_close(out, aten.addmm(None, a, w.t(), beta=0.0), "bf16", "dl strided A, odd ldc")
    assert (big[:, N:].cpu() == 0).all()


def _gcu_allocations():
    import torch_gcu
    return torch_gcu._C._memory_stats(0)["allocation.all.allocated"]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K,bias", [(4096, 4160, 320, True), (2048, 8200, 192, False),
                                        (4000, 4096, 64, True)])
def test_row_major_b_read_in_place(dtype, M, N, K, bias):
    """B as a row-major [K, N] matrix with M <= 4096 is read in place by the
    large-tile kernel (transposed fragment reads from LDS): no workspace is
    taken, ragged last row and column tiles included."""
    a, b = rn((M, K), 59, dtype, 1.0), rn((K, N), 60, dtype, 1.0)
    bi = rn((N,), 61, dtype, 1.0) if bias else None
    out = torch.empty(M, N, dtype=dtype, device="cuda")
    ad, bd, bid = a.cuda(), b.cuda(), (bi.cuda() if bias else None)
    torch.cuda.synchronize()
    n0 = _gcu_allocations()
    if bias:
        _abi.addmm(out, bid, ad, bd)
    else:
        _abi.mm(out, ad, bd)
    torch.cuda.synchronize()
    assert _gcu_allocations() == n0, "row-major B took workspace (the transpose copy)"
    assert_close(out, aten.addmm(bi, a, b, beta=1.0 if bias else 0.0), "bf16",
                 f"row-major B {M}x{N}x{K}")


def test_row_major_b_strided_batched_and_fallback():
    """Row-major B inside a wider buffer (row stride > N), a batched product
    with row-major B, and an N that is not a multiple of 8 (whole 16-byte
    column chunks are required), which goes through the transpose copy."""
    M, N, K = 4096, 4096, 192
    a = rn((M, K), 65, std=1.0)
    wide = rn((K, N + 64), 66, std=1.0)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    _abi.mm(out, a.cuda(), wide.cuda()[:, 16:16 + N])
    assert_close(out, aten.addmm(None, a, wide[:, 16:16 + N], beta=0.0), "bf16",
                 "row-major B, row stride > N")
    Bn, M, N, K = 64, 512, 512, 128
    a, b = rn((Bn, M, K), 67, std=1.0), rn((Bn, K, N), 68, std=1.0)
    out = torch.empty(Bn, M, N, dtype=torch.bfloat16, device="cuda")
    _abi.bmm(out, a.cuda(), b.cuda())
    assert_close(out, aten.bmm(a, b), "bf16", "batched row-major B")
    M, N, K = 4096, 4098, 128
    a, b = rn((M, K), 69, std=1.0), rn((K, N), 70, std=1.0)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ad, bd = a.cuda(), b.cuda()
    torch.cuda.synchronize()
    n0 = _gcu_allocations()
    _abi.mm(out, ad, bd)
    torch.cuda.synchronize()
    assert _gcu_allocations() > n0, "N % 8 != 0 should take the transpose copy"
    assert_close(out, aten.addmm(None, a, b, beta=0.0), "bf16", "row-major B, N % 8 != 0")
    # M > 4096: the K-contiguous copy of B, then the large-tile kernel
    M, N, K = 8192, 4096, 128
    a, b, bias = rn((M, K), 71, std=1.0), rn((K, N), 72, std=1.0), rn((N,), 73, std=1.0)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ad, bd, bid = a.cuda(), b.cuda(), bias.cuda()
    torch.cuda.synchronize()
    n0 = _gcu_allocations()
    _abi.addmm(out, bid, ad, bd)
    torch.cuda.synchronize()
    assert _gcu_allocations() > n0, "M > 4096 should take the transpose copy"
    assert_close(out, aten.addmm(bias, a, b), "bf16", "row-major B, M > 4096")


@pytest.mark.parametrize("M,N,K", [(1, 1000, 256), (16, 11008, 4096), (33, 520, 1024),
                                   (64, 4096, 640), (7, 17, 128), (5, 40, 192),
                                   (48, 1000, 2048), (2, 33, 3072), (64, 96, 5120)])
@pytest.mark.parametrize("bias", [None, "bf16", "f32"])
def test_int8_linear_skinny(M, N, K, bias):
    """M <= 64: K % 1024 == 0 takes the LDS-staged weight stream (N / CUs W
    rows per block, at least 16 and at most 48, in 1 KiB slabs that each
    wave streams through its own ring: slab counts of 1, 2, 3 and 5 against
    the three-slot ring, ragged N, blocks with a single row), other
    K % 128 == 0 the register weight stream (K split over eight waves);
    partial tiles are added in a fixed order.  K = 192 exercises the general
    kernel's int8 path."""
    x, w, scales = int8_inputs(M, N=N, K=K, seed=70 + M)
    b = None
    if bias == "bf16":
        b = torch.randn(N, generator=g(71)).to(torch.bfloat16)
    elif bias == "f32":
        b = torch.randn(N, generator=g(72))
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    _abi.int8_linear(out, x.cuda(), w.cuda(), scales.cuda(), None if b is None else b.cuda())
    assert_close(out, aten.int8_linear(x, w, scales, b), "bf16", f"skinny M={M} N={N} K={K} {bias}")


@pytest.mark.parametrize("K", [512, 2048])
def test_int8_linear_skinny_f16(K):
    x, w, scales = int8_inputs(24, N=777, K=K, seed=80)
    x = x.to(torch.float16)
    out = torch.empty(24, 777, dtype=torch.float16, device="cuda")
    _abi.int8_linear(out, x.cuda(), w.cuda(), scales.cuda())
    assert_close(out, aten.int8_linear(x, w, scales), "bf16", f"skinny f16 K={K}")


@pytest.mark.parametrize("dtype,bias", [(torch.bfloat16, None), (torch.bfloat16, "bf16"),
                                        (torch.float16, "f32")])
def test_int8_linear_large_tile_path(dtype, bias):
    """M > 64 with >= 256 tiles of 256 x 256: int8 W rows DMA'd into LDS and
    widened to 16-bit at fragment read, per-column scale in the epilogue."""
    M, N, K = 4096, 4100, 192
    x, w, scales = int8_inputs(M, N=N, K=K, seed=90)
    x = x.to(dtype)
    b = None
    if bias == "bf16":
        b = torch.randn(N, generator=g(91)).to(torch.bfloat16)
    elif bias == "f32":
        b = torch.randn(N, generator=g(92))
    out = torch.empty(M, N, dtype=dtype, device="cuda")
    _abi.int8_linear(out, x.cuda(), w.cuda(), scales.cuda(), None if b is None else b.cuda())
    assert_close(out, aten.int8_linear(x, w, scales, b), "bf16", f"int8 large tile {dtype} {bias}")


@pytest.mark.parametrize("M,N,K,dtype,bias", [
    (256, 1000, 1024, torch.bfloat16, None),     # split-K: 4 tiles x 16 slices of one K step
    (256, 1001, 512, torch.bfloat16, "f32"),     # split-K, N not a multiple of 4, fp32 bias
    (512, 4104, 512, torch.float16, "f32"),      # split-K: 2 x 17 tiles x 7 uneven slices
    (65, 96, 128, torch.bfloat16, "row"),        # split-K, smallest M of the path, [M, N] bias
    (200, 777, 64, torch.bfloat16, "bf16"),      # one K step: 128-row tiles, odd N
    (130, 65536, 128, torch.bfloat16, "bf16"),   # 256 tiles fill the CUs: 128-row tiles
])
def test_int8_linear_mid_path(M, N, K, dtype, bias):
    """64 < M <= 512: split-K over 256 x 256 tiles with an fp32 combine when
    the tiles are too few to fill the CUs (config 4's M = 256: 43 tiles x 5
    slices), else 128-row x tiles against W panels sized to the CUs."""
    x, w, scales = int8_inputs(M, N=N, K=K, seed=100 + M)
    x = x.to(dtype)
    b = None
    if bias == "bf16":
        b = torch.randn(N, generator=g(101)).to(torch.bfloat16)
    elif bias == "f32":
        b = torch.randn(N, generator=g(102))
    elif bias == "row":
        b = torch.randn(M, N, generator=g(103)).to(dtype)
    out = torch.empty(M, N, dtype=dtype, device="cuda")
    _abi.int8_linear(out, x.cuda(), w.cuda(), scales.cuda(), None if b is None else b.cuda())
    assert_close(out, aten.int8_linear(x, w, scales, b), "bf16", f"int8 mid {M},{N},{K} {dtype} {bias}")


@pytest.mark.parametrize("dtype,bias", [(torch.float16, "f32"), (torch.float16, None),
                                        (torch.bfloat16, "f32")])
def test_int8_linear_register_staged_path(dtype, bias):
    """M > 512 with fewer 256 x 256 tiles than CUs: 128 x 64 tiles whose int8
    W rows are widened to the type of x on the way into LDS (an f16 x used to
    get bf16 bit patterns there)."""
    M, N, K = 1024, 4104, 512
    x, w, scales = int8_inputs(M, N=N, K=K, seed=110)
    x = x.to(dtype)
    b = torch.randn(N, generator=g(111)) if bias == "f32" else None
    out = torch.empty(M, N, dtype=dtype, device="cuda")
    _abi.int8_linear(out, x.cuda(), w.cuda(), scales.cuda(), None if b is None else b.cuda())
    assert_close(out, aten.int8_linear(x, w, scales, b), "bf16", f"int8 staged {dtype} {bias}")


# ---- addmv (GEMV) and the linear / matmul override ---------------------------------

def _kind(dtype):
    return "fp32" if dtype == torch.float32 else "bf16"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M,K", [(11008, 4096), (1000, 37), (1, 4096), (77, 1), (300, 520)])
@pytest.mark.parametrize("layout", ["rows", "transposed", "sliced"])
def test_addmv_parity(dtype, M, K, layout):
    """mat K-contiguous (the kernel's own layout), a transposed view and a
    column slice (row stride that breaks 16-byte alignment: both copied
    densely first); bias [M], beta and alpha not 1."""
    if layout == "rows":
        mat = rn((M, K), 30, dtype, 1.0)
    elif layout == "transposed":
        mat = rn((K, M), 30, dtype, 1.0).t()
    else:
        mat = rn((M, K + 3), 30, dtype, 1.0)[:, 1:K + 1]
    vec = rn((K,), 31, dtype, 1.0)
    bias = rn((M,), 32, dtype, 1.0)
    ref = aten.addmv(bias, mat, vec, beta=0.5, alpha=2.0)
    md = mat.cuda() if layout == "rows" else (
        mat.t().contiguous().cuda().t() if layout == "transposed" else
        rn((M, K + 3), 30, dtype, 1.0).cuda()[:, 1:K + 1])
    out = torch.empty(M, dtype=dtype, device="cuda")
    _abi.addmv(out, bias.cuda(), md, vec.cuda(), beta=0.5, alpha=2.0)
    assert_close(out, ref, _kind(dtype), f"addmv {dtype} {M}x{K} {layout}")


def test_addmv_edges():
    """Strided vec, scalar and fp32 bias, beta = 0 with a NaN bias, alpha = 0
    with NaN in mat, K = 0, a strided output."""
    M, K = 513, 300
    mat, v2 = rn((M, K), 33, torch.bfloat16, 1.0), rn((2 * K,), 34, torch.bfloat16, 1.0)
    vec = v2[::2]
    out = torch.empty(M, dtype=torch.bfloat16, device="cuda")
    _abi.addmv(out, torch.tensor([0.25], dtype=torch.bfloat16).cuda(), mat.cuda(), v2.cuda()[::2])
    assert_close(out, aten.addmv(torch.full((M,), 0.25).bfloat16(), mat, vec), "bf16", "strided vec")
    b32 = torch.randn(M, generator=g(35))
    _abi.addmv(out, b32.cuda(), mat.cuda(), vec.contiguous().cuda(), beta=1.0, alpha=0.5)
    assert_close(out, aten.addmv(b32, mat.float(), vec.float(), alpha=0.5).bfloat16(), "bf16",
                 "fp32 bias")
    nanb = torch.full((M,), float("nan"), dtype=torch.bfloat16)
    _abi.addmv(out, nanb.cuda(), mat.cuda(), vec.contiguous().cuda(), beta=0.0)
    assert torch.isfinite(out.float()).all()
    nm = mat.clone()
    nm[7, 11] = float("nan")
    bias = rn((M,), 36, torch.bfloat16, 1.0)
    _abi.addmv(out, bias.cuda(), nm.cuda(), vec.contiguous().cuda(), beta=1.0, alpha=0.0)
    assert torch.equal(out.cpu(), bias)
    e = torch.empty(M, 0, dtype=torch.bfloat16, device="cuda")
    _abi.addmv(out, bias.cuda(), e, torch.empty(0, dtype=torch.bfloat16, device="cuda"), beta=2.0)
    assert_close(out, (2.0 * bias.float()).bfloat16(), "bf16", "K = 0")
    wide = torch.zeros(2 * M, dtype=torch.bfloat16, device="cuda")
    _abi.addmv(wide[::2], None, mat.cuda(), vec.contiguous().cuda(), beta=0.0)
    assert_close(wide[::2], aten.addmv(None, mat, vec), "bf16", "strided out")
    assert torch.count_nonzero(wide[1::2].float()) == 0


def test_mv_and_matmul_on_gcu_run_native_addmv():
    """torch.mv / torch.addmv / matmul(2-D, 1-D) on gcu tensors reach the
    native addmv (no CPU fallback counted)."""
    import torch_gcu

    mat = rn((640, 256), 37, torch.bfloat16, 1.0)
    vec = rn((256,), 38, torch.bfloat16, 1.0)
    bias = rn((640,), 39, torch.bfloat16, 1.0)
    torch_gcu._C._set_op_debug_config("op_statistics=true")
    torch_gcu._C._clear_op_statistics()
    try:
        mg, vg, bg = mat.to("gcu"), vec.to("gcu"), bias.to("gcu")
        r1 = torch.mv(mg, vg)
        r2 = torch.addmv(bg, mg, vg, beta=0.5, alpha=1.5)
        r3 = mg @ vg
        stats = torch_gcu._C._op_statistics()
    finally:
        torch_gcu._C._set_op_debug_config("")
    ref = aten.addmv(None, mat, vec)
    assert_close(r1.cpu(), ref, "bf16", "mv")
    assert_close(r3.cpu(), ref, "bf16", "matmul 2-D x 1-D")
    assert_close(r2.cpu(), aten.addmv(bias, mat, vec, beta=0.5, alpha=1.5), "bf16", "addmv")
    native = {k: v for k, v in stats.items() if k.startswith("addmv")}
    assert sum(v[0] for v in native.values()) >= 3, stats
    assert all(v[1] == 0 for v in native.values()), stats


_OVERRIDE_SCRIPT = r"""
import sys, torch, torch.nn.functional as F
import torch_gcu
from oracle import aten
from oracle.tolerance import assert_close
names = ("aten::linear", "aten::linear.out", "aten::matmul", "aten::matmul.out")
assert all(torch._C._dispatch_has_kernel_for_dispatch_key(n, "PrivateUse1") for n in names)
g = torch.Generator().manual_seed(40)
x3 = torch.randn(4, 96, 256, generator=g).bfloat16()
w = (torch.randn(384, 256, generator=g) * 0.05).bfloat16()
b = torch.randn(384, generator=g).bfloat16()
torch_gcu._C._set_op_debug_config("op_statistics=true")
torch_gcu._C._clear_op_statistics()
y = F.linear(x3.to("gcu"), w.to("gcu"), b.to("gcu"))
y2 = F.linear(x3[:, ::2].to("gcu"), w.to("gcu"))            # strided input, no bias
m = torch.matmul(x3.to("gcu"), w.t().to("gcu"))              # 3-D x 2-D: folded to mm
mv = torch.matmul(w.to("gcu"), x3[0, 0].to("gcu"))           # 2-D x 1-D: mv
bm = torch.matmul(x3.to("gcu"), x3.transpose(1, 2).contiguous().to("gcu"))  # batched
out = torch.empty(0, dtype=torch.bfloat16, device="gcu")
torch.matmul(x3[0].to("gcu"), w.t().to("gcu"), out=out)
stats = torch_gcu._C._op_statistics()
torch_gcu._C._set_op_debug_config("")
ref = (x3.float() @ w.float().t() + b.float()).bfloat16()
assert_close(y.cpu(), ref, "bf16", "linear 3-D + bias")
assert_close(y2.cpu(), (x3[:, ::2].float() @ w.float().t()).bfloat16(), "bf16", "linear strided")
assert_close(m.cpu(), (x3.float() @ w.float().t()).bfloat16(), "bf16", "matmul 3-D x 2-D")
assert_close(mv.cpu(), aten.addmv(None, w, x3[0, 0]), "bf16", "matmul 2-D x 1-D")
assert_close(bm.cpu(), aten.bmm(x3, x3.transpose(1, 2).contiguous()), "bf16", "matmul batched")
assert_close(out.cpu(), (x3[0].float() @ w.float().t()).bfloat16(), "bf16", "matmul.out")
assert stats.get("linear", (0, 0))[0] == 2, stats
assert stats.get("matmul", (0, 0))[0] == 3 and stats.get("matmul.out", (0, 0))[0] == 1, stats
assert all(v[1] == 0 for k, v in stats.items()), stats   # nothing fell back to CPU
print("override ok")
"""


def test_linear_matmul_override_on_gpu():
    """With ENFLAME_PT_ENABLE_LINEAR_OVERRIDE=true (read at library load, so
    in a child process), linear and matmul on gcu run the native folding
    onto mm / addmm / bmm / addmv and match CPU ATen."""
    import os
    import subprocess
    import sys

    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, ENFLAME_PT_ENABLE_LINEAR_OVERRIDE="true")
    env["PYTHONPATH"] = os.pathsep.join([os.path.join(repo, "torch-gcu_amd"), repo,
                                         env.get("PYTHONPATH", "")])
    r = subprocess.run([sys.executable, "-c", _OVERRIDE_SCRIPT], env=env, capture_output=True,
                       text=True, timeout=110)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-3000:])
    assert "override ok" in r.stdout
