"""GPU regression test for the direct-to-LDS tile copies (lds_copy16) of the
flash attention and large-tile GEMM kernels.

A copy takes a wave-uniform 64-bit base read as two 32-bit words.  A build
that widened the low word with sign extension turned every base whose low
word has bit 31 set into an address with all-ones high bits.  These tests
place the copied operands at such addresses and check that the results equal,
bit for bit, the same calls on ordinary allocations."""
import pytest
import torch

from torch_gcu import _abi

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _setup():
    torch.cuda.init()
    _abi.install_workspace()
    yield
    torch.cuda.synchronize()


def high_half(shape, dtype):
    """An uninitialised tensor whose every byte lies at an address with bit 31
    of its low 32-bit word set (a view into a 4 GiB + n allocation)."""
    n = int(torch.Size(shape).numel()) * torch.empty((), dtype=dtype).element_size()
    assert n < (1 << 30)
    buf = torch.empty((1 << 32) + n + 4096, dtype=torch.uint8, device="cuda")
    low = buf.data_ptr() & 0xFFFFFFFF
    off = 0 if low >= 0x80000000 and low + n < (1 << 32) else (0x80000000 - low) % (1 << 32)
    t = buf[off:off + n].view(dtype).view(shape)
    a = t.data_ptr()
    assert (a & 0xFFFFFFFF) >= 0x80000000 and ((a + n - 1) & 0xFFFFFFFF) >= 0x80000000
    return t, buf


def rn(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def assert_equal_bits(a, b, what):
    a, b = a.cpu(), b.cpu()
    same = a.view(torch.int16) == b.view(torch.int16)
    assert bool(same.all()), f"{what}: {int((~same).sum())} of {a.numel()} elements differ"


@pytest.mark.parametrize("Sk", [256, 200])  # full key tiles, then a ragged last tile
def test_flash_attention_kv_at_bit31_addresses(Sk):
    B, H, Sq, D = 1, 4, 256, 128
    q, k, v = rn((B, H, Sq, D), 1), rn((B, H, Sk, D), 2), rn((B, H, Sk, D), 3)
    qd = q.cuda()
    k_hi, kbuf = high_half((B, H, Sk, D), torch.bfloat16)
    v_hi, vbuf = high_half((B, H, Sk, D), torch.bfloat16)
    k_hi.copy_(k.cuda())
    v_hi.copy_(v.cuda())
    want = torch.empty(B, H, Sq, D, dtype=torch.bfloat16, device="cuda")
    got = torch.empty_like(want)
    lse_w = torch.empty(B, H, Sq, dtype=torch.float32, device="cuda")
    lse_g = torch.empty_like(lse_w)
    _abi.flash_attention_fwd(want, lse_w, qd, k.cuda(), v.cuda(), True)
    _abi.flash_attention_fwd(got, lse_g, qd, k_hi, v_hi, True)
    torch.cuda.synchronize()
    assert_equal_bits(got, want, f"attention, K/V at bit-31 addresses, Sk={Sk}")
    assert torch.equal(lse_g.cpu(), lse_w.cpu())
    del kbuf, vbuf


def test_gemm_operands_at_bit31_addresses():
    # 16 x 16 tiles of 256 x 256: the large-tile kernel, whose copies read A and B
    M, N, K = 4096, 4096, 256
    a, b = rn((M, K), 4), rn((N, K), 5, 0.2)
    a_hi, abuf = high_half((M, K), torch.bfloat16)
    b_hi, bbuf = high_half((N, K), torch.bfloat16)
    a_hi.copy_(a.cuda())
    b_hi.copy_(b.cuda())
    want = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    got = torch.empty_like(want)
    _abi.mm(want, a.cuda(), b.cuda().t())
    _abi.mm(got, a_hi, b_hi.t())
    torch.cuda.synchronize()
    assert_equal_bits(got, want, "mm, A and B at bit-31 addresses")
    del abuf, bbuf
