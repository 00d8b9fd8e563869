"""Copies and transfers on the "gcu" device on the GPU: pinned host memory
from the caching host allocator, host-device copies (blocking and
non-blocking, casts on the device, strided and broadcast operands), and
torch.cat, each checked bit-exact against CPU ATen (the reference's fallback
path) on the same inputs."""
import pytest
import torch

import torch_gcu
from oracle import aten
from oracle.tolerance import assert_exact

pytestmark = pytest.mark.gpu

C = torch_gcu._C


def g(seed):
    return torch.Generator().manual_seed(seed)


def rand(shape, dtype, seed):
    if dtype.is_floating_point:
        return torch.randn(shape, generator=g(seed)).to(dtype)
    if dtype == torch.bool:
        return torch.randint(0, 2, shape, generator=g(seed)).bool()
    lo, hi = (0, 255) if dtype == torch.uint8 else (-1000, 1000)
    return torch.randint(lo, hi, shape, generator=g(seed)).to(dtype)


@pytest.fixture(autouse=True)
def _clean():
    C._set_op_debug_config("")
    yield
    C._set_op_debug_config("")
    torch.gcu.synchronize()


# ---- pinned host memory --------------------------------------------------------------

def test_pinned_memory_comes_from_the_host_caching_allocator():
    st0 = torch.gcu.host_memory_stats()
    a = torch.empty(3 << 20, dtype=torch.uint8, pin_memory=True)
    assert a.is_pinned() and a[12345:].is_pinned()
    st1 = torch.gcu.host_memory_stats()
    assert st1["allocated_bytes"] - st0["allocated_bytes"] == 4 << 20, (st0, st1)
    x = rand((300, 7), torch.float32, 1)
    assert not x.is_pinned()
    y = x.pin_memory()
    assert y.is_pinned() and torch.equal(x, y)
    pa = a.data_ptr()
    del a
    b = torch.empty(4 << 20, dtype=torch.uint8, pin_memory=True)  # same 4 MiB class
    assert b.data_ptr() == pa
    del b, y
    torch.gcu.host_empty_cache()
    st2 = torch.gcu.host_memory_stats()
    assert st2["allocated_bytes"] == st0["allocated_bytes"], st2
    assert st2["num_host_free"] > st0["num_host_free"], st2


# ---- host <-> device copies ---------------------------------------------------------

_CASTS = [
    (torch.float32, torch.float32), (torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32),
    (torch.float32, torch.float16), (torch.int64, torch.float32), (torch.float32, torch.int32),
    (torch.bool, torch.float32), (torch.float32, torch.bool), (torch.uint8, torch.int64),
    (torch.float64, torch.bfloat16),
]


@pytest.mark.parametrize("src_dt,dst_dt", _CASTS)
@pytest.mark.parametrize("non_blocking", [False, True])
@pytest.mark.parametrize("pinned", [False, True])
def test_h2d_d2h_parity(src_dt, dst_dt, non_blocking, pinned):
    """host -> device and device -> host, each into dst's dtype, from and into
    pageable or pinned memory; dense operands take the one-memcpy path."""
    x = rand((257, 129), src_dt, 2)
    if pinned:
        x = x.pin_memory()
    d = torch.empty(257, 129, dtype=dst_dt, device="gcu")
    d.copy_(x, non_blocking=non_blocking)
    back = torch.empty(257, 129, dtype=src_dt, pin_memory=pinned)
    back.copy_(d, non_blocking=non_blocking)
    torch.gcu.synchronize()
    want = aten.copy(torch.empty(257, 129, dtype=dst_dt), x)
    assert_exact(d.cpu(), want, f"H2D {src_dt}->{dst_dt}")
    assert_exact(back, aten.copy(torch.empty(257, 129, dtype=src_dt), want), f"D2H {dst_dt}->{src_dt}")


@pytest.mark.parametrize("non_blocking", [False, True])
def test_h2d_d2h_layouts(non_blocking):
    """Strided, broadcast and channels-last operands on either side."""
    base = rand((64, 96), torch.float32, 3)
    # a transposed and a stepped host source
    for src in (base.t(), base[::3, 5:70]):
        d = torch.empty(src.shape, dtype=torch.bfloat16, device="gcu")
        d.copy_(src, non_blocking=non_blocking)
        torch.gcu.synchronize()
        assert_exact(d.cpu(), aten.copy(torch.empty(src.shape, dtype=torch.bfloat16), src), "strided src")
    # broadcast: one host row into every row of a device matrix
    row = rand((96,), torch.float32, 4)
    d = torch.empty(64, 96, device="gcu")
    d.copy_(row, non_blocking=non_blocking)
    torch.gcu.synchronize()
    assert_exact(d.cpu(), row.expand(64, 96), "broadcast src")
    # a strided device destination (a column band of a wider tensor)
    wide = torch.zeros(64, 200, device="gcu")
    wide[:, 50:146].copy_(base, non_blocking=non_blocking)
    torch.gcu.synchronize()
    w = wide.cpu()
    assert_exact(w[:, 50:146], base, "strided dst")
    assert float(w[:, :50].abs().sum()) == 0.0 and float(w[:, 146:].abs().sum()) == 0.0
    # channels-last on both sides
    img = rand((2, 3, 8, 5), torch.float32, 5).contiguous(memory_format=torch.channels_last)
    d = torch.empty(2, 3, 8, 5, dtype=torch.float16, device="gcu")
    d.copy_(img, non_blocking=non_blocking)
    cl = torch.empty(2, 3, 8, 5).contiguous(memory_format=torch.channels_last)
    cl.copy_(d, non_blocking=non_blocking)
    torch.gcu.synchronize()
    assert_exact(cl, img.half().float(), "channels-last round trip")
    # a strided host destination (device -> transposed host view)
    dd = base.to("gcu")
    ht = torch.zeros(96, 64).t()
    ht.copy_(dd, non_blocking=non_blocking)
    torch.gcu.synchronize()
    assert_exact(ht, base, "strided dst on the host")
    # dtypes the copy kernel does not convert are cast on the host
    u = torch.arange(0, 2000, 7).to(torch.uint32)
    d = torch.empty(u.shape, dtype=torch.int64, device="gcu")
    d.copy_(u, non_blocking=non_blocking)
    back = torch.empty(u.shape, dtype=torch.uint32)
    back.copy_(d, non_blocking=non_blocking)
    torch.gcu.synchronize()
    assert torch.equal(d.cpu(), u.long()) and torch.equal(back, u)
    # empty tensors
    e = torch.empty(0, 5, device="gcu")
    e.copy_(torch.empty(0, 5), non_blocking=non_blocking)
    assert e.cpu().shape == (0, 5)


def test_to_and_to_copy_run_natively():
    """x.to("gcu"), x.to(dtype) and x.to("cpu") go through _to_copy (a
    composite of empty + copy_) to the native _copy_from and nothing falls
    back to CPU ATen; a non-blocking device -> host .to() lands in pinned memory."""
    x = rand((33, 65), torch.float32, 6)
    C._set_op_debug_config("op_statistics=true")
    C._clear_op_statistics()
    try:
        d = x.to("gcu")
        h = d.to(torch.bfloat16)
        back = h.to("cpu")
        nb = d.to("cpu", non_blocking=True)
        torch.gcu.synchronize()
        stats = C._op_statistics()
    finally:
        C._set_op_debug_config("")
    assert_exact(back, x.bfloat16(), "to chain")
    assert nb.is_pinned()
    assert_exact(nb, x, "non-blocking to(cpu)")
    assert stats.get("_copy_from", (0, 0))[0] >= 4, stats
    assert all(v[1] == 0 for v in stats.values()), stats


def test_non_blocking_h2d_does_not_reuse_a_block_in_flight():
    """Pinned sources freed right after a non-blocking H2D copy: the block is
    held back until the copy has run (an event recorded at free time), so the
    next allocation cannot overwrite data the stream has not read yet."""
    a = torch.randn(2048, 2048, dtype=torch.bfloat16, device="gcu")
    for _ in range(4):
        a = a @ a * 0.01  # keep the stream busy while the copies are queued
    n = 8 << 20
    outs = []
    for i in range(6):
        h = torch.full((n,), float(i), pin_memory=True)
        outs.append(h.to("gcu", non_blocking=True))
        del h
        assert torch.gcu.host_memory_stats()["pending_events"] >= 1
    torch.gcu.synchronize()
    for i, o in enumerate(outs):
        assert float(o.min()) == float(i) and float(o.max()) == float(i), i
    # after the copies have run the block is reused
    hits = torch.gcu.host_memory_stats()["num_cache_hits"]
    h = torch.empty(n, pin_memory=True)
    assert torch.gcu.host_memory_stats()["num_cache_hits"] == hits + 1
    assert torch.gcu.host_memory_stats()["pending_events"] == 0
    del h


def test_copies_under_graph_capture():
    """A non-blocking H2D copy from pinned memory is recorded into a graph and
    reads the host buffer at every replay; a pageable one is refused."""
    hbuf = torch.zeros(4096, pin_memory=True)
    d = torch.empty(4096, device="gcu")
    gr = torch.gcu.GCUGraph()
    torch.gcu.synchronize()
    with torch.gcu.graph(gr):
        d.copy_(hbuf, non_blocking=True)
        out = d * 2
    for v in (1.0, 5.0, -3.0):
        hbuf.fill_(v)
        gr.replay()
        torch.gcu.synchronize()
        assert float(out.min()) == 2 * v and float(out.max()) == 2 * v, v
    gr.reset()
    gr2 = torch.gcu.GCUGraph()
    with pytest.raises(RuntimeError, match="pinned host memory"):
        with torch.gcu.graph(gr2):
            d.copy_(torch.zeros(4096))
    torch.gcu.synchronize()


# ---- cat ------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.int64, torch.bool])
def test_cat_matches_cpu(dtype):
    cases = [
        ([(8, 32, 100, 128), (8, 32, 1, 128)], 2),   # append one position to a KV cache
        ([(4096, 64), (4096, 64)], -1),              # rotate-half
        ([(3, 5), (2, 5), (0, 5)], 0),
        ([(2, 3, 4)], 1),
    ]
    for shapes, dim in cases:
        xs = [rand(s, dtype, 10 + i) for i, s in enumerate(shapes)]
        got = torch.cat([x.to("gcu") for x in xs], dim)
        assert got.device.type == "gcu" and got.dtype == dtype
        assert_exact(got.cpu(), aten.cat(xs, dim), f"cat {shapes}")


def test_cat_rules_and_out_variant():
    """ATen's cat rules hold on the device: the legacy 1-D empty input is
    skipped, dtypes promote, out= is resized, checked for a castable dtype and
    for overlap, channels-last inputs give a channels-last result, and errors
    carry CPU ATen's messages; nothing falls back to CPU."""
    x = rand((4, 3), torch.float32, 20)
    i = rand((2, 3), torch.int32, 21)
    b = rand((4, 3), torch.bfloat16, 22)
    C._set_op_debug_config("op_statistics=true")
    C._clear_op_statistics()
    try:
        got = torch.cat([x.to("gcu"), torch.empty(0, device="gcu"), i.to("gcu")])
        mixed = torch.cat([b.to("gcu"), x.to("gcu")], 1)
        out = torch.empty(0, dtype=torch.float64, device="gcu")
        torch.cat([x.to("gcu"), i.to("gcu")], 0, out=out)
        cl = rand((2, 3, 4, 5), torch.bfloat16, 23).contiguous(memory_format=torch.channels_last)
        cl2 = rand((2, 2, 4, 5), torch.bfloat16, 24).contiguous(memory_format=torch.channels_last)
        got_cl = torch.cat([cl.to("gcu"), cl2.to("gcu")], 1)
        stats = C._op_statistics()
    finally:
        C._set_op_debug_config("")
    assert_exact(got.cpu(), aten.cat([x, torch.empty(0), i], 0), "skip + promote")
    assert_exact(mixed.cpu(), aten.cat([b, x], 1), "bf16 + f32")
    assert out.shape == (6, 3) and out.dtype == torch.float64
    assert_exact(out.cpu(), aten.cat([x, i], 0).double(), "out=")
    assert got_cl.is_contiguous(memory_format=torch.channels_last)
    assert_exact(got_cl.cpu(), aten.cat([cl, cl2], 1), "channels-last")
    assert stats.get("cat", (0, 0))[0] >= 3 and stats.get("cat.out", (0, 0))[0] >= 1, stats
    assert all(v[1] == 0 for v in stats.values()), stats
    # errors: the same checks (ATen's structured meta function) as on the CPU
    for args, kw in [(([x, rand((4, 2), torch.float32, 25)], 0), {}),
                     (([x, x[0]], 0), {}),
                     (([x, i], 0), {"out": torch.empty(0, dtype=torch.int32)})]:
        with pytest.raises((RuntimeError, TypeError)) as cpu_err:
            torch.cat(*args, **kw)
        dargs = ([t.to("gcu") for t in args[0]], args[1])
        dkw = {k: v.to("gcu") for k, v in kw.items()}
        with pytest.raises((RuntimeError, TypeError)) as dev_err:
            torch.cat(*dargs, **dkw)
        assert type(cpu_err.value) is type(dev_err.value)
        assert str(cpu_err.value).split("\n")[0] == str(dev_err.value).split("\n")[0]
    # out aliasing an input
    buf = torch.zeros(8, 3, device="gcu")
    with pytest.raises(RuntimeError, match="memory location"):
        torch.cat([buf[:4], buf[4:]], 0, out=buf)


def test_stack_and_split_cat_run_natively():
    """torch.stack (a cat of unsqueezed views) and re-joining torch.chunk
    pieces reach the native cat; results equal CPU ATen's."""
    xs = [rand((7, 33), torch.bfloat16, 60 + i) for i in range(5)]
    C._set_op_debug_config("op_statistics=true")
    C._clear_op_statistics()
    try:
        st = torch.stack([x.to("gcu") for x in xs], 1)
        big = rand((12, 40), torch.float32, 70).to("gcu")
        rejoined = torch.cat(torch.chunk(big, 3, 1)[::-1], 1)
        stats = C._op_statistics()
    finally:
        C._set_op_debug_config("")
    assert_exact(st.cpu(), torch.stack(xs, 1), "stack")
    assert_exact(rejoined.cpu(), torch.cat(torch.chunk(big.cpu(), 3, 1)[::-1], 1), "chunk + cat")
    assert stats.get("cat", (0, 0))[0] >= 2 and stats.get("cat", (0, 0))[1] == 0, stats


def test_dataloader_pin_memory_batches_come_from_the_host_allocator():
    """DataLoader(pin_memory=True) pins its batches through the gcu host
    allocator (the current accelerator is gcu); the batches reach the device
    with non-blocking copies and equal their sources."""
    data = torch.randn(64, 8, generator=g(80))
    labels = torch.arange(64)
    dl = torch.utils.data.DataLoader(torch.utils.data.TensorDataset(data, labels), batch_size=16,
                                     pin_memory=True, num_workers=0)
    before = torch.gcu.host_memory_stats()["num_host_alloc"] + torch.gcu.host_memory_stats()["num_cache_hits"]
    outs = []
    for xb, yb in dl:
        assert xb.is_pinned() and yb.is_pinned()
        outs.append((xb.to("gcu", non_blocking=True), yb.to("gcu", non_blocking=True)))
    torch.gcu.synchronize()
    after = torch.gcu.host_memory_stats()["num_host_alloc"] + torch.gcu.host_memory_stats()["num_cache_hits"]
    assert after - before >= 8  # two pinned tensors per batch
    assert torch.equal(torch.cat([x.cpu() for x, _ in outs]), data)
    assert torch.equal(torch.cat([y.cpu() for _, y in outs]), labels)
