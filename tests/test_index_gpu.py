"""The efficient op int32_indices_index (torch.gcu.efficient.gcu_index) on the
GPU: advanced indexing with int32 index tensors read as int32 by one native
gather (mi_index), compared bit for bit with CPU ATen's aten::index on the
same indices widened to int64, over the patterns the reference's make_info
handles (torch_gcu/csrc/efficient_ops/ops.cpp:221-342): one index, N-D
indices, several broadcast indices, indexed dims in the middle or not
adjacent, 0-dim indices, strided self, host-side indices; its error cases;
and capture in a GCUGraph (no CPU fallback on the path)."""
import pytest
import torch

import torch_gcu
from oracle import aten
from oracle.tolerance import assert_exact

pytestmark = pytest.mark.gpu

C = torch_gcu._C
gcu_index = torch.gcu.efficient.gcu_index


def g(seed):
    return torch.Generator().manual_seed(seed)


def ri(lo, hi, shape, seed):
    return torch.randint(lo, hi, shape, generator=g(seed), dtype=torch.int32)


def table(shape, dtype, seed):
    if dtype == torch.int64:
        return torch.randint(-2**63, 2**63 - 1, shape, generator=g(seed), dtype=torch.int64)
    return torch.randn(shape, generator=g(seed)).to(dtype)


PATTERNS = {
    "rows": ((70, 33), lambda: [ri(-70, 70, (41,), 1)]),
    "2-D index": ((60, 12, 5), lambda: [ri(0, 60, (7, 9), 2)]),
    "middle dim": ((6, 80, 16), lambda: [None, ri(-80, 80, (25,), 3)]),
    "two broadcast": ((50, 60, 8), lambda: [ri(0, 50, (9, 1), 4), ri(0, 60, (13,), 5)]),
    "non-adjacent": ((20, 3, 30, 8), lambda: [ri(0, 20, (4, 5), 6), None, ri(-30, 30, (5,), 7)]),
    "0-dim index": ((40, 24), lambda: [torch.tensor(17, dtype=torch.int32)]),
    "last dim": ((4, 6, 90), lambda: [None, None, ri(0, 90, (31,), 8)]),
    "three indices": ((9, 10, 11), lambda: [ri(0, 9, (6,), 9), ri(0, 10, (6,), 10),
                                            ri(-11, 11, (6,), 11)]),
}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.int64, torch.uint8])
@pytest.mark.parametrize("name", sorted(PATTERNS))
def test_gcu_index_patterns_bit_exact(name, dtype):
    shape, mk = PATTERNS[name]
    x = table(shape, dtype, 100)
    idx = mk()
    want = aten.int32_indices_index(x, idx)
    got = gcu_index(x.to("gcu"), [None if i is None else i.to("gcu") for i in idx])
    assert_exact(got.cpu(), want, f"{name} {dtype}")


def test_gcu_index_embedding_rows_config5_shape():
    """The config-5 embedding as an int32 gather: bf16 [32000, 4096] rows by
    16384 token ids (8 KiB rows, 16-byte words, a wave per row)."""
    w = table((32000, 4096), torch.bfloat16, 200)
    ids = ri(0, 32000, (8, 2048), 201)
    got = gcu_index(w.to("gcu"), [ids.to("gcu")])
    assert got.shape == (8, 2048, 4096)
    assert_exact(got.cpu(), aten.int32_indices_index(w, [ids]), "embedding gather")


def test_gcu_index_strided_self_and_host_indices():
    x = table((16, 24, 10), torch.float32, 300)
    xt = x.to("gcu").permute(2, 0, 1)  # [10, 16, 24], no dim contiguous in order
    idx = [ri(0, 10, (5,), 301), None, ri(-24, 24, (5,), 302)]
    got = gcu_index(xt, [None if i is None else i.to("gcu") for i in idx])
    assert_exact(got.cpu(), aten.int32_indices_index(x.permute(2, 0, 1), idx), "permuted self")
    sl = x.to("gcu")[::2, 3:, ::3]  # sliced, misaligned rows: 4-byte words
    idx2 = [ri(0, 8, (6,), 303)]
    assert_exact(gcu_index(sl, [idx2[0].to("gcu")]).cpu(),
                 aten.int32_indices_index(x[::2, 3:, ::3], idx2), "sliced self")
    # indices on the host are range-checked there and copied to the device
    assert_exact(gcu_index(x.to("gcu"), [idx2[0]]).cpu(),
                 aten.int32_indices_index(x, idx2), "host indices")
    with pytest.raises(IndexError, match="out of bounds"):
        gcu_index(x.to("gcu"), [torch.tensor([3, 16], dtype=torch.int32)])


def test_gcu_index_empty_and_out_of_range_device_index():
    x = table((12, 7), torch.float32, 400)
    e = gcu_index(x.to("gcu"), [torch.empty(0, dtype=torch.int32, device="gcu")])
    assert e.shape == (0, 7)
    z = table((0, 7), torch.float32, 401)
    assert gcu_index(z.to("gcu"), [torch.empty(0, 3, dtype=torch.int32, device="gcu")]).shape == (0, 3, 7)
    # a device index out of range is not range-checked on the host (that
    # would synchronise): its row is written as zeros, nothing outside self
    # is read, and the kernel's record raises CPU ATen's IndexError at the
    # next synchronisation (here the copy to the host), once
    idx = torch.tensor([2, 40, -1, -13], dtype=torch.int32)
    with pytest.raises(IndexError, match="out of bounds for dimension with size 12"):
        gcu_index(x.to("gcu"), [idx.to("gcu")]).cpu()
    with pytest.raises(IndexError):
        aten.int32_indices_index(x, [idx])
    got = gcu_index(x.to("gcu"), [idx.to("gcu")])
    with pytest.raises(IndexError, match="reported at the next synchronization"):
        torch.gcu.synchronize()
    torch.gcu.synchronize()  # cleared: no second error
    got = got.cpu()
    assert_exact(got[0], x[2], "in range")
    assert_exact(got[2], x[-1], "negative index")
    assert bool((got[1] == 0).all()) and bool((got[3] == 0).all())


def test_index_select_out_of_range_device_index_raises_at_sync():
    """index_select through the dispatcher with a device index past the
    table: CPU ATen raises IndexError at the call; on gcu the gather writes
    zeros and the error is raised at the next synchronisation (the value
    read by .item() here)."""
    x = table((64, 8), torch.int64, 402)
    bad = torch.tensor([3, 64, 5])
    with pytest.raises(IndexError):
        torch.index_select(x, 0, bad)
    y = torch.index_select(x.to("gcu"), 0, bad.to("gcu"))
    with pytest.raises(IndexError, match="index 64 is out of bounds for dimension with size 64"):
        y[0, 0].item()
    assert_exact(y.cpu()[0], x[3], "row before the bad one")
    assert bool((y.cpu()[1] == 0).all())
    # op_sync_mode reports it at the op that read it
    torch_gcu._C._set_op_debug_config("op_sync_mode=true")
    try:
        with pytest.raises(IndexError, match="out of bounds"):
            torch.index_select(x.to("gcu"), 0, bad.to("gcu"))
    finally:
        torch_gcu._C._set_op_debug_config("")
    torch.gcu.synchronize()


def test_gcu_index_errors_follow_the_reference():
    x = torch.randn(5, 6).to("gcu")
    with pytest.raises(IndexError, match="should be int"):
        gcu_index(x, [torch.tensor([1, 2], device="gcu")])  # int64 indices
    with pytest.raises(IndexError, match="should be int"):
        gcu_index(x, [torch.tensor([True, False, True, False, False], device="gcu")])  # a mask
    with pytest.raises(IndexError, match="broadcast"):
        gcu_index(x, [ri(0, 5, (3,), 1).to("gcu"), ri(0, 6, (4,), 2).to("gcu")])
    with pytest.raises(IndexError, match="too many indices"):
        gcu_index(x, [ri(0, 5, (3,), 1).to("gcu")] * 3)
    with pytest.raises(IndexError, match="long, int, byte or bool"):
        gcu_index(x, [torch.tensor([1.0], device="gcu")])


def test_gcu_index_is_native_and_capturable():
    x = table((300, 64), torch.bfloat16, 500).to("gcu")
    ids = ri(0, 300, (4, 50), 501).to("gcu")
    C._set_op_debug_config("op_statistics=true")
    C._clear_op_statistics()
    try:
        eager = gcu_index(x, [ids, ri(0, 64, (50,), 502).to("gcu")])
        stats = C._op_statistics()
    finally:
        C._set_op_debug_config("")
    assert all(v[1] == 0 for v in stats.values()), stats  # nothing fell back to CPU
    idx2 = ri(0, 64, (50,), 502).to("gcu")
    graph = torch.gcu.GCUGraph()
    torch.gcu.synchronize()
    with torch.gcu.graph(graph):
        out = gcu_index(x, [ids, idx2])
    for k in range(3):
        graph.replay()
        torch.gcu.synchronize()
        assert_exact(out.cpu(), eager.cpu(), f"replay {k}")
    ids.copy_(ri(0, 300, (4, 50), 503).to("gcu"))
    graph.replay()
    torch.gcu.synchronize()
    assert_exact(out.cpu(), gcu_index(x, [ids, idx2]).cpu(), "replay with new ids")
    graph.reset()
