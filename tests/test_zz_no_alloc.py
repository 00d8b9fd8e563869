"""mi_mean_noalloc: the reduction entry point that allocates nothing.

It runs mi_mean's kernels with their temporary memory in the library's static
per-GPU scratch, so its results must equal mi_mean's bit for bit, on two calls
in a row (the second smaller, so stale scratch contents from the first call
would show), and stay within the fp32 bar of CPU ATen.  While it runs, a
counting workspace allocator is registered: mi_mean calls it, the no-alloc
entry point must not.  A request beyond the scratch's size is refused before
the output is written."""
import ctypes

import pytest
import torch

import torch_gcu  # noqa: F401
from oracle import aten
from oracle.tolerance import assert_close, assert_exact
from torch_gcu import _abi

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


def rn(shape, seed, dtype=torch.float32):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)).to(dtype)


class CountingWorkspace:
    """A workspace allocator on torch's CUDA caching allocator that counts
    the library's requests; restores the gcu allocator on exit."""

    def __init__(self):
        self.allocs = 0
        self.live = {}

        def alloc(nbytes, stream, ctx):
            self.allocs += 1
            t = torch.empty(max(1, nbytes), dtype=torch.uint8, device="cuda")
            self.live[t.data_ptr()] = t
            return t.data_ptr()

        def free(ptr, stream, ctx):
            self.live.pop(ptr, None)

        self._alloc = _abi._ALLOC_FN(alloc)
        self._free = _abi._FREE_FN(free)

    def __enter__(self):
        _abi.check("mi_set_workspace_allocator",
                   _abi.lib().mi_set_workspace_allocator(self._alloc, self._free, None))
        return self

    def __exit__(self, *exc):
        torch.cuda.synchronize()
        torch_gcu._C._register_library_workspace()
        self.live.clear()
        return False


def both(x, dims, keepdim=False, out_shape=None, out_dtype=torch.float32):
    """(mean through mi_mean, through mi_mean_noalloc, allocator requests of each)."""
    shape = out_shape if out_shape is not None else [
        1 if d in [dd % x.dim() for dd in dims] else s for d, s in enumerate(x.shape)
        if keepdim or d not in [dd % x.dim() for dd in dims]]
    ref = torch.full(shape, float("nan"), dtype=out_dtype, device="cuda")
    got = torch.full(shape, float("nan"), dtype=out_dtype, device="cuda")
    with CountingWorkspace() as ws:
        _abi.mean(ref, x, dims, keepdim)
        torch.cuda.synchronize()
        n_ref = ws.allocs
        _abi.mean_noalloc(got, x, dims, keepdim)
        torch.cuda.synchronize()
        n_got = ws.allocs - n_ref
    return ref, got, n_ref, n_got


def test_noalloc_mean_matches_mean_two_calls_second_smaller():
    _abi.install_workspace()
    # config 2's mean over dim 0 of fp32 [16384, 4096]: split-column partials
    # (256 splits x 4096 floats = 4 MiB of scratch)
    x1 = rn((16384, 4096), 1)
    r1, g1, n_ref1, n_got1 = both(x1.cuda(), [0])
    assert n_ref1 > 0, "mi_mean was expected to take workspace for the split partials"
    assert n_got1 == 0, f"mi_mean_noalloc called the workspace allocator {n_got1} times"
    assert_exact(g1, r1, "noalloc mean(0) [16384,4096] vs mi_mean")
    assert_close(g1, aten.mean(x1, 0), "fp32", "noalloc mean(0) vs CPU ATen")
    # a smaller second call: fewer splits and columns reuse the start of the
    # scratch the first call filled
    x2 = rn((3000, 1000), 2)
    r2, g2, _, n_got2 = both(x2.cuda(), [0])
    assert n_got2 == 0
    assert_exact(g2, r2, "noalloc mean(0) [3000,1000] vs mi_mean")
    assert_close(g2, aten.mean(x2, 0), "fp32", "noalloc mean(0) small vs CPU ATen")


def test_noalloc_mean_row_split_and_staging_paths():
    _abi.install_workspace()
    # few long bf16 rows: the row reduction is split over blocks (partials)
    x = rn((4, 1 << 20), 3, torch.bfloat16)
    r, g, _, n = both(x.cuda(), [-1], out_dtype=torch.bfloat16)
    assert n == 0
    assert_exact(g, r, "noalloc row-split mean vs mi_mean")
    assert_close(g, aten.mean(x, -1), "bf16", "noalloc row-split mean vs CPU ATen")
    # reduced dims that are not one dense block (permuted staging copy) and
    # an output that is not dense (staged, then copied)
    y = rn((64, 48, 80), 4)
    yd = y.cuda()
    r, g, _, n = both(yd, [0, 2])
    assert n == 0
    assert_exact(g, r, "noalloc mean over dims (0, 2)")
    assert_close(g, aten.mean(y, [0, 2]), "fp32", "noalloc mean (0, 2) vs CPU ATen")
    out_r = torch.full((96, 64), float("nan"), device="cuda").t()  # non-dense [64, 96]
    out_g = torch.full((96, 64), float("nan"), device="cuda").t()
    z = rn((64, 96, 40), 5)
    with CountingWorkspace() as ws:
        _abi.mean(out_r, z.cuda(), [2])
        n0 = ws.allocs
        _abi.mean_noalloc(out_g, z.cuda(), [2])
        torch.cuda.synchronize()
        assert ws.allocs == n0
    assert_exact(out_g, out_r, "noalloc mean into a transposed out")
    assert_close(out_g, aten.mean(z, 2), "fp32", "noalloc transposed out vs CPU ATen")


def test_noalloc_mean_refuses_more_than_its_scratch():
    _abi.install_workspace()
    # a transposed fp32 [4096, 4096] reduced over dim 0 needs a 64 MiB
    # permuted copy, more than the 16 MiB scratch
    x = rn((4096, 4096), 6).cuda().t()
    out = torch.full((4096,), 7.0, device="cuda")
    arr, n = _abi._dims([0])
    st = _abi.lib().mi_mean_noalloc(_abi.desc(out), _abi.desc(x), arr, n, 0, _abi.stream_of(out))
    torch.cuda.synchronize()
    assert st == 5, _abi.STATUS_NAMES.get(st, st)  # MI_ERR_TOO_LARGE
    msg = _abi.lib().mi_last_error().decode()
    assert "scratch" in msg and str(SCRATCH_BYTES) in msg, msg
    assert bool((out.cpu() == 7.0).all()), "out was written by a refused call"
    # the same request through mi_mean (which may allocate) still works
    ref = torch.empty(4096, device="cuda")
    _abi.mean(ref, x, [0])
    assert_close(ref, aten.mean(x.cpu(), 0), "fp32", "mi_mean transposed")


def _noalloc_on_current_gcu_stream(out, x, dims, keepdim=False):
    arr, n = _abi._dims(dims)
    st = _abi.lib().mi_mean_noalloc(_abi.desc(out), _abi.desc(x), arr, n, int(keepdim),
                                    torch.gcu.current_stream().gcu_stream)
    _abi.check("mi_mean_noalloc", st)


def test_noalloc_mean_captured_in_a_gcu_graph_replays_equal_eager():
    """A GCUGraph capture of mi_mean_noalloc on the capture side stream, on
    config 2's mean over dim 0 (which takes 4 MiB of the scratch): the
    scratch's address is fixed in the graph, so every replay must equal the
    eager mean bit for bit although eager no-alloc calls on other inputs
    overwrite the scratch between replays; no workspace request is made
    during the capture or the replays."""
    _abi.install_workspace()
    x = rn((16384, 4096), 7).to("gcu")
    small = rn((3000, 1000), 8).to("gcu")
    eager = torch.mean(x, 0)  # mi_mean through the gcu dispatcher
    eager_small = torch.mean(small, 0)
    out = torch.full((4096,), float("nan"), device="gcu")
    small_out = torch.empty(1000, device="gcu")
    graph = torch.gcu.GCUGraph()
    torch.gcu.synchronize()
    with CountingWorkspace() as ws:
        with torch.gcu.graph(graph):
            _noalloc_on_current_gcu_stream(out, x, [0])
        for k in range(3):
            graph.replay()
            torch.gcu.synchronize()
            assert_exact(out.cpu(), eager.cpu(), f"no-alloc mean replay {k}")
            # eager work between replays that rewrites the scratch
            _noalloc_on_current_gcu_stream(small_out, small, [0])
            torch.gcu.synchronize()
            assert_exact(small_out.cpu(), eager_small.cpu(), f"eager no-alloc {k}")
            out.fill_(float("nan"))
        assert ws.allocs == 0, f"{ws.allocs} workspace requests"
    x.copy_(rn((16384, 4096), 9).to("gcu"))
    graph.replay()
    torch.gcu.synchronize()
    assert_exact(out.cpu(), torch.mean(x, 0).cpu(), "no-alloc mean replay with new input")
    assert_close(out, aten.mean(rn((16384, 4096), 9), 0), "fp32", "replay vs CPU ATen")
    graph.reset()
