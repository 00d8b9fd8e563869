"""The caching allocator's memory history, snapshots, raw allocation, memory
pools and graph-pool checkpoints on the GPU (the reference's
torch_gcu/gcu/memory.py:54-100, :635-785, :856-934 and
gcu_caching_allocator.cpp:531-566, :861-950, :1007-1222)."""
import pickle

import pytest
import torch

import torch_gcu  # noqa: F401
from oracle.tolerance import assert_close

pytestmark = pytest.mark.gpu

C = torch_gcu._C
M = torch.gcu.memory


def g(seed):
    return torch.Generator().manual_seed(seed)


def _trace():
    return M._snapshot()["device_traces"][0]


def _capture_step(x):
    """The captured work: two elementwise ops (one intermediate, one output)."""
    return torch.log_softmax(x * 2.0 + 1.0, -1)


def test_memory_history_across_graph_capture(tmp_path):
    """History recorded across a GCUGraph capture: the capture's segment
    comes from the graph's private pool, the output's alloc event names
    this test's frames, and the snapshot read back from _dump_snapshot
    matches; replays allocate nothing."""
    x = torch.randn(256, 4096, generator=g(1)).to("gcu")
    torch.gcu.synchronize()
    M._record_memory_history("all", context="all", stacks="python")
    try:
        graph = torch.gcu.GCUGraph()
        with torch.gcu.graph(graph):
            out = _capture_step(x)
        n_before = len(_trace())
        for _ in range(3):
            graph.replay()
        torch.gcu.synchronize()
        path = tmp_path / "snap.pickle"
        M._dump_snapshot(str(path))
        with open(path, "rb") as f:
            snap = pickle.load(f)
    finally:
        M._record_memory_history(None)
    assert_close(out.cpu(), torch.log_softmax(x.cpu() * 2.0 + 1.0, -1), "fp32", "replay output")
    pool = tuple(graph.pool())
    pool_segs = [s for s in snap["segments"] if tuple(s["segment_pool_id"]) == pool]
    assert pool_segs, [s["segment_pool_id"] for s in snap["segments"]]
    trace = snap["device_traces"][0]
    # every capture-time allocation landed in a segment of the graph's pool
    allocs = [e for e in trace if e["action"] == "alloc"]
    in_pool = [e for e in allocs if any(s["address"] <= e["addr"] < s["address"] + s["total_size"]
                                         for s in pool_segs)]
    out_alloc = [e for e in in_pool if e["addr"] == out.data_ptr()]
    assert out_alloc, (out.data_ptr(), allocs)
    names = [f["name"] for f in out_alloc[-1]["frames"]]
    assert "_capture_step" in names and "test_memory_history_across_graph_capture" in names, names
    # the intermediate x * 2.0 + 1.0 was freed inside the capture
    assert any(e["action"] == "free_requested" and e["addr"] != out.data_ptr() for e in trace)
    assert any(e["action"] == "segment_alloc" and e["addr"] == pool_segs[0]["address"] for e in trace)
    # the live output's block carries its stack in the segment list
    blk = [b for s in pool_segs for b in s["blocks"] if b["address"] == out.data_ptr()]
    assert blk and blk[0]["state"] == "active_allocated" and blk[0]["frames"]
    # replays allocate nothing: only the dump's own snapshot event was added
    assert [e["action"] for e in trace[n_before:]] == ["snapshot"], trace[n_before:]
    graph.reset()


def test_caching_allocator_alloc_and_delete():
    torch.gcu.synchronize()
    before = torch.gcu.memory_allocated()
    p = torch.gcu.caching_allocator_alloc(3 << 20)
    assert torch.gcu.memory_allocated() == before + (3 << 20)
    base, size = C._get_base_allocation(p)
    assert base <= p < base + size and size >= 3 << 20
    # an explicit stream argument (torch.gcu.Stream or a raw handle)
    s = torch.gcu.current_stream()
    q = torch.gcu.caching_allocator_alloc(4096, stream=s)
    assert q != p
    torch.gcu.caching_allocator_delete(q)
    torch.gcu.caching_allocator_delete(p)
    assert torch.gcu.memory_allocated() == before
    with pytest.raises(TypeError):
        torch.gcu.caching_allocator_alloc(16, stream="nope")


def test_use_mem_pool_routes_gcu_tensors():
    pool = torch.gcu.MemPool()
    with torch.gcu.use_mem_pool(pool):
        t = torch.empty(1 << 20, device="gcu")
        t.fill_(3.0)
    u = torch.empty(1 << 20, device="gcu")
    segs = pool.snapshot()
    assert len(segs) == 1 and segs[0]["address"] <= t.data_ptr() < segs[0]["address"] + segs[0]["total_size"]
    assert not (segs[0]["address"] <= u.data_ptr() < segs[0]["address"] + segs[0]["total_size"])
    assert float(t.sum()) == 3.0 * (1 << 20)
    del t
    torch.gcu.synchronize()
    assert pool.snapshot() == []  # the released pool's segment went back when t died
    del u


def test_checkpoint_restore_with_storages():
    """A graph pool checkpointed after one capture; a second capture into the
    same pool adds an output; restoring the checkpoint frees that output's
    block, its storage loses the allocator's deleter (passed as stale), and
    the pool's live set is the first capture's output again."""
    x = torch.randn(512, 1024, generator=g(2)).to("gcu")
    pool = torch.gcu.graph_pool_handle()
    g1, g2 = torch.gcu.GCUGraph(), torch.gcu.GCUGraph()
    torch.gcu.synchronize()
    with torch.gcu.graph(g1, pool=pool):
        out1 = _capture_step(x)
    pid = tuple(g1.pool())
    layout0 = [[b for b in seg] for seg in C._get_checkpoint_state(0, pid).segments]
    ck = C._get_checkpoint_state(0, pid)
    assert C._check_pool_live_allocations(0, pid, {out1.data_ptr()})
    with torch.gcu.graph(g2, pool=pool):
        out2 = out1 * 3.0
    assert C._check_pool_live_allocations(0, pid, {out1.data_ptr(), out2.data_ptr()})
    st2 = C._storage_ptr(out2)
    assert C._has_standard_deleter(st2)
    with pytest.raises(RuntimeError, match="stale"):
        C._set_checkpoint_pool_state(0, ck)
    freed, allocd = C._set_checkpoint_pool_state(0, ck, [st2])
    assert out2.data_ptr() in freed and out1.data_ptr() in allocd
    assert not C._has_standard_deleter(st2)
    assert C._check_pool_live_allocations(0, pid, {out1.data_ptr()})
    now = [[b for b in seg] for seg in C._get_checkpoint_state(0, pid).segments]
    heads0 = {seg[0][0] for seg in layout0}
    assert [seg for seg in now if seg[0][0] in heads0] == layout0
    # a segment the second capture added (if any) is left entirely free
    assert all(not b[2] for seg in now if seg[0][0] not in heads0 for b in seg)
    g1.replay()
    torch.gcu.synchronize()
    assert_close(out1.cpu(), torch.log_softmax(x.cpu() * 2.0 + 1.0, -1), "fp32",
                 "replay after restore")
    del out2  # no deleter any more: the block is not freed twice
    g2.reset()
    g1.reset()
    del out1
    torch.gcu.synchronize()
