"""Caching-allocator bookkeeping on host memory (CPU only).

torch_gcu._C can serve the allocator's segments from host memory with
events that complete at once; these tests drive the C++ allocator through
that mode in a fresh process and check the invariants of the reference's
allocator (torch_gcu/csrc/gcu/gcu_caching_allocator.cpp): size rounding and
segment sizes, best-fit reuse per stream, splitting and merging, deferred
frees after recordStream, private graph pools, empty_cache, the memory
fraction cap with its OutOfMemoryError, and stat equalities.
"""
import os
import subprocess
import sys
import textwrap

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PRELUDE = textwrap.dedent(
    """
    import sys
    sys.path.insert(0, %r)
    import torch, torch_gcu
    C = torch_gcu._C
    C._allocator_use_host_memory(1 << 30)
    S1, S2 = 0x1000, 0x2000   # two fake stream handles
    MiB = 1 << 20
    def st():
        return C._memory_stats(0)
    """ % os.path.join(REPO, "torch-gcu_amd"))


def run(body: str) -> str:
    code = PRELUDE + textwrap.dedent(body)
    p = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stdout + p.stderr
    return p.stdout


def test_rounding_segments_and_stats():
    run("""
    a = C._allocator_alloc(0, 1, S1)          # rounds to 512 B in a 2 MiB small segment
    s = st()
    assert s["allocated_bytes.all.current"] == 512
    assert s["reserved_bytes.all.current"] == 2 * MiB
    assert s["segment.small_pool.current"] == 1
    b = C._allocator_alloc(0, 3 * MiB, S1)     # 1-10 MiB -> 20 MiB large segment
    assert st()["reserved_bytes.large_pool.current"] == 20 * MiB
    c = C._allocator_alloc(0, 33 * MiB + 5, S1)  # >= 10 MiB -> rounded up to 2 MiB multiple
    assert st()["reserved_bytes.large_pool.current"] == 20 * MiB + 34 * MiB
    for p in (a, b, c):
        C._allocator_free(p)
    s = st()
    assert s["allocated_bytes.all.current"] == 0
    assert s["allocation.all.current"] == 0
    # the 1 MiB tail of c's 34 MiB segment is too small to split off, so the
    # block keeps it; the 3 MiB block was split from its 20 MiB segment
    assert s["allocated_bytes.all.peak"] == 512 + 3 * MiB + 34 * MiB
    assert s["requested_bytes.all.peak"] == 1 + 3 * MiB + 33 * MiB + 5
    C._empty_cache()
    assert st()["reserved_bytes.all.current"] == 0
    assert st()["num_device_free"] == 3
    """)


def test_reuse_is_per_stream_and_best_fit():
    run("""
    a = C._allocator_alloc(0, 4096, S1)
    C._allocator_free(a)
    b = C._allocator_alloc(0, 4096, S1)
    assert b == a                      # same stream: cached block reused
    c = C._allocator_alloc(0, 4096, S2)
    assert c != b                      # other stream: never handed a block in flight on S1
    x = C._allocator_alloc(0, 12 * MiB, S1)
    y = C._allocator_alloc(0, 16 * MiB, S1)
    C._allocator_free(x); C._allocator_free(y)
    z = C._allocator_alloc(0, 11 * MiB, S1)
    assert z == x                      # best fit: the 12 MiB block, not the 16 MiB one
    """)


def test_split_and_merge():
    run("""
    a = C._allocator_alloc(0, 1000, S1)
    b = C._allocator_alloc(0, 1000, S1)
    assert b == a + 1024               # carved from the same 2 MiB segment
    s = st()
    assert s["inactive_split.small_pool.current"] == 1
    C._allocator_free(a); C._allocator_free(b)
    s = st()
    assert s["inactive_split.all.current"] == 0   # merged back into one segment
    assert s["inactive_split_bytes.all.current"] == 0
    C._empty_cache()
    assert st()["segment.all.current"] == 0
    """)


def test_record_stream_defers_free():
    run("""
    a = C._allocator_alloc(0, 8192, S1)
    C._allocator_record_stream(a, S2)
    C._allocator_free(a)
    s = st()
    assert s["allocated_bytes.all.current"] == 0
    assert s["active_bytes.all.current"] == 8192   # still in use by S2 until its event completes
    b = C._allocator_alloc(0, 8192, S1)           # polls events; the fake event has completed
    assert b == a
    """)


def test_graph_private_pool():
    run("""
    pool = C._allocator_new_pool()
    C._allocator_begin_pool(0, pool[0], pool[1], S2)
    g = C._allocator_alloc(0, 4096, S2)       # capturing stream -> private pool
    n = C._allocator_alloc(0, 4096, S1)       # other stream -> shared pool
    C._allocator_end_pool(0, pool[0], pool[1])
    snap = C._memory_snapshot()
    owners = {s["segment_pool_id"] for s in snap}
    assert tuple(pool) in owners and (0, 0) in owners
    C._allocator_free(g)
    h = C._allocator_alloc(0, 4096, S2)       # capture over: S2 uses the shared pool now
    assert h != g
    C._allocator_release_pool(0, pool[0], pool[1])   # pool freed once unused
    snap = C._memory_snapshot()
    assert tuple(pool) not in {s["segment_pool_id"] for s in snap}
    C._allocator_free(n); C._allocator_free(h)
    """)


def test_memory_fraction_and_oom():
    out = run("""
    C._set_memory_fraction(0.05, 0)      # 51 MiB of the fake 1 GiB
    a = C._allocator_alloc(0, 40 * MiB, S1)
    try:
        C._allocator_alloc(0, 40 * MiB, S1)
        print("no error")
    except torch.OutOfMemoryError as e:
        print("OOM:", str(e).splitlines()[0])
    s = st()
    assert s["num_ooms"] == 1 and s["num_alloc_retries"] == 1
    C._allocator_free(a)
    b = C._allocator_alloc(0, 40 * MiB, S1)   # fits again after the free
    """)
    assert "OOM: GCU out of memory. Tried to allocate 40" in out


def test_alloc_conf_parsing():
    run("""
    d = C._parse_alloc_conf("max_split_size_mb:128,garbage_collection_threshold:0.6,roundup_power2_divisions:4")
    assert d["max_split_size"] == 128 * MiB
    assert abs(d["garbage_collection_threshold"] - 0.6) < 1e-12
    assert d["roundup_power2_divisions"] == 4
    for bad in ["max_split_size_mb:10", "roundup_power2_divisions:3", "nope:1", "backend:topsMallocAsync"]:
        try:
            C._parse_alloc_conf(bad)
            raise SystemExit("accepted " + bad)
        except RuntimeError:
            pass
    """)


def test_pinned_host_allocator_bookkeeping():
    """The caching host allocator (torch_gcu/csrc/gcu/gcu_caching_host_allocator.cpp)
    on ordinary host memory: pin_memory() / pin_memory=True come from it and
    read back as pinned, freed blocks are reused by size class, a cached block
    is taken only by a request of at most its class and no less than half of
    it, slices of a block are pinned, and empty_cache releases what is cached."""
    run("""
    C._host_allocator_use_plain_memory()
    hs = C._host_memory_stats
    a = torch.empty(1000, pin_memory=True)          # 4000 B -> 4 KiB class
    assert a.is_pinned() and a[500:].is_pinned()
    assert hs()["num_host_alloc"] == 1 and hs()["reserved_bytes"] == 4096, hs()
    pa = a.data_ptr()
    del a
    b = torch.empty(1024, pin_memory=True)           # same class: reused
    assert b.data_ptr() == pa and hs()["num_cache_hits"] == 1, hs()
    c = torch.empty(3000, pin_memory=True)           # 12000 B -> 16 KiB
    assert hs()["reserved_bytes"] == 4096 + 16384 and hs()["allocated_bytes"] == 4096 + 16384
    x = torch.randn(5, 7)
    y = x.pin_memory()
    assert y.is_pinned() and not x.is_pinned() and torch.equal(x, y)
    assert not torch.randn(3).is_pinned()
    del b, c, y
    assert hs()["allocated_bytes"] == 0, hs()
    # 100 MiB -> 2 MiB multiples above 64 MiB; a 40 MiB request (64 MiB class)
    # may take it, a 20 MiB one (32 MiB class) may not
    big = torch.empty(100 * MiB, dtype=torch.uint8, pin_memory=True)
    pb = big.data_ptr()
    assert hs()["reserved_bytes"] == 4096 + 16384 + 4096 + 100 * MiB, hs()
    del big
    s1 = torch.empty(20 * MiB, dtype=torch.uint8, pin_memory=True)
    assert s1.data_ptr() != pb
    s2 = torch.empty(40 * MiB, dtype=torch.uint8, pin_memory=True)
    assert s2.data_ptr() == pb
    del s1, s2
    torch.gcu.host_empty_cache()
    st = torch.gcu.host_memory_stats()
    assert st["reserved_bytes"] == 0 and st["num_blocks"] == 0, st
    assert st["num_host_free"] == st["num_host_alloc"], st
    print("ok")
    """)


# ---- history, snapshots, checkpoints and the rest of the allocator interface ----

def test_base_allocation_and_cache_info():
    """getBaseAllocation of a block split from a segment is the segment's
    start and size (gcu_caching_allocator.cpp:861-880); cacheInfo reports the
    largest free cached block (:936-950)."""
    run("""
    a = C._allocator_alloc(0, 3 * MiB, S1)      # 20 MiB segment, split
    b = C._allocator_alloc(0, 5 * MiB, S1)      # the next piece of it
    assert b == a + 3 * MiB
    assert C._get_base_allocation(b) == (a, 20 * MiB)
    assert C._get_base_allocation(a) == (a, 20 * MiB)
    try:
        C._get_base_allocation(a + 512)
        raise SystemExit("an interior pointer was accepted")
    except RuntimeError:
        pass
    # free cached: the 12 MiB tail of the segment; a start of 0 is replaced
    # by the device's free memory, so ask from a start of 1 byte
    assert C._cache_info_from(0, 1) == 12 * MiB
    C._allocator_free(a)                         # 3 MiB free, not merged (b is live)
    assert C._cache_info_from(0, 1) == 12 * MiB
    C._allocator_free(b)                         # all merged: one 20 MiB free block
    assert C._cache_info_from(0, 1) == 20 * MiB
    assert C._cache_info(0) >= 20 * MiB          # starts from the fake device's free bytes
    """)


def test_check_pool_live_allocations():
    """checkPoolLiveAllocations (:547-566) on a graph pool: true exactly when
    the expected set equals the pool's allocated blocks."""
    run("""
    pool = C._allocator_new_pool()
    C._allocator_begin_pool(0, pool[0], pool[1], S2)
    x = C._allocator_alloc(0, 4096, S2)
    y = C._allocator_alloc(0, 2 * MiB, S2)
    C._allocator_end_pool(0, pool[0], pool[1])
    z = C._allocator_alloc(0, 4096, S1)          # default pool, never counted
    assert C._check_pool_live_allocations(0, pool, {x, y})
    assert not C._check_pool_live_allocations(0, pool, {x})         # y is live too
    assert not C._check_pool_live_allocations(0, pool, {x, y, z})   # z is not in the pool
    C._allocator_free(x)
    assert C._check_pool_live_allocations(0, pool, {y})
    assert not C._check_pool_live_allocations(0, pool, {x, y})
    try:
        C._check_pool_live_allocations(0, (9, 9), set())
        raise SystemExit("an unknown pool was accepted")
    except RuntimeError:
        pass
    """)


def test_checkpoint_restore_reproduces_pool_layout_and_stats():
    """getCheckpointState / setCheckpointPoolState (:1007-1222): after the
    checkpoint the pool's blocks change (frees, new allocations, a new
    split); restoring frees what the pool holds now and re-creates the
    checkpointed blocks at the same addresses, with the same allocated set
    and the same statistics."""
    run("""
    pool = C._allocator_new_pool()
    C._allocator_begin_pool(0, pool[0], pool[1], S2)
    a = C._allocator_alloc(0, 1000, S2)
    b = C._allocator_alloc(0, 3000, S2)
    c = C._allocator_alloc(0, 5000, S2)
    big = C._allocator_alloc(0, 12 * MiB, S2)
    C._allocator_free(b)                      # a hole between a and c
    ck = C._get_checkpoint_state(0, pool)
    layout = [list(seg) for seg in ck.segments]
    assert ck.pool_id == tuple(pool) and len(layout) == 2, layout
    def pool_layout():
        return [[(bl["address"], bl["size"], bl["state"] == "active_allocated")
                 for bl in s["blocks"]] for s in sorted(C._memory_snapshot(), key=lambda s: s["address"])
                if tuple(s["segment_pool_id"]) == tuple(pool)]
    assert pool_layout() == [[tuple(b) for b in seg] for seg in layout]
    keys = ["allocated_bytes.all.current", "allocation.all.current", "active_bytes.all.current",
            "inactive_split.all.current", "inactive_split_bytes.all.current",
            "reserved_bytes.all.current", "segment.all.current"]
    before = {k: st()[k] for k in keys}
    # change the pool: free a and big, allocate new blocks with other sizes
    C._allocator_free(a); C._allocator_free(big)
    d = C._allocator_alloc(0, 7000, S2)
    e = C._allocator_alloc(0, 2 * MiB + 512, S2)
    assert pool_layout() != [[tuple(b) for b in seg] for seg in layout]
    try:
        C._set_checkpoint_pool_state(0, ck)   # storage form: d and e would go stale unnamed
        raise SystemExit("the restore did not ask for the stale storages")
    except RuntimeError as err:
        assert "stale" in str(err)
    assert pool_layout() != [[tuple(b) for b in seg] for seg in layout]   # nothing changed
    freed, allocd = C._set_checkpoint_pool_state_raw(0, ck)
    assert sorted(freed) == sorted([c, d, e]), (freed, [c, d, e])
    assert sorted(allocd) == sorted([a, c, big])
    assert pool_layout() == [[tuple(b) for b in seg] for seg in layout]
    assert {k: st()[k] for k in keys} == before
    # the restored blocks are ordinary live allocations again
    assert C._check_pool_live_allocations(0, pool, {a, c, big})
    C._allocator_end_pool(0, pool[0], pool[1])
    for p in (a, c, big):
        C._allocator_free(p)
    assert st()["allocated_bytes.all.current"] == 0
    """)


def test_memory_history_records_events_with_stacks():
    """_record_memory_history (:531-546, memory.py:635-690): alloc,
    free_requested, free_completed, segment_alloc, segment_free and snapshot
    events with their addresses and sizes, Python frames of the calls, a
    ring of max_entries, and nothing after recording stops."""
    run('''
    import torch_gcu.gcu.memory as M
    def make_block():
        return C._allocator_alloc(0, 3 * MiB, S1)
    M._record_memory_history("all", context="all", stacks="python")
    assert C._is_history_enabled()
    a = make_block()
    C._allocator_free(a)
    C._empty_cache()
    snap = M._snapshot()
    tr = snap["device_traces"][0]
    acts = [e["action"] for e in tr]
    assert acts == ["segment_alloc", "alloc", "free_requested", "free_completed",
                    "segment_free", "snapshot"], acts
    seg_alloc, alloc = tr[0], tr[1]
    assert alloc["addr"] == a and alloc["size"] == 3 * MiB and alloc["stream"] == S1
    assert seg_alloc["addr"] == a and seg_alloc["size"] == 20 * MiB
    assert tr[4]["addr"] == a and tr[4]["size"] == 20 * MiB
    names = [f["name"] for f in alloc["frames"]]
    assert "make_block" in names, alloc["frames"]
    assert all(e["time_us"] >= tr[0]["time_us"] for e in tr)
    # live blocks carry the stack that allocated them
    b = make_block()
    snap = M._snapshot()
    blk = [bl for s in snap["segments"] for bl in s["blocks"] if bl["address"] == b][0]
    assert blk["state"] == "active_allocated" and blk["requested_size"] == 3 * MiB
    assert "make_block" in [f["name"] for f in blk["frames"]]
    assert set(snap["allocator_settings"]) >= {"max_split_size", "expandable_segments"}
    C._allocator_free(b)
    # a ring of 4 entries keeps the last 4 events
    M._record_memory_history("all", max_entries=4)
    for _ in range(3):
        C._allocator_free(make_block())
    tr = M._snapshot()["device_traces"][0]
    assert len(tr) == 4 and tr[-1]["action"] == "snapshot", [e["action"] for e in tr]
    # context=None: events but no stacks (stopping first drops the history)
    M._record_memory_history(None)
    M._record_memory_history("all", context=None)
    C._allocator_free(make_block())
    tr = M._snapshot()["device_traces"][0]
    assert tr and all(e["frames"] == [] for e in tr)
    M._record_memory_history(None)
    assert not C._is_history_enabled()
    C._allocator_free(make_block())
    assert M._snapshot()["device_traces"][0] == []
    # the legacy boolean form
    M._record_memory_history(True, trace_alloc_max_entries=100, trace_alloc_record_context=True)
    C._allocator_free(make_block())
    assert [e["action"] for e in M._snapshot()["device_traces"][0]][:2] == ["alloc", "free_requested"]
    M._record_memory_history(False)
    for bad in [dict(enabled="x"), dict(context="x"), dict(stacks="x")]:
        try:
            M._record_memory_history(**{**dict(enabled="all"), **bad})
            raise SystemExit("accepted " + repr(bad))
        except RuntimeError:
            pass
    ''')


def test_dump_snapshot_pickle_and_summary(tmp_path):
    out = run(f'''
    import pickle
    import torch_gcu.gcu.memory as M
    M._record_memory_history("all")
    a = C._allocator_alloc(0, 4096, S1)
    M._dump_snapshot({str(tmp_path / "snap.pickle")!r})
    with open({str(tmp_path / "snap.pickle")!r}, "rb") as f:
        s = pickle.load(f)
    assert [e["action"] for e in s["device_traces"][0]] == ["segment_alloc", "alloc", "snapshot"]
    assert s["segments"][0]["blocks"][0]["address"] == a
    nested = M.memory_stats_as_nested_dict(0)
    assert nested["allocated_bytes"]["all"]["current"] == 4096
    assert nested["segment"]["small_pool"]["current"] == 1
    assert nested["num_device_alloc"] == 1
    text = M.memory_summary(0)
    assert "Allocated memory" in text and "from small pool" in text
    row = [l for l in text.splitlines() if l.startswith("| Allocations")][0]
    assert row.split("|")[2].strip() == "1", row
    assert "from small pool" not in M.memory_summary(0, abbreviated=True)
    print("ok")
    ''')
    assert "ok" in out


def test_mem_pool_routes_one_threads_allocations():
    """use_mem_pool (memory.py:914-934): inside the block the calling
    thread's allocations come from the pool's own segments; another thread's
    do not; after the block the pool's memory returns once it is freed."""
    run("""
    import threading
    import torch_gcu.gcu.memory as M
    pool = M.MemPool()
    other = []
    with M.use_mem_pool(pool, device=0):
        assert pool.use_count() == 1
        a = C._caching_allocator_alloc(0, 4096, S1)
        t = threading.Thread(target=lambda: other.append(C._caching_allocator_alloc(0, 4096, S1)))
        t.start(); t.join()
    assert pool.use_count() == 0
    owner = {bl["address"]: tuple(s["segment_pool_id"]) for s in C._memory_snapshot()
             for bl in s["blocks"]}
    assert owner[a] == pool.id and owner[other[0]] == (0, 0), (owner, pool.id)
    assert [s["address"] for s in pool.snapshot()] == [a]
    b = C._caching_allocator_alloc(0, 4096, S1)       # outside the block: default pool
    assert b != a and {tuple(s["segment_pool_id"]) for s in C._memory_snapshot()
                       if s["address"] <= b < s["address"] + s["total_size"]} == {(0, 0)}
    C._caching_allocator_delete(a)                     # the released pool's segment goes back
    assert pool.snapshot() == []
    C._caching_allocator_delete(b); C._caching_allocator_delete(other[0])
    """)
