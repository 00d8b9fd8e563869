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
