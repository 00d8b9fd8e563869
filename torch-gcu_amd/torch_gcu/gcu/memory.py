"""Caching-allocator statistics and controls of the gcu device (the
reference's torch_gcu/gcu/memory.py:54-914 surface): statistics, raw
allocation, memory history and snapshots, memory pools."""
from __future__ import annotations

import contextlib
import pickle
import sys
import threading
from typing import Any, Optional

import torch

from .. import _C


def _idx(device) -> int:
    from . import _index
    return _index(device)


def memory_stats(device=None) -> dict[str, Any]:
    """Flat dict of allocator counters, keyed as torch.cuda.memory_stats."""
    return dict(sorted(_C._memory_stats(_idx(device)).items()))


def memory_allocated(device=None) -> int:
    return memory_stats(device)["allocated_bytes.all.current"]


def max_memory_allocated(device=None) -> int:
    return memory_stats(device)["allocated_bytes.all.peak"]


def memory_reserved(device=None) -> int:
    return memory_stats(device)["reserved_bytes.all.current"]


def max_memory_reserved(device=None) -> int:
    return memory_stats(device)["reserved_bytes.all.peak"]


def reset_peak_memory_stats(device=None) -> None:
    _C._reset_peak_memory_stats(_idx(device))


def reset_max_memory_allocated(device=None) -> None:
    reset_peak_memory_stats(device)


def reset_accumulated_memory_stats(device=None) -> None:
    _C._reset_accumulated_memory_stats(_idx(device))


def empty_cache() -> None:
    """Returns every unused cached segment to the device (hipFree)."""
    _C._empty_cache()


def host_memory_stats() -> dict[str, int]:
    """Counters of the caching allocator of pinned host memory (pin_memory(),
    torch.empty(..., pin_memory=True) and non-blocking copy staging)."""
    return dict(sorted(_C._host_memory_stats().items()))


def host_empty_cache() -> None:
    """Unpins (hipHostFree) every cached pinned block that no copy still uses."""
    _C._host_empty_cache()


def set_per_process_memory_fraction(fraction: float, device=None) -> None:
    if not isinstance(fraction, float):
        raise TypeError("Invalid type for fraction argument, must be `float`")
    if fraction < 0 or fraction > 1:
        raise ValueError(f"Invalid fraction value: {fraction}. Allowed range: 0~1")
    _C._set_memory_fraction(fraction, _idx(device))


def get_per_process_memory_fraction(device=None) -> float:
    return _C._get_memory_fraction(_idx(device))


def mem_get_info(device=None) -> tuple[int, int]:
    """(free, total) bytes of the device."""
    return tuple(_C._mem_get_info(_idx(device)))


def memory_snapshot() -> list[dict]:
    return _C._memory_snapshot()


def memory_cached(device=None) -> int:
    """Deprecated name of memory_reserved."""
    return memory_reserved(device)


def max_memory_cached(device=None) -> int:
    """Deprecated name of max_memory_reserved."""
    return max_memory_reserved(device)


def reset_max_memory_cached(device=None) -> None:
    reset_peak_memory_stats(device)


def memory_stats_as_nested_dict(device=None) -> dict[str, Any]:
    """The counters of memory_stats() nested by their dotted key parts
    ("allocated_bytes.all.current" -> result["allocated_bytes"]["all"]["current"])."""
    out: dict[str, Any] = {}
    for key, value in _C._memory_stats(_idx(device)).items():
        node = out
        parts = key.split(".")
        for p in parts[:-1]:
            node = node.setdefault(p, {})
        node[parts[-1]] = value
    return out


# ---- raw allocation (interoperability with other frameworks) ------------------

def caching_allocator_alloc(size: int, device=None, stream=None) -> int:
    """Allocates `size` bytes from the gcu caching allocator on `device` for
    `stream` (a torch.gcu.Stream or a raw hipStream_t handle; the current
    stream when None) and returns the device address.  Free it with
    caching_allocator_delete."""
    from . import Stream, current_stream

    d = _idx(device)
    if stream is None:
        stream = current_stream(d)
    if isinstance(stream, Stream):
        stream = stream.gcu_stream
    if not isinstance(stream, int):
        raise TypeError("Invalid type for stream argument, must be `torch.gcu.Stream` or `int` "
                        "representing a pointer to a existing stream")
    return _C._caching_allocator_alloc(d, int(size), stream)


def caching_allocator_delete(mem_ptr: int) -> None:
    """Returns memory from caching_allocator_alloc to the allocator (its device
    and stream are tracked by the allocator)."""
    _C._caching_allocator_delete(int(mem_ptr))


# ---- summary ---------------------------------------------------------------------

def _fmt_size(n: int) -> str:
    for unit in ("B  ", "KiB", "MiB", "GiB", "TiB"):
        if abs(n) < 1024 or unit == "TiB":
            return f"{n:6d} {unit}" if unit == "B  " else f"{n:6.2f} {unit}"
        n /= 1024.0
    return str(n)


def _fmt_count(n: int) -> str:
    return f"{n:10d}"


def memory_summary(device=None, abbreviated: bool = False) -> str:
    """A table of the allocator's counters for `device`: current, peak,
    allocated and freed totals of memory and of allocations, by pool (all,
    large, small; the per-pool rows are left out when `abbreviated`)."""
    st = _C._memory_stats(_idx(device))
    rows = [
        ("Allocated memory", "allocated_bytes", _fmt_size),
        ("Active memory", "active_bytes", _fmt_size),
        ("Requested memory", "requested_bytes", _fmt_size),
        ("GPU reserved memory", "reserved_bytes", _fmt_size),
        ("Non-releasable memory", "inactive_split_bytes", _fmt_size),
        ("Allocations", "allocation", _fmt_count),
        ("Active allocs", "active", _fmt_count),
        ("GPU reserved segments", "segment", _fmt_count),
        ("Non-releasable allocs", "inactive_split", _fmt_count),
    ]
    pools = [("all", "")] + ([] if abbreviated else
                              [("large_pool", "from large pool"), ("small_pool", "from small pool")])
    width = 92
    line = "|" + "=" * (width - 2) + "|"
    sep = "|" + "-" * (width - 2) + "|"
    out = [line,
           "|{:^{w}}|".format(f"PyTorch GCU memory summary, device ID {_idx(device)}", w=width - 2),
           sep,
           "|{:^{w}}|".format(f"GCU OOMs: {st['num_ooms']:<12d}|  hipMalloc retries: "
                              f"{st['num_alloc_retries']:<10d}", w=width - 2),
           line,
           "| {:<26}| {:>13} | {:>13} | {:>13} | {:>13} |".format(
               "Metric", "Cur Usage", "Peak Usage", "Tot Alloc", "Tot Freed"),
           sep]
    for title, key, fmt in rows:
        for pool, label in pools:
            name = title if pool == "all" else "      " + label
            vals = [st[f"{key}.{pool}.{f}"] for f in ("current", "peak", "allocated", "freed")]
            out.append("| {:<26}| {:>13} | {:>13} | {:>13} | {:>13} |".format(
                name, *[fmt(v) for v in vals]))
        out.append(sep)
    out.append("| {:<26}| {:>13} | {:>13} | {:>13} | {:>13} |".format(
        "hipMalloc / hipFree calls", _fmt_count(st["num_device_alloc"]),
        "", "", _fmt_count(st["num_device_free"])))
    out.append(line)
    return "\n".join(out) + "\n"


# ---- memory history and snapshots ------------------------------------------------

def _record_memory_history(enabled="all", *args, **kwargs):
    """Records allocator events and the stacks that caused them.

    enabled: None (stop and drop the history), "state" (stacks of live
    memory only) or "all" (also a history of every alloc / free / segment
    event).  context: None, "state", "alloc" (also stacks of alloc events)
    or "all" (also of frees).  stacks: "python" or "all" (plus C++ frames).
    max_entries: size of the history ring.  A bool `enabled` takes the
    legacy arguments (record_context, trace_alloc_max_entries,
    trace_alloc_record_context, device, record_context_cpp)."""
    if isinstance(enabled, bool):
        return _record_memory_history_legacy(enabled, *args, **kwargs)
    return _record_memory_history_impl(enabled, *args, **kwargs)


def _record_memory_history_impl(enabled: Optional[str] = "all", context: Optional[str] = "all",
                                stacks: str = "all", max_entries: int = sys.maxsize,
                                device=None):
    _C._record_memory_history(enabled, context, stacks, max_entries)


def _record_memory_history_legacy(enabled: bool, record_context=True, trace_alloc_max_entries=1,
                                  trace_alloc_record_context=False, device=None,
                                  record_context_cpp=False):
    _C._record_memory_history_legacy(enabled, record_context, record_context_cpp,
                                     trace_alloc_max_entries, trace_alloc_record_context)


def _snapshot(device=None) -> dict:
    """The allocator's state: {"segments": [...], "device_traces": [[...]],
    "allocator_settings": {...}} in the layout of torch.cuda.memory._snapshot()
    (segments with their blocks and the stacks that allocated them; one
    history list per device, oldest event first)."""
    return _C._memory_snapshot_full()


def _dump_snapshot(filename: str = "dump_snapshot.pickle") -> None:
    """Writes _snapshot() to `filename` as a pickle (the format the PyTorch
    memory viewer reads)."""
    s = _snapshot()
    with open(filename, "wb") as f:
        pickle.dump(s, f)


def _set_allocator_settings(env: str) -> None:
    raise RuntimeError("the gcu allocator reads PYTORCH_GCU_ALLOC_CONF once, at its first use")


def get_allocator_backend() -> str:
    """"native": the stream-ordered caching allocator over hipMalloc."""
    return "native"


# ---- memory pools -----------------------------------------------------------------

class MemPool:
    """An isolated pool of the caching allocator (torch.cuda.MemPool's
    counterpart): allocations made under use_mem_pool(pool) come from segments
    that only this pool uses.  `allocator` and `use_on_oom` are accepted for
    compatibility; only the built-in allocator exists."""

    def __init__(self, allocator=None, use_on_oom: bool = False):
        self._id = tuple(_C._graph_pool_handle())
        self._allocator = allocator
        self._use_on_oom = use_on_oom
        self._use_count = 0
        self._lock = threading.Lock()

    @property
    def id(self) -> tuple:
        return self._id

    @property
    def allocator(self):
        return self._allocator

    def use_count(self) -> int:
        return self._use_count

    def snapshot(self) -> list:
        """memory_snapshot() restricted to this pool's segments."""
        return [s for s in memory_snapshot() if tuple(s["segment_pool_id"]) == self._id]


@contextlib.contextmanager
def use_mem_pool(pool: MemPool, device=None):
    """Routes the current thread's allocations on `device` to `pool` inside the
    block.  On exit the pool stops receiving allocations; its memory returns
    to the device cache once the tensors allocated from it are freed."""
    d = _idx(device)
    with pool._lock:
        pool._use_count += 1
    _C._begin_allocate_current_thread_to_pool(d, pool.id)
    try:
        yield
    finally:
        _C._end_allocate_to_pool(d, pool.id)
        _C._release_pool(d, pool.id)
        with pool._lock:
            pool._use_count -= 1
