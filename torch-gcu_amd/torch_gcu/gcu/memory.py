"""Caching-allocator statistics and controls of the gcu device (the
reference's torch_gcu/gcu/memory.py:54-914 surface)."""
from __future__ import annotations

from typing import Any

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
