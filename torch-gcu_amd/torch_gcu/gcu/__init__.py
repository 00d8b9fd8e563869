"""``torch.gcu``: device, stream, event, memory, RNG and graph APIs of the gcu
device (the reference's torch_gcu/gcu/__init__.py:160-216,673-733,
memory.py:54-914, graphs.py:50-224, random.py:23-173)."""
from __future__ import annotations

import contextlib
import os
from typing import Any, Optional, Union

import torch

from .. import _C
from .graphs import (  # noqa: F401
    GCUGraph, graph, graph_pool_handle, is_current_stream_capturing, make_graphed_callables,
)
from .memory import (  # noqa: F401
    MemPool, caching_allocator_alloc, caching_allocator_delete, empty_cache,
    get_allocator_backend, get_per_process_memory_fraction, host_empty_cache, host_memory_stats,
    max_memory_allocated, max_memory_cached, max_memory_reserved, mem_get_info,
    memory_allocated, memory_cached, memory_reserved, memory_snapshot, memory_stats,
    memory_stats_as_nested_dict, memory_summary, reset_accumulated_memory_stats,
    reset_max_memory_allocated, reset_max_memory_cached, reset_peak_memory_stats,
    set_per_process_memory_fraction, use_mem_pool,
)
from . import memory  # noqa: F401

_DeviceLike = Union[torch.device, str, int, None]


def _index(device: _DeviceLike) -> int:
    if device is None:
        return current_device()
    if isinstance(device, int):
        return device
    if isinstance(device, str):
        device = torch.device(device)
    if device.type != "gcu":
        raise ValueError(f"expected a gcu device, got {device}")
    return current_device() if device.index is None else device.index


def is_available() -> bool:
    return _C._device_count() > 0


def is_initialized() -> bool:
    return bool(_C._is_initialized())


def _lazy_init() -> None:
    _C._init()


def init() -> None:
    _C._init()


def device_count() -> int:
    return _C._device_count()


def current_device() -> int:
    return _C._current_device()


def set_device(device: _DeviceLike) -> None:
    d = _index(device)
    if d >= 0:
        _C._set_device(d)


class device:
    """Context manager that changes the current gcu device."""

    def __init__(self, device: _DeviceLike):
        self.idx = -1 if device is None else _index(device)
        self.prev = -1

    def __enter__(self):
        self.prev = current_device()
        if self.idx >= 0 and self.idx != self.prev:
            _C._set_device(self.idx)

    def __exit__(self, *args):
        if self.idx >= 0 and self.idx != self.prev:
            _C._set_device(self.prev)
        return False


def synchronize(device: _DeviceLike = None) -> None:
    _C._synchronize(_index(device))


def get_device_properties(device: _DeviceLike = None) -> dict:
    return _C._device_properties(_index(device))


def get_device_name(device: _DeviceLike = None) -> str:
    return get_device_properties(device)["name"]


# ---- streams and events -------------------------------------------------------------

class Stream(torch.Stream):
    """A gcu stream (default priority only).  ``Stream()`` creates a new HIP
    stream on the current device."""

    def __new__(cls, device: _DeviceLike = None, priority: int = 0, **kwargs):
        if kwargs:
            return super().__new__(cls, **kwargs)
        return super().__new__(cls, device=torch.device("gcu", _index(device)), priority=priority)

    @property
    def gcu_stream(self) -> int:
        """The raw hipStream_t handle."""
        return _C._stream_handle(self.stream_id, self.device_index)


class Event(torch.Event):
    def __new__(cls, enable_timing: bool = False, blocking: bool = False, interprocess: bool = False):
        return super().__new__(cls, device="gcu", enable_timing=enable_timing, blocking=blocking,
                               interprocess=interprocess)


def _stream_from(t) -> Stream:
    sid, dev, dtype = t
    return Stream(stream_id=sid, device_index=dev, device_type=dtype)


def current_stream(device: _DeviceLike = None) -> Stream:
    return _stream_from(_C._current_stream(_index(device)))


def default_stream(device: _DeviceLike = None) -> Stream:
    return _stream_from(_C._default_stream(_index(device)))


def set_stream(stream: torch.Stream) -> None:
    if stream is None:
        return
    _C._set_current_stream(stream.stream_id, stream.device_index)


def ExternalStream(stream_ptr: int, device: _DeviceLike = None) -> Stream:
    return _stream_from(_C._wrap_external_stream(stream_ptr, _index(device)))


@contextlib.contextmanager
def stream(s: Optional[torch.Stream]):
    """Makes ``s`` the current stream of its device inside the block."""
    if s is None:
        yield
        return
    prev = current_stream(s.device_index)
    with device(s.device_index):
        set_stream(s)
        try:
            yield
        finally:
            set_stream(prev)


# ---- random state (bookkeeping only; random ops run on the CPU) ----------------

_GENS: dict = {}


def _gens(idx: int):
    g = _GENS.get(idx)
    if g is None:
        g = torch.Generator(device=f"gcu:{idx}")
        _GENS[idx] = g
    return g


def manual_seed(seed: int) -> None:
    _gens(current_device()).manual_seed(int(seed))


def manual_seed_all(seed: int) -> None:
    for i in range(device_count()):
        _gens(i).manual_seed(int(seed))


def seed() -> int:
    return _gens(current_device()).seed()


def initial_seed() -> int:
    return _gens(current_device()).initial_seed()


def get_rng_state(device: _DeviceLike = None) -> torch.Tensor:
    return _gens(_index(device)).get_state()


def set_rng_state(new_state: torch.Tensor, device: _DeviceLike = None) -> None:
    _gens(_index(device)).set_state(new_state)


def get_rng_state_all() -> list:
    return [get_rng_state(i) for i in range(device_count())]


def set_rng_state_all(new_states) -> None:
    for i, st in enumerate(new_states):
        set_rng_state(st, i)


_BAD_FORK = False


def _after_fork_in_child() -> None:
    global _BAD_FORK
    _BAD_FORK = is_initialized()  # the HIP runtime does not survive a fork


def _is_in_bad_fork() -> bool:
    """True in a child forked after the device was initialised (torch.manual_seed
    then leaves the gcu generators alone, as it does for CUDA)."""
    return _BAD_FORK


if hasattr(os, "register_at_fork"):
    os.register_at_fork(after_in_child=_after_fork_in_child)


from . import debug, efficient  # noqa: E402,F401
