"""Op-debug helpers of the gcu device (the reference's torch_gcu/gcu/debug.py:
73-170): scoped switches for op-name logging, forced CPU fallback and op
check, and the op statistics.

The process-wide switches come from ENFLAME_PT_OP_DEBUG_CONFIG (see
``torch_gcu._C._set_op_debug_config`` for changing them at run time); the
scopes here act on every native op called while they are entered.
"""
from __future__ import annotations

from typing import Callable, Optional

from .. import _C

__all__ = [
    "OpDebugCtx", "get_pre_func", "get_post_func", "get_op_statistics_info",
    "dump_op_statistics_info", "clear_op_statistics_info",
]


class OpDebugCtx:
    """Within the block: log each native op's names (enable_dump_op_name),
    run every native op on CPU ATen (enable_fallback_cpu), or check every
    native op against CPU ATen (enable_op_check)."""

    def __init__(self, enable_dump_op_name: bool = True, enable_fallback_cpu: bool = False,
                 enable_op_check: bool = False):
        self.enable_dump_op_name = enable_dump_op_name
        self.enable_fallback_cpu = enable_fallback_cpu
        self.enable_op_check = enable_op_check

    def __enter__(self):
        self.enable_scope()
        return self

    def __exit__(self, exc_type, exc_val, exc_tb):
        self.disable_scope()
        return False

    # also usable as autograd node pre / post hooks (any hook arguments)
    def enable_scope(self, *_):
        if self.enable_dump_op_name:
            _C._enter_dump_op_name_scope()
        if self.enable_fallback_cpu:
            _C._enter_fallback_cpu_scope()
        if self.enable_op_check:
            _C._enter_op_check_scope()

    def disable_scope(self, *_):
        _C._exit_print_cpp_name_scope()
        _C._exit_fallback_cpu_scope()
        _C._exit_op_check_scope()

    @staticmethod
    def current_state() -> dict:
        return {"dump_op_name": _C._get_dump_op_name_scope_state(),
                "fallback_cpu": _C._get_fallback_cpu_scope_state(),
                "op_check": _C._get_op_check_scope_state()}


def get_pre_func(h: Optional[OpDebugCtx] = None) -> Callable:
    """A hook that enters h's scopes, whatever arguments it is called with."""
    return (h if h is not None else OpDebugCtx()).enable_scope


def get_post_func(h: Optional[OpDebugCtx] = None) -> Callable:
    """A hook that leaves the scopes."""
    return (h if h is not None else OpDebugCtx()).disable_scope


def get_op_statistics_info() -> str:
    """The recorded op statistics as a table (op_statistics=true)."""
    return _C._get_op_statistics_info()


def dump_op_statistics_info() -> str:
    """Writes the op statistics as JSON under dump_path; returns the file."""
    return _C._dump_op_statistics_to_json()


def clear_op_statistics_info() -> None:
    _C._clear_statistics()
