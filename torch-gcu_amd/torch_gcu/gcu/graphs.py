"""GCUGraph: capture a sequence of gcu ops once, replay it with one launch
(the reference's torch_gcu/gcu/graphs.py:50-224 over
torch_gcu/csrc/gcu/gcu_graph.cpp, here on hipGraph)."""
from __future__ import annotations

import gc
from typing import Optional

import torch

from .. import _C


def graph_pool_handle():
    """An id that lets several graphs share one private memory pool."""
    return _C._graph_pool_handle()


class GCUGraph:
    """Wrapper of one captured hipGraph executable."""

    def __init__(self):
        self._g = _C._GCUGraph()

    def capture_begin(self, pool=None, capture_error_mode: str = "global"):
        self._g.capture_begin(tuple(pool) if pool is not None else (),
                              capture_error_mode=capture_error_mode)

    def capture_end(self):
        self._g.capture_end()

    def replay(self):
        self._g.replay()

    def reset(self):
        self._g.reset()

    def pool(self):
        return self._g.pool()

    def enable_debug_mode(self):
        self._g.enable_debug_mode()

    def debug_dump(self, debug_path: str):
        self._g.debug_dump(debug_path)

    def num_nodes(self) -> int:
        return self._g.num_nodes()


class graph:
    """Context manager capturing the ops of its block into ``gcu_graph``.

    As in the reference (graphs.py:206-218): synchronise, empty the cache,
    switch to a side stream and begin capture; on exit end the capture and
    restore the stream."""

    default_capture_stream: Optional[torch.Stream] = None

    def __init__(self, gcu_graph: GCUGraph, pool=None, stream: Optional[torch.Stream] = None,
                 capture_error_mode: str = "global"):
        from . import Stream

        if self.__class__.default_capture_stream is None:
            self.__class__.default_capture_stream = Stream()
        self.pool = () if pool is None else tuple(pool)
        self.capture_stream = stream if stream is not None else self.__class__.default_capture_stream
        self.gcu_graph = gcu_graph
        self.capture_error_mode = capture_error_mode
        self._ctx = None

    def __enter__(self):
        from . import empty_cache, stream, synchronize

        synchronize()
        gc.collect()
        empty_cache()
        self._ctx = stream(self.capture_stream)
        self._ctx.__enter__()
        self.gcu_graph.capture_begin(self.pool or None, capture_error_mode=self.capture_error_mode)

    def __exit__(self, *args):
        try:
            self.gcu_graph.capture_end()
        finally:
            self._ctx.__exit__(None, None, None)
        return False
