"""GCUGraph: capture a sequence of gcu ops once, replay it with one launch
(the reference's torch_gcu/gcu/graphs.py:28-516 over
torch_gcu/csrc/gcu/gcu_graph.cpp, here on hipGraph), plus
make_graphed_callables for forward and backward passes."""
from __future__ import annotations

import gc
from typing import Optional

import torch
from torch.utils._pytree import tree_flatten, tree_unflatten

from .. import _C


def is_current_stream_capturing() -> bool:
    """True while a graph capture is under way on the current gcu stream
    (False, without initialising the device, before the device is used)."""
    return bool(_C._is_current_stream_capturing())


def graph_pool_handle():
    """An id that lets several graphs share one private memory pool."""
    return _C._graph_pool_handle()


class GCUGraph:
    """Wrapper of one captured hipGraph executable.

    Random-number generators of the device are kept consistent with eager
    execution: the current device's default generator and every generator
    given to register_generator_state() have their Philox offset recorded at
    capture_begin; what the captured work advanced it by is undone at
    capture_end (nothing ran yet) and applied again at every replay, as if
    the captured ops had run eagerly."""

    def __init__(self):
        self._g = _C._GCUGraph()
        self._generators: list = []
        self._gen_start: list = []
        self._gen_step: list = []
        self._capturing = False

    def register_generator_state(self, generator: torch.Generator) -> None:
        """Adds a (non-default) gcu generator whose state this graph keeps in
        step with its replays; call it before capture_begin."""
        if not isinstance(generator, torch.Generator) or generator.device.type != "gcu":
            raise ValueError("register_generator_state expects a torch.Generator on a gcu device")
        if self._capturing or self._gen_step:
            raise RuntimeError("register_generator_state must be called before capture_begin")
        if not any(g is generator for g in self._generators):
            self._generators.append(generator)

    def _tracked_generators(self) -> list:
        from . import _gens, current_device

        default = _gens(current_device())
        gens = [default] if not any(g is default for g in self._generators) else []
        return gens + list(self._generators)

    def capture_begin(self, pool=None, capture_error_mode: str = "global"):
        self._gen_start = [(g, g.get_offset()) for g in self._tracked_generators()]
        self._g.capture_begin(tuple(pool) if pool is not None else (),
                              capture_error_mode=capture_error_mode)
        self._capturing = True

    def capture_end(self):
        try:
            self._g.capture_end()
        finally:
            self._capturing = False
            steps = []
            for g, start in self._gen_start:
                steps.append((g, g.get_offset() - start))
                g.set_offset(start)
            self._gen_step = steps

    def replay(self):
        for g, step in self._gen_step:
            if step:
                g.set_offset(g.get_offset() + step)
        self._g.replay()

    def reset(self):
        self._g.reset()
        self._gen_step = []

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


# ---- make_graphed_callables ----------------------------------------------------------

class _Capture:
    """One callable's captured forward and backward passes and the static
    tensors they read and write."""

    def __init__(self, fn, args):
        self.fn = fn
        flat, _ = tree_flatten(args)
        if not all(isinstance(a, torch.Tensor) for a in flat):
            raise TypeError("make_graphed_callables: sample_args may hold tensors only")
        if isinstance(fn, torch.nn.Module):
            if fn._backward_hooks or fn._forward_hooks or fn._forward_pre_hooks:
                raise RuntimeError("make_graphed_callables: a module must have no hooks when it is "
                                   "graphed (hooks may be added afterwards)")
            if any(b.requires_grad for b in fn.buffers()):
                raise RuntimeError("make_graphed_callables: module buffers must not require grad")
            self.params = tuple(fn.parameters())
        else:
            self.params = ()
        self.args = args
        self.n_user = len(flat)
        # everything the captured passes read: the user's tensors, then the
        # module's parameters
        self.inputs = tuple(flat) + self.params
        self.fwd, self.bwd = GCUGraph(), GCUGraph()
        self.outputs = ()
        self.out_spec = None
        self.grad_outputs = ()
        self.grad_inputs = ()

    def grads_of(self, outputs, grad_outputs, allow_unused):
        need = [o for o in outputs if o.requires_grad]
        wrt = [i for i in self.inputs if i.requires_grad]
        if not need or not wrt:
            return ()
        return torch.autograd.grad(need, wrt, grad_outputs=[g for g in grad_outputs if g is not None],
                                   only_inputs=True, allow_unused=allow_unused)

    def warm_up(self, iters, allow_unused):
        for _ in range(iters):
            outs, _ = tree_flatten(self.fn(*self.args))
            self.grads_of(outs, [torch.empty_like(o) if o.requires_grad else None for o in outs],
                          allow_unused)

    def capture_forward(self, pool):
        with graph(self.fwd, pool=pool):
            out = self.fn(*self.args)
        flat, self.out_spec = tree_flatten(out)
        self.outputs = tuple(flat)

    def capture_backward(self, pool, allow_unused):
        self.grad_outputs = tuple(torch.empty_like(o) if o.requires_grad else None
                                  for o in self.outputs)
        with graph(self.bwd, pool=pool):
            got = self.grads_of(self.outputs, self.grad_outputs, allow_unused)
        it = iter(got)
        # one slot per input, None where the input takes no gradient
        self.grad_inputs = tuple(next(it) if i.requires_grad else None for i in self.inputs)

    def autograd_function(self):
        cap = self

        class Graphed(torch.autograd.Function):
            @staticmethod
            def forward(ctx, *inputs):
                for static, new in zip(cap.inputs[:cap.n_user], inputs[:cap.n_user]):
                    if static.data_ptr() != new.data_ptr():
                        static.copy_(new)
                cap.fwd.replay()
                return tuple(o.detach() for o in cap.outputs)

            @staticmethod
            @torch.autograd.function.once_differentiable
            def backward(ctx, *grads):
                for static, new in zip(cap.grad_outputs, grads):
                    if static is not None and new is not None and static.data_ptr() != new.data_ptr():
                        static.copy_(new)
                cap.bwd.replay()
                return tuple(g.detach() if g is not None else None for g in cap.grad_inputs)

        def run(*user_args):
            flat, _ = tree_flatten(user_args)
            if len(flat) != cap.n_user:
                raise TypeError(f"graphed callable expects {cap.n_user} tensor arguments, "
                                f"got {len(flat)}")
            out = Graphed.apply(*(tuple(flat) + cap.params))
            return tree_unflatten(list(out), cap.out_spec)

        return run


def make_graphed_callables(callables, sample_args, num_warmup_iters: int = 3,
                           allow_unused_input: bool = False):
    """Graphed versions of callables (functions or nn.Modules): each call
    replays the callable's forward pass as one GCUGraph inside a single
    autograd node whose backward replays the captured backward pass (the
    reference's graphs.py:226-516 contract).

    ``callables`` is one callable or a tuple of them, in the order they run;
    ``sample_args`` the matching tuple of argument tensors (a tuple of tuples
    for several callables), whose ``requires_grad`` flags must be those of the
    real inputs.  All captures share one memory pool, forward passes captured
    in order and backward passes in reverse order, as they run in training.
    A graphed module runs its graph only in the training mode it was graphed
    in (its original forward otherwise).  Returned outputs are the graph's
    static outputs: the next call overwrites them."""
    if torch.is_autocast_enabled() and torch.is_autocast_cache_enabled():
        raise RuntimeError("make_graphed_callables needs autocast with cache_enabled=False")
    single = not isinstance(callables, tuple)
    if single:
        callables, sample_args = (callables,), (sample_args,)
    if len(callables) != len(sample_args):
        raise ValueError("make_graphed_callables: one sample_args tuple per callable")
    caps = [_Capture(fn, args) for fn, args in zip(callables, sample_args)]
    pool = graph_pool_handle()

    from . import Stream, stream, synchronize

    # lazy initialisation (workspaces, first-call caches) stays out of the graphs
    synchronize()
    with stream(Stream()):
        for cap in caps:
            cap.warm_up(num_warmup_iters, allow_unused_input)
    synchronize()
    for cap in caps:
        cap.capture_forward(pool)
    for cap in reversed(caps):
        cap.capture_backward(pool, allow_unused_input)

    results = []
    for cap in caps:
        run = cap.autograd_function()
        if isinstance(cap.fn, torch.nn.Module):
            module, mode, eager_forward = cap.fn, cap.fn.training, cap.fn.forward

            def forward(*user_args, _run=run, _module=module, _mode=mode, _eager=eager_forward):
                return _run(*user_args) if _module.training == _mode else _eager(*user_args)

            module.forward = forward
            results.append(module)
        else:
            results.append(run)
    return results[0] if single else tuple(results)
