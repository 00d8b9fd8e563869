"""The GCUGraph Python surface beyond capture / replay (the reference's
torch_gcu/gcu/graphs.py:28-34, :128-150, :226-516): is_current_stream_capturing,
register_generator_state and make_graphed_callables, whose graphed forward
and backward passes must reproduce eager execution bit for bit."""
import copy

import pytest
import torch
import torch.nn.functional as F

import torch_gcu  # noqa: F401
from oracle import aten
from oracle.tolerance import assert_close, assert_exact

pytestmark = pytest.mark.gpu


def g(seed):
    return torch.Generator().manual_seed(seed)


class SwiGLU(torch.nn.Module):
    """linear -> SiLU-mul -> linear, as the decoder layer's FFN."""

    def __init__(self, hidden=256, ffn=512, seed=0):
        super().__init__()
        gen = g(seed)
        self.w_gate = torch.nn.Parameter((torch.randn(ffn, hidden, generator=gen) * 0.05).bfloat16())
        self.w_up = torch.nn.Parameter((torch.randn(ffn, hidden, generator=gen) * 0.05).bfloat16())
        self.w_down = torch.nn.Parameter((torch.randn(hidden, ffn, generator=gen) * 0.05).bfloat16())

    def forward(self, x):
        return F.linear(F.silu(F.linear(x, self.w_gate)) * F.linear(x, self.w_up), self.w_down)


def test_is_current_stream_capturing():
    x = torch.randn(64, generator=g(1)).to("gcu")
    assert torch.gcu.is_current_stream_capturing() is False
    seen = []
    graph = torch.gcu.GCUGraph()
    with torch.gcu.graph(graph):
        seen.append(torch.gcu.is_current_stream_capturing())
        y = x * 2
    seen.append(torch.gcu.is_current_stream_capturing())
    assert seen == [True, False]
    graph.replay()
    torch.gcu.synchronize()
    assert_exact(y.cpu(), x.cpu() * 2, "replay")
    graph.reset()


def test_silu_native_parity():
    """silu / silu_ / silu.out (the op the SwiGLU module's backward pairs with
    silu_backward) on the gfx950 kernel against CPU ATen."""
    for dt, kind in [(torch.bfloat16, "bf16"), (torch.float16, "bf16"), (torch.float32, "fp32")]:
        x = (torch.randn(1000, 333, generator=g(2)) * 4).to(dt)
        torch_gcu._C._set_op_debug_config("op_statistics=true")
        torch_gcu._C._clear_op_statistics()
        try:
            y = F.silu(x.to("gcu"))
            z = x.to("gcu")
            F.silu(z, inplace=True)
            o = torch.empty(1000, 333, dtype=dt, device="gcu")
            torch.ops.aten.silu.out(x.to("gcu").t().contiguous().t(), out=o)  # strided input
            stats = torch_gcu._C._op_statistics()
        finally:
            torch_gcu._C._set_op_debug_config("")
        ref = F.silu(x.float()).to(dt) if dt != torch.float32 else F.silu(x)
        for name, got in (("silu", y), ("silu_", z), ("silu.out", o)):
            assert_close(got.cpu(), ref, kind, f"{name} {dt}")
        for op in ("silu", "silu_", "silu.out"):
            assert stats.get(op, (0, 0)) == (1, 0), (op, stats)


def _eager_step(module, x, gy):
    out = module(x)
    out.backward(gy)
    return out.detach().clone(), x.grad.clone(), [p.grad.clone() for p in module.parameters()]


def test_make_graphed_callables_module_forward_and_backward_bit_exact():
    torch.manual_seed(0)
    eager = SwiGLU(seed=3).to("gcu")
    graphed = copy.deepcopy(eager)
    xs = [(torch.randn(128, 256, generator=g(10 + i)) * 0.5).bfloat16().to("gcu") for i in range(3)]
    gys = [(torch.randn(128, 256, generator=g(20 + i)) * 0.1).bfloat16().to("gcu") for i in range(3)]
    sample = xs[0].clone().requires_grad_()
    graphed = torch.gcu.make_graphed_callables(graphed, (sample,))
    for i in range(3):
        xe = xs[i].clone().requires_grad_()
        xg = xs[i].clone().requires_grad_()
        for p in eager.parameters():
            p.grad = None
        for p in graphed.parameters():
            p.grad = None
        oe, gxe, gpe = _eager_step(eager, xe, gys[i])
        og, gxg, gpg = _eager_step(graphed, xg, gys[i])
        torch.gcu.synchronize()
        assert_exact(og.cpu(), oe.cpu(), f"call {i}: output")
        assert_exact(gxg.cpu(), gxe.cpu(), f"call {i}: input grad")
        for k, (a, b) in enumerate(zip(gpg, gpe)):
            assert_exact(a.cpu(), b.cpu(), f"call {i}: parameter {k} grad")
    # and the eager pass itself against CPU ATen (bf16 chain bar on the output)
    cpu = copy.deepcopy(eager).to("cpu")
    assert_close(oe.cpu(), cpu(xs[2].cpu()).detach(), "bf16", "eager gcu vs CPU ATen")
    # eval mode runs the module's original forward
    graphed.eval()
    with torch.no_grad():
        assert_exact(graphed(xs[1]).cpu(), eager(xs[1]).cpu(), "eval mode, eager forward")


def test_make_graphed_callables_two_functions_share_a_pool():
    w1 = (torch.randn(256, 256, generator=g(30)) * 0.05).bfloat16().to("gcu").requires_grad_()
    w2 = (torch.randn(256, 256, generator=g(31)) * 0.05).bfloat16().to("gcu").requires_grad_()

    def f1(x, w):
        return F.silu(x @ w)

    def f2(h, w):
        return (h @ w) * 2.0

    x0 = (torch.randn(64, 256, generator=g(32))).bfloat16().to("gcu").requires_grad_()
    h0 = f1(x0, w1).detach().requires_grad_()
    gf1, gf2 = torch.gcu.make_graphed_callables((f1, f2), ((x0, w1), (h0, w2)))
    x = (torch.randn(64, 256, generator=g(33))).bfloat16().to("gcu")
    gy = (torch.randn(64, 256, generator=g(34)) * 0.1).bfloat16().to("gcu")

    def run(fa, fb):
        xi = x.clone().requires_grad_()
        a, b = w1.detach().clone().requires_grad_(), w2.detach().clone().requires_grad_()
        out = fb(fa(xi, a), b)
        out.backward(gy)
        return out.detach(), xi.grad, a.grad, b.grad

    got = run(gf1, gf2)
    want = run(f1, f2)
    torch.gcu.synchronize()
    for name, a, b in zip(("out", "dx", "dw1", "dw2"), got, want):
        assert_exact(a.cpu(), b.cpu(), f"chained graphs: {name}")


def test_register_generator_state():
    gen = torch.Generator(device="gcu")
    gen.manual_seed(123)
    graph = torch.gcu.GCUGraph()
    graph.register_generator_state(gen)
    graph.register_generator_state(gen)  # registering twice keeps one entry
    with pytest.raises(ValueError):
        graph.register_generator_state(torch.Generator())
    x = torch.randn(16, generator=g(40)).to("gcu")
    before = gen.get_offset()
    with torch.gcu.graph(graph):
        y = x + 1
    with pytest.raises(RuntimeError, match="before capture_begin"):
        graph.register_generator_state(torch.Generator(device="gcu"))
    # nothing in the graph draws random numbers: replays leave the offset alone
    for _ in range(3):
        graph.replay()
    torch.gcu.synchronize()
    assert gen.get_offset() == before
    assert_exact(y.cpu(), x.cpu() + 1, "replay")
    graph.reset()
    # an advance made during capture is undone at capture_end and applied per replay
    g2 = torch.gcu.GCUGraph()
    g2.register_generator_state(gen)
    start = gen.get_offset()
    with torch.gcu.graph(g2):
        z = x * 3
        gen.set_offset(gen.get_offset() + 8)  # stands in for a captured Philox draw of 8
    assert gen.get_offset() == start
    g2.replay()
    g2.replay()
    torch.gcu.synchronize()
    assert gen.get_offset() == start + 16
    assert_exact(z.cpu(), x.cpu() * 3, "replay")
    g2.reset()
