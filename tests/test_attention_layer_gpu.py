"""Flash-attention forward and the config-5 decoder layer on the GPU.

Attention is compared with CPU ATen's flash attention (oracle.aten.sdpa, which
like the kernel rounds the softmax weights to bf16 before the P V product);
the decoder layer on gcu is held to the composed-chain bar against the same
layer on CPU ATen (bf16) and in fp32, and its GCUGraph replay must equal its
eager output bit for bit."""
import math

import pytest
import torch
import torch.nn.functional as F

import torch_gcu  # noqa: F401
from oracle import aten
from oracle import numpy_ref as npr
from oracle.tolerance import assert_close, assert_composed_close, assert_exact, bar_ratio
from torch_gcu import _abi
from torch_gcu.utils import decoder_layer as dl

pytestmark = pytest.mark.gpu


def g(seed):
    return torch.Generator().manual_seed(seed)


def rn(shape, seed, dtype=torch.bfloat16):
    return torch.randn(shape, generator=g(seed)).to(dtype)


def ref_attention(q, k, v, causal, scale=None):
    """CPU ATen flash attention (oracle.aten.sdpa): (out, lse)."""
    return aten.sdpa(q, k, v, causal, scale)


@pytest.mark.parametrize("B,H,Hk,Sq,Sk,D,causal", [
    (2, 4, 4, 256, 256, 128, True),
    (1, 2, 2, 200, 200, 64, False),
    (1, 8, 2, 130, 130, 128, True),
    (2, 2, 2, 96, 300, 128, False),
    (1, 1, 1, 1, 77, 128, False),
    (1, 2, 2, 129, 129, 64, True),
    (1, 2, 2, 40, 33, 128, False),   # fewer keys than one tile: only the clamped copy form
    (1, 2, 2, 17, 17, 64, True),
])
def test_flash_attention_parity(B, H, Hk, Sq, Sk, D, causal):
    q, k, v = rn((B, H, Sq, D), 1), rn((B, Hk, Sk, D), 2), rn((B, Hk, Sk, D), 3)
    ref, ref_lse = ref_attention(q, k, v, causal)
    out = torch.empty(B, H, Sq, D, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(B, H, Sq, dtype=torch.float32, device="cuda")
    _abi.flash_attention_fwd(out, lse, q.cuda(), k.cuda(), v.cuda(), causal)
    assert_close(out, ref, "bf16", f"attention {B},{H},{Hk},{Sq},{Sk},{D},{causal}")
    assert (lse.cpu() - ref_lse).abs().max().item() < 2e-2 * max(1.0, ref_lse.abs().max().item())


@pytest.mark.parametrize("scale,ramp,causal", [
    (0.3, False, True), (-0.05, False, True), (-0.05, False, False),
    (None, True, True), (None, True, False), (-0.08, True, False),
])
def test_flash_attention_scale_and_rescale(scale, ramp, causal):
    """Explicit positive and negative scales (the scale is folded into the
    exponent, so the running max is taken over sign-adjusted raw scores), and
    keys whose scores grow along the sequence (ramp), so the row max keeps
    growing and O is rescaled many times."""
    B, H, S, D = 1, 2, 320, 128
    q, k, v = rn((B, H, S, D), 11), rn((B, H, S, D), 12), rn((B, H, S, D), 13)
    if ramp:
        k = (k.float() * torch.linspace(0.2, 3.0, S)[None, None, :, None]).to(torch.bfloat16)
    if scale is None or scale > 0:
        ref, ref_lse = ref_attention(q, k, v, causal, scale)
    else:
        # CPU ATen's flash attention returns NaN (causal) or zeros for a
        # negative scale, so the float64 closed form is the reference there
        ro, rl = npr.attention64(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal,
                                 scale)
        ref, ref_lse = torch.from_numpy(ro).bfloat16(), torch.from_numpy(rl).float()
    out = torch.empty(B, H, S, D, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(B, H, S, dtype=torch.float32, device="cuda")
    _abi.flash_attention_fwd(out, lse, q.cuda(), k.cuda(), v.cuda(), causal, scale)
    assert_close(out, ref, "bf16", f"attention scale={scale} ramp={ramp} causal={causal}")
    assert (lse.cpu() - ref_lse).abs().max().item() < 2e-2 * max(1.0, ref_lse.abs().max().item())


@pytest.mark.parametrize("causal", [True, False])
def test_flash_attention_long_ramp_forces_late_rescales(causal):
    """1024 keys (16 tiles) whose scale ramps from 0.2 to 8 along the
    sequence: after the first 8 tiles (exact running max) the row max keeps
    growing by more than 8 log2 units, so the late rescale branch runs, and
    rows between two rescales carry p up to 2^8 into the P V product."""
    B, H, S, D = 1, 2, 1024, 128
    q, k, v = rn((B, H, S, D), 41), rn((B, H, S, D), 42), rn((B, H, S, D), 43)
    k = (k.float() * torch.linspace(0.2, 8.0, S)[None, None, :, None]).to(torch.bfloat16)
    # the late branch is reached: some row's scaled max grows by > 8 log2
    # units after key 512 (checked on the fp32 scores of the first head)
    s = (q[0, 0].float() @ k[0, 0].float().t()) * (D ** -0.5) * 1.4426950408889634
    if causal:
        s = s.masked_fill(torch.ones(S, S).triu(1).bool(), float("-inf"))
    growth = s[:, 512:].amax(1) - s[:, :512].amax(1)
    assert (growth > 8.0).any(), growth.max()
    ref, ref_lse = ref_attention(q, k, v, causal)
    out = torch.empty(B, H, S, D, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(B, H, S, dtype=torch.float32, device="cuda")
    _abi.flash_attention_fwd(out, lse, q.cuda(), k.cuda(), v.cuda(), causal)
    r = bar_ratio(out, ref, "bf16")
    print(f"long ramp causal={causal}: max |error| / bar = {r:.3f}", flush=True)
    assert_close(out, ref, "bf16", f"long ramp causal={causal}")
    assert (lse.cpu() - ref_lse).abs().max().item() < 2e-2 * max(1.0, ref_lse.abs().max().item())


def test_flash_attention_long_non_causal_keys():
    """[1, 2, 128 x 2048, 128] non-causal: 32 key tiles, 24 of them past
    the exact-max tiles."""
    q, k, v = rn((1, 2, 128, 128), 44), rn((1, 2, 2048, 128), 45), rn((1, 2, 2048, 128), 46)
    ref, ref_lse = ref_attention(q, k, v, False)
    out = torch.empty(1, 2, 128, 128, dtype=torch.bfloat16, device="cuda")
    lse = torch.empty(1, 2, 128, dtype=torch.float32, device="cuda")
    _abi.flash_attention_fwd(out, lse, q.cuda(), k.cuda(), v.cuda(), False)
    print(f"long non-causal: max |error| / bar = {bar_ratio(out, ref, 'bf16'):.3f}", flush=True)
    assert_close(out, ref, "bf16", "long non-causal")
    assert (lse.cpu() - ref_lse).abs().max().item() < 2e-2 * max(1.0, ref_lse.abs().max().item())


def test_config5_attention_shape_head_sample():
    """[8, 32, 2048, 128] causal: all heads computed, 3 heads checked."""
    B, H, S, D = 8, 32, 2048, 128
    q, k, v = rn((B, H, S, D), 4), rn((B, H, S, D), 5), rn((B, H, S, D), 6)
    out = torch.empty(B, H, S, D, dtype=torch.bfloat16, device="cuda")
    _abi.flash_attention_fwd(out, None, q.cuda(), k.cuda(), v.cuda(), True)
    o = out.cpu()
    for b, h in [(0, 0), (3, 17), (7, 31)]:
        ref, _ = ref_attention(q[b:b + 1, h:h + 1], k[b:b + 1, h:h + 1], v[b:b + 1, h:h + 1], True)
        r = bar_ratio(o[b:b + 1, h:h + 1], ref, "bf16")
        print(f"config-5 head {b},{h}: max |error| / bar = {r:.3f}", flush=True)
        assert_close(o[b:b + 1, h:h + 1], ref, "bf16", f"head {b},{h}")


def test_sdpa_on_gcu_uses_flash_and_matches():
    q, k, v = rn((2, 4, 160, 128), 7), rn((2, 4, 160, 128), 8), rn((2, 4, 160, 128), 9)
    torch_gcu._C._set_op_debug_config("op_statistics=true")
    torch_gcu._C._clear_op_statistics()
    try:
        out = F.scaled_dot_product_attention(q.to("gcu"), k.to("gcu"), v.to("gcu"), is_causal=True)
        stats = torch_gcu._C._op_statistics()
    finally:
        torch_gcu._C._set_op_debug_config("")
    assert stats.get("_scaled_dot_product_fused_attention_overrideable", (0, 0))[0] == 1, stats
    ref, _ = ref_attention(q, k, v, True)
    assert_close(out.cpu(), ref, "bf16", "sdpa gcu")
    # a float32 mask selects the math path (native bmm + softmax)
    mask = torch.zeros(160, 160)
    out2 = F.scaled_dot_product_attention(q.float().to("gcu"), k.float().to("gcu"),
                                          v.float().to("gcu"), attn_mask=mask.to("gcu"))
    ref2, _ = ref_attention(q.float(), k.float(), v.float(), False)
    assert_close(out2.cpu(), ref2, "fp32", "sdpa math path")


SMALL = dl.LayerConfig(vocab=1000, hidden=256, heads=2, head_dim=128, ffn=512)


def test_decoder_layer_gcu_matches_cpu():
    w = dl.init_weights(SMALL, seed=11)
    ids = torch.randint(0, SMALL.vocab, (2, 96), generator=g(12))
    ref = dl.forward(w, ids, SMALL)
    truth = dl.forward({k: v.float() for k, v in w.items()}, ids, SMALL)
    wg = {k: v.to("gcu") for k, v in w.items()}
    out = dl.forward(wg, ids.to("gcu"), SMALL)
    assert_composed_close(out.cpu(), ref, truth, "decoder layer")


def test_decoder_layer_graph_replay_equals_eager():
    w = {k: v.to("gcu") for k, v in dl.init_weights(SMALL, seed=13).items()}
    ids = torch.randint(0, SMALL.vocab, (2, 128), generator=g(14)).to("gcu")
    pos = dl.positions(2, 128, "gcu")
    eager = dl.forward(w, ids, SMALL, pos)
    graph = torch.gcu.GCUGraph()
    torch.gcu.synchronize()
    with torch.gcu.graph(graph):
        out = dl.forward(w, ids, SMALL, pos)
    for k in range(3):
        graph.replay()
        torch.gcu.synchronize()
        assert_exact(out.cpu(), eager.cpu(), f"replay {k}")
    new_ids = torch.randint(0, SMALL.vocab, (2, 128), generator=g(15))
    ids.copy_(new_ids.to("gcu"))
    graph.replay()
    torch.gcu.synchronize()
    assert_exact(out.cpu(), dl.forward(w, ids, SMALL, pos).cpu(), "replay with new ids")
    graph.reset()


# ---- config 5 at its configured shape -------------------------------------------

C5 = dl.LayerConfig()  # hidden 4096, 32 heads x 128, FFN 11008, vocab 32000
C5_B, C5_S = 8, 2048


@pytest.fixture(scope="module")
def c5_layer():
    """The config-5 layer (random-init bf16 weights) over B8 x S2048 token ids,
    run once on gcu: (weights on CPU, fp32 weights, ids, weights on gcu,
    the gcu output on the host)."""
    w = dl.init_weights(C5, seed=20261205)
    w32 = {k: v.float() for k, v in w.items()}
    ids = torch.randint(0, C5.vocab, (C5_B, C5_S), generator=g(20261206))
    wg = {k: v.to("gcu") for k, v in w.items()}
    out = dl.forward(wg, ids.to("gcu"), C5).cpu()
    return w, w32, ids, wg, out


@pytest.mark.parametrize("b", range(C5_B))
def test_config5_layer_full_shape_matches_cpu_per_sequence(c5_layer, b):
    """Sequences of a causal layer are independent, so row block b of the
    full-batch gcu output must match the CPU ATen layer run on sequence b
    alone: every projection, the attention and the FFN at their config-5
    shapes ([16384, 4096] x [4096, 11008] and the rest) are checked through
    the output they produce."""
    w, w32, ids, _, out = c5_layer
    rows = slice(b * C5_S, (b + 1) * C5_S)
    ref = dl.forward(w, ids[b:b + 1], C5)       # CPU ATen, bf16
    truth = dl.forward(w32, ids[b:b + 1], C5)   # the same chain in fp32
    assert out[rows].shape == ref.shape
    assert torch.isfinite(out[rows].float()).all()
    assert_composed_close(out[rows], ref, truth, f"config-5 layer, sequence {b}")


def test_config5_layer_full_shape_under_op_check(c5_layer):
    """The full B8 x S2048 layer, unfused (every projection a plain linear,
    then the adds and silu_mul), with op_check on every native op: each call
    runs on gcu, then on CPU ATen over host copies of its arguments, and the
    outputs are compared at the bf16 op bar (rtol 1e-2; atol 1e-3, which the
    test requires to be at most 1e-2 x the rms of every output compared
    inexactly, so it is no looser than the bar's absolute floor; the
    embedding gather and the adds must match bit for bit).  Op-check statistics
    show what was compared: the projections at their three shapes (mm),
    the embedding (index_select) and the residual adds.  The host copies
    themselves (_copy_from) and the fused and attention ops have no CPU ATen
    kernel under the same schema and are not op-checked (as in the
    reference's YAML); their parity is tested above and in the kernel
    tests.  The unfused layer's output under op_check equals the fused
    layer's eager output bit for bit (op_check returns the gcu result, and the
    fused matmul epilogues round as linear + add and linear, linear +
    silu_mul do), so the per-op bar holds for the fused layer too."""
    _, _, ids, wg, out = c5_layer
    idg = ids.to("gcu")
    C = torch_gcu._C
    C._set_op_debug_config("op_check=all_ops op_check_tol_bf16=1e-2,1e-3 "
                           "op_check_tol_fp32=1e-5,1e-5 op_statistics=true")
    C._clear_op_check_statistics()
    C._clear_op_statistics()
    try:
        got = dl.forward(wg, idg, C5, fused=False).cpu()
        checks = C._op_check_statistics()
        info = C._get_op_statistics_info()
    finally:
        C._set_op_debug_config("")
    for op, e in sorted(checks.items()):
        print(f"op_check {op}: compared {e['compared']} failed {e['failed']} "
              f"max |d|/tol {e['max_ratio']:.3f} min rms(ref) {e['min_ref_rms']:.4g}", flush=True)
    assert checks["mm"]["compared"] == 7, checks
    assert checks["index_select"]["compared"] == 1, checks
    assert checks["add_Tensor"]["compared"] == 2, checks
    for op, e in checks.items():
        assert e["failed"] == 0 and e["max_ratio"] <= 1.0, (op, e)
        if e["max_ratio"] > 0 and e["min_ref_rms"] >= 0:
            assert 1e-3 <= 1e-2 * e["min_ref_rms"], (op, e)
    # the gather and the residual adds (fp32 sum, one rounding) are bit-exact
    assert checks["index_select"]["max_ratio"] == 0.0, checks
    assert checks["add_Tensor"]["max_ratio"] == 0.0, checks
    mm_lines = [ln for ln in info.splitlines() if "x (self=Tensor" in ln and "mat2=" in ln]
    shapes = {(ln.split("shape")[1].split("]")[0], ln.split("mat2=Tensor(shape")[1].split("]")[0])
              for ln in mm_lines}
    assert shapes == {("[16384, 4096", "[4096, 4096"), ("[16384, 4096", "[4096, 11008"),
                      ("[16384, 11008", "[11008, 4096")}, mm_lines
    assert_exact(got, out, "unfused layer under op_check equals the fused eager layer")


def test_config5_layer_full_shape_graph_replay_equals_eager(c5_layer):
    """GCUGraph capture of the full-shape layer: every replay equals eager
    execution bit for bit, and eager execution is deterministic (equal to
    the fixture's run)."""
    _, _, ids, wg, out = c5_layer
    idg = ids.to("gcu")
    pos = dl.positions(C5_B, C5_S, "gcu")
    eager = dl.forward(wg, idg, C5, pos)
    assert_exact(eager.cpu(), out, "eager run-to-run")
    graph = torch.gcu.GCUGraph()
    torch.gcu.synchronize()
    with torch.gcu.graph(graph):
        gout = dl.forward(wg, idg, C5, pos)
    for k in range(2):
        graph.replay()
        torch.gcu.synchronize()
        assert_exact(gout.cpu(), out, f"full-shape replay {k}")
    graph.reset()


# ---- SDPA under autograd and the grouped-query rule --------------------------------

def test_sdpa_backward_on_gcu_matches_cpu():
    """With q/k/v requiring grad the math path runs (the flash kernel is
    forward only); gradients match CPU ATen's."""
    B, H, S, D = 2, 4, 96, 64
    q0, k0, v0 = rn((B, H, S, D), 21), rn((B, H, S, D), 22), rn((B, H, S, D), 23)
    dout = rn((B, H, S, D), 24)

    def grads(dev, dtype):
        q, k, v = (t.detach().to(dtype).to(dev).clone().requires_grad_() for t in (q0, k0, v0))
        o = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        o.backward(dout.to(dtype).to(dev))
        return [o.detach().cpu()] + [t.grad.cpu() for t in (q, k, v)]

    torch_gcu._C._set_op_debug_config("op_statistics=true")
    torch_gcu._C._clear_op_statistics()
    try:
        gcu = grads("gcu", torch.bfloat16)
        stats = torch_gcu._C._op_statistics()
    finally:
        torch_gcu._C._set_op_debug_config("")
    assert "_scaled_dot_product_fused_attention_overrideable" not in stats, stats
    cpu = grads("cpu", torch.bfloat16)
    f32 = grads("cpu", torch.float32)
    for name, a, c, t in zip(("out", "dq", "dk", "dv"), gcu, cpu, f32):
        assert_composed_close(a, c, t, f"sdpa backward {name}")
    # without grad the flash kernel still runs
    with torch.no_grad():
        out = F.scaled_dot_product_attention(q0.to("gcu"), k0.to("gcu"), v0.to("gcu"),
                                             is_causal=True)
    assert_close(out.cpu(), ref_attention(q0, k0, v0, True)[0], "bf16", "sdpa no_grad")


def test_sdpa_grouped_query_heads_follow_enable_gqa():
    q, k, v = rn((1, 8, 64, 128), 31), rn((1, 2, 64, 128), 32), rn((1, 2, 64, 128), 33)
    with pytest.raises(RuntimeError) as cpu_err:
        F.scaled_dot_product_attention(q, k, v)
    with pytest.raises(RuntimeError):
        F.scaled_dot_product_attention(q.to("gcu"), k.to("gcu"), v.to("gcu"))
    assert cpu_err.value is not None
    out = F.scaled_dot_product_attention(q.to("gcu"), k.to("gcu"), v.to("gcu"), enable_gqa=True)
    ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), enable_gqa=True)
    assert_close(out.cpu(), ref.to(torch.bfloat16), "bf16", "sdpa enable_gqa")
    # a k/v batch of 1 broadcast by the math path, not handed to the kernel
    kb, vb = rn((1, 8, 64, 128), 34), rn((1, 8, 64, 128), 35)
    q2 = rn((2, 8, 64, 128), 36)
    out2 = F.scaled_dot_product_attention(q2.to("gcu"), kb.to("gcu"), vb.to("gcu"))
    ref2 = F.scaled_dot_product_attention(q2.float(), kb.float(), vb.float())
    assert_close(out2.cpu(), ref2.to(torch.bfloat16), "bf16", "sdpa broadcast batch")
