"""The CPU fallback and the op-debug tools on gcu tensors.

* Ops whose CPU kernel lacks Half / BFloat16 run in float and come back in
  their own dtype (the reference's aten_cpu_fallback.cpp:193-340), compared
  with oracle.aten.widened_fallback.
* The fallback policy of codegen/gcu_op_fallback.yaml routes calls whose
  arguments match a rule (complex tensors, integer GEMM operands, a complex
  dtype= argument) to CPU ATen and leaves the others native.
* ENFLAME_PT_OP_DEBUG_CONFIG's dumps, op_check dump, calltrace, op-name and
  fallback / op-check scopes, exclusions and the statistics JSON
  (op_debug_config.cpp:25-118, gcu_op_check.h:19-82, InitGcuBindings.cpp:
  131-153).
"""
import json
import os

import pytest
import torch

import torch_gcu
from oracle import aten
from oracle.tolerance import assert_close, assert_exact

pytestmark = pytest.mark.gpu

C = torch_gcu._C


def g(seed):
    return torch.Generator().manual_seed(seed)


@pytest.fixture(autouse=True)
def _clean_debug():
    C._set_op_debug_config("")
    C._clear_op_statistics()
    yield
    C._set_op_debug_config("")
    for f in ("_exit_print_cpp_name_scope", "_exit_fallback_cpu_scope", "_exit_op_check_scope"):
        getattr(C, f)()
    torch.gcu.synchronize()


def stats_of(fn):
    C._set_op_debug_config("op_statistics=true")
    C._clear_op_statistics()
    try:
        out = fn()
        torch.gcu.synchronize()
        return out, C._op_statistics()
    finally:
        C._set_op_debug_config("")


# ---- the fallback widened to float ------------------------------------------------------

@pytest.mark.parametrize("low", [torch.float16, torch.bfloat16])
def test_fallback_retries_in_float_when_cpu_lacks_the_dtype(low):
    m = torch.randn(40, 40, generator=g(1)).to(low)
    x = (torch.rand(3000, generator=g(2)) * 6 - 2).to(low)
    # at most 25 rows each: cdist's own kernel (_cdist_forward), not its
    # matmul decomposition
    a, b = torch.randn(20, 16, generator=g(3)).to(low), torch.randn(12, 16, generator=g(4)).to(low)
    with pytest.warns(UserWarning, match="convert"):
        t = torch.trace(m.to("gcu"))
    assert t.device.type == "gcu" and t.dtype == low
    assert_exact(t.cpu(), aten.widened_fallback(torch.trace, m), f"trace {low}")
    e = torch.special.erfcx(x.to("gcu"))
    assert e.dtype == low
    assert_exact(e.cpu(), aten.widened_fallback(torch.special.erfcx, x), f"erfcx {low}")
    d = torch.cdist(a.to("gcu"), b.to("gcu"))
    assert d.dtype == low
    assert_exact(d.cpu(), aten.widened_fallback(torch.cdist, a, b), f"cdist {low}")


def test_fallback_retry_writes_out_arguments_in_their_dtype():
    x = (torch.rand(777, generator=g(5)) * 4 - 1).half()
    out = torch.full((777,), 7.0, dtype=torch.float16, device="gcu")
    r = torch.special.erfcx(x.to("gcu"), out=out)
    assert r is out and out.dtype == torch.float16
    assert_exact(out.cpu(), aten.widened_fallback(torch.special.erfcx, x), "erfcx out=")
    # a resized out
    out2 = torch.empty(0, dtype=torch.float16, device="gcu")
    torch.special.erfcx(x.to("gcu"), out=out2)
    assert out2.shape == (777,)
    assert_exact(out2.cpu(), aten.widened_fallback(torch.special.erfcx, x), "erfcx resized out")
    # ops with a Half kernel on CPU are not widened
    (y, st) = stats_of(lambda: torch.cos(x.to("gcu")))
    assert_exact(y.cpu(), torch.cos(x), "cos Half (no widening)")


# ---- fallback policy ---------------------------------------------------------------------

def test_policy_routes_complex_tensors_to_cpu():
    a = torch.randn(64, 3, dtype=torch.complex64, generator=g(6))
    b = torch.randn(64, 3, dtype=torch.complex64, generator=g(7))
    (r, st) = stats_of(lambda: a.to("gcu") + b.to("gcu"))
    assert_exact(r.cpu(), a + b, "complex add")
    assert st["add.Tensor"] == (0, 1), st
    x = torch.randn(64, 3, generator=g(8))
    (r, st) = stats_of(lambda: x.to("gcu") + x.to("gcu"))
    assert_exact(r.cpu(), x + x, "float add")
    assert st["add.Tensor"] == (1, 0), st
    (r, st) = stats_of(lambda: torch.cat([a.to("gcu"), b.to("gcu")], 0))
    assert_exact(r.cpu(), torch.cat([a, b], 0), "complex cat")
    assert st["cat"][1] == 1, st
    # a rule on a dtype= argument: a float tensor summed into complex
    (r, st) = stats_of(lambda: torch.sum(x.to("gcu"), 0, dtype=torch.complex64))
    assert_close(r.cpu().real, x.sum(0), "fp32", "sum dtype=complex64")
    assert st["sum.dim_IntList"] == (0, 1), st


def test_policy_routes_integer_and_fp64_gemm_operands_to_cpu():
    a = torch.randint(-5, 5, (17, 9), generator=g(9))
    b = torch.randint(-5, 5, (9, 11), generator=g(10))
    (r, st) = stats_of(lambda: torch.mm(a.to("gcu"), b.to("gcu")))
    assert_exact(r.cpu(), a @ b, "int64 mm")
    assert st["mm"] == (0, 1), st
    (r, st) = stats_of(lambda: torch.mm(a.double().to("gcu"), b.double().to("gcu")))
    assert_exact(r.cpu(), a.double() @ b.double(), "fp64 mm")
    assert st["mm"] == (0, 1), st
    (r, st) = stats_of(lambda: torch.mm(a.float().to("gcu"), b.float().to("gcu")))
    assert_exact(r.cpu(), a.float() @ b.float(), "fp32 mm (integer values, exact)")
    assert st["mm"] == (1, 0), st


# ---- dumps, op_check dump, calltrace, scopes ----------------------------------------------

def test_op_input_and_output_dump(tmp_path):
    x = torch.randn(33, 5, generator=g(11))
    C._set_op_debug_config(f"op_input_dump=mul op_output_dump=all_ops,-add dump_path={tmp_path} "
                           "test_mode=true")
    y = x.to("gcu") * 3.5
    z = y + 1
    torch.gcu.synchronize()
    d = tmp_path / "op_dump"
    files = sorted(os.listdir(d))
    ins = [f for f in files if f.startswith("mul_Tensor_") and "_input_args0" in f]
    outs = [f for f in files if f.startswith("mul_Tensor_") and "_output_args0" in f]
    assert len(ins) == 1 and len(outs) == 1, files
    assert not [f for f in files if f.startswith("add_")], files  # excluded by -add
    got_in = torch.load(d / ins[0], weights_only=True)
    assert_exact(got_in, x, "dumped input")
    got_out = torch.load(d / outs[0], weights_only=True)
    assert_exact(got_out, y.cpu(), "dumped output")
    # the Python number reaches mul.Tensor as a wrapped 0-dim CPU tensor
    scalar = torch.load(d / ins[0].replace("_args0.pt", "_args1.pt"), weights_only=True)
    assert scalar.dim() == 0 and float(scalar) == 3.5
    assert_exact(z.cpu(), x * 3.5 + 1, "dumped run result")


def test_op_check_mismatch_dumps_inputs_and_both_outputs(tmp_path):
    """A column mean of fp32 [16384, 512] adds in another order than CPU
    ATen, so at a zero tolerance op_check reports it; with op_check_dump the
    input and both outputs are saved (gcu_op_check.h:54-82)."""
    x = torch.randn(16384, 512, generator=g(12))
    C._set_op_debug_config(f"op_check=mean op_check_tol_fp32=0,0 op_check_dump=true "
                           f"dump_path={tmp_path} test_mode=true")
    with pytest.raises(RuntimeError, match="op_check failed for aten::mean") as err:
        torch.mean(x.to("gcu"), 0)
    assert "saved under" in str(err.value)
    d = tmp_path / "op_check_dump"
    files = os.listdir(d)
    inp = [f for f in files if "_input_args0.pt" in f]
    gcu = [f for f in files if "_gcu_output_args0.pt" in f]
    cpu = [f for f in files if "_cpu_output_args0.pt" in f]
    assert len(inp) == 1 and len(gcu) == 1 and len(cpu) == 1, files
    assert inp[0].startswith("mean_dim_")
    assert_exact(torch.load(d / inp[0], weights_only=True), x, "op_check dumped input")
    assert_exact(torch.load(d / cpu[0], weights_only=True), torch.mean(x, 0), "dumped CPU output")
    gout = torch.load(d / gcu[0], weights_only=True)
    assert_close(gout, torch.mean(x, 0), "fp32", "dumped gcu output")
    assert not torch.equal(gout, torch.mean(x, 0))
    # op_check_no_break logs instead of raising, and the run goes on
    C._set_op_debug_config(f"op_check=mean op_check_tol_fp32=0,0 op_check_no_break=true "
                           f"dump_path={tmp_path} test_mode=true")
    r = torch.mean(x.to("gcu"), 0)
    assert_close(r.cpu(), torch.mean(x, 0), "fp32", "no_break result")


def test_op_check_half_passes_at_the_default_tolerance():
    """op_check of a Half op at the reference's default fp16 tolerance."""
    x = torch.randn(500, generator=g(13)).half()
    C._set_op_debug_config("op_check=mul")
    y = x.to("gcu") * x.to("gcu")
    assert_exact(y.cpu(), x * x, "checked mul")


def test_calltrace_and_op_name_scope(capfd):
    x = torch.randn(8, generator=g(14)).to("gcu")
    C._set_op_debug_config("op_calltrace=true")
    x * 2
    torch.gcu.synchronize()
    C._set_op_debug_config("")
    err = capfd.readouterr().err
    assert "torch_gcu op calltrace: mul_Tensor (aten::mul.Tensor)" in err, err[-2000:]
    assert "test_calltrace_and_op_name_scope" in err  # the Python frame of the call
    with torch.gcu.debug.OpDebugCtx():
        x + 1
    err = capfd.readouterr().err
    assert 'torch_gcu op name "add_Tensor" (aten::add.Tensor)' in err, err[-2000:]


def test_fallback_and_op_check_scopes():
    x = torch.randn(100, generator=g(15))
    d = x.to("gcu")
    C._set_op_debug_config("op_statistics=true")
    with torch.gcu.debug.OpDebugCtx(enable_dump_op_name=False, enable_fallback_cpu=True):
        y = d * 2
    torch.gcu.synchronize()
    assert C._op_statistics()["mul.Tensor"] == (0, 1)
    assert_exact(y.cpu(), x * 2, "scoped fallback")
    C._clear_op_statistics()
    y = d * 2
    assert C._op_statistics()["mul.Tensor"] == (1, 0)
    # exclusions: every op on CPU except mul
    C._set_op_debug_config("fallback_cpu=all_ops,-mul op_statistics=true")
    C._clear_op_statistics()
    (d * 2) + 1
    st = C._op_statistics()
    assert st["mul.Tensor"] == (1, 0) and st["add.Tensor"] == (0, 1), st
    C._set_op_debug_config("op_check_tol_fp32=1e-5,1e-5")
    with torch.gcu.debug.OpDebugCtx(enable_dump_op_name=False, enable_op_check=True):
        z = (d * 3).sum()
    assert_close(z.cpu(), (x * 3).sum(), "fp32", "scoped op_check")


def test_statistics_info_and_json(tmp_path):
    x = torch.randn(20, 4, generator=g(16)).to("gcu")
    C._set_op_debug_config(f"op_statistics=true dump_path={tmp_path}")
    C._clear_op_statistics()
    for _ in range(3):
        x * 2
    x + torch.ones(4, device="gcu")
    torch.cos(x)
    torch.gcu.synchronize()
    info = torch.gcu.debug.get_op_statistics_info()
    assert "mul.Tensor" in info and "cos" in info
    path = torch.gcu.debug.dump_op_statistics_info()
    assert os.path.dirname(path) == str(tmp_path)
    assert os.path.basename(path).startswith(f"op_stat_{os.getpid()}_")
    recs = {r["aten_op_name"]: r for r in json.load(open(path))}
    mul = recs["mul.Tensor"]
    assert mul["native_count"] == 3 and mul["use_count"] == 3 and mul["params_count"] == 1
    assert "shape[20, 4]" in mul["params"][0]["args"] and mul["params"][0]["count"] == 3
    assert mul["schema"].startswith("aten::mul.Tensor(")
    cos = [r for n, r in recs.items() if n.startswith("cos")]
    assert cos and sum(r["fallback_count"] for r in cos) >= 1
    torch.gcu.debug.clear_op_statistics_info()
    assert C._op_statistics() == {}
