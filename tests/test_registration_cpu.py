"""The generated PrivateUse1 registrations and the host runtime's CPU-side
behaviour (CPU only: nothing here launches a kernel)."""
import os
import sys
import tempfile

import pytest
import torch

import torch_gcu  # noqa: F401  (registers the gcu backend)

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "torch-gcu_amd", "codegen"))
import gen_register  # noqa: E402


def test_backend_is_named_gcu():
    assert torch._C._get_privateuse1_backend_name() == "gcu"
    assert hasattr(torch, "gcu") and hasattr(torch.Tensor, "gcu")
    assert torch.gcu.device_count() >= 0


def test_every_yaml_op_has_a_schema_and_a_kernel():
    entries = gen_register.load_entries()
    schemas = gen_register.native_schemas()
    assert len(entries) >= 40
    for e in entries:
        assert e.name in schemas, e.name
        name, _, overload = e.name.partition(".")
        full = f"aten::{name}" + (f".{overload}" if overload else "")
        want = e.env_gate is None or os.environ.get(e.env_gate, "").strip().lower() == "true"
        assert torch._C._dispatch_has_kernel_for_dispatch_key(full, "PrivateUse1") == want, full


@pytest.mark.parametrize("value,registered", [("true", True), (" TRUE ", True), ("false", False),
                                              ("1", False), (None, False)])
def test_linear_override_is_env_gated(value, registered):
    """linear / matmul (and their .out forms) are registered on PrivateUse1
    only when ENFLAME_PT_ENABLE_LINEAR_OVERRIDE reads "true" at library load,
    as the reference's RegisterLinearOverrideGCU.cpp:575-590 does."""
    import subprocess

    env = dict(os.environ)
    env.pop("ENFLAME_PT_ENABLE_LINEAR_OVERRIDE", None)
    if value is not None:
        env["ENFLAME_PT_ENABLE_LINEAR_OVERRIDE"] = value
    code = ("import torch, torch_gcu\n"
            "print([torch._C._dispatch_has_kernel_for_dispatch_key(o, 'PrivateUse1') for o in "
            "('aten::linear', 'aten::linear.out', 'aten::matmul', 'aten::matmul.out', 'aten::addmv')])")
    env["PYTHONPATH"] = os.pathsep.join([os.path.join(REPO, "torch-gcu_amd"), REPO,
                                         env.get("PYTHONPATH", "")])
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    flags = eval(r.stdout.strip().splitlines()[-1])
    assert flags == [registered] * 4 + [True], flags


def test_generated_sources_are_deterministic():
    with tempfile.TemporaryDirectory() as d1, tempfile.TemporaryDirectory() as d2:
        gen_register.generate(d1)
        gen_register.generate(d2)
        for f in ("RegisterGCU.cpp", "aotops.h"):
            assert open(os.path.join(d1, f)).read() == open(os.path.join(d2, f)).read()
        src = open(os.path.join(d1, "RegisterGCU.cpp")).read()
        assert ('if (!torch_gcu::deregistered("add.out", "add_out")) '
                'm.impl("add.out", TORCH_FN(wrapper_PrivateUse1_add_out));') in src
        assert ('if (torch_gcu::env_true("ENFLAME_PT_ENABLE_LINEAR_OVERRIDE")) { '
                'if (!torch_gcu::deregistered("linear", "linear")) '
                'm.impl("linear", TORCH_FN(wrapper_PrivateUse1_linear)); }') in src
        # factory ops guard on their device argument, compute ops on a tensor
        assert "const c10::OptionalDeviceGuard device_guard(device);" in src
        assert "call_fallback_fn<&torch_gcu::gcu_cpu_fallback, ATEN_OP2(mul, Tensor)>" in src


def test_unknown_op_is_rejected(tmp_path):
    bad = tmp_path / "ops.yaml"
    bad.write_text("backend: GCU\ncpp_namespace: torch_gcu\nsupported:\n- name: not_an_op.out\n")
    old = gen_register.OPS_YAML
    try:
        gen_register.OPS_YAML = str(bad)
        with pytest.raises(KeyError):
            gen_register.generate(str(tmp_path))
    finally:
        gen_register.OPS_YAML = old


def test_efficient_ops_are_dispatcher_ops():
    for op in ("rms_norm", "rope", "rope_", "silu_mul", "int32_indices_index"):
        assert hasattr(torch.ops.torch_gcu, op)
        assert torch._C._dispatch_has_kernel_for_dispatch_key(f"torch_gcu::{op}", "PrivateUse1")


def test_op_debug_config_parsing():
    C = torch_gcu._C
    C._set_op_debug_config("fallback_cpu=add.out,mul op_check=all_ops op_check_no_break=true")
    C._set_op_debug_config("")  # back to defaults
    with pytest.raises(RuntimeError):
        C._set_op_debug_config("fallback_cpu")  # missing '='
    C._clear_op_statistics()
    assert C._op_statistics() == {}


def test_gcu_module_surface():
    g = torch.gcu
    for name in ["is_available", "device_count", "current_device", "set_device", "synchronize",
                 "Stream", "Event", "current_stream", "default_stream", "stream", "set_stream",
                 "memory_allocated", "max_memory_allocated", "memory_reserved", "memory_stats",
                 "empty_cache", "set_per_process_memory_fraction", "mem_get_info",
                 "GCUGraph", "graph", "graph_pool_handle", "manual_seed", "get_rng_state",
                 "efficient"]:
        assert hasattr(g, name), name
    for name in ["rms_norm", "rope", "rope_", "silu_mul", "gcu_index"]:
        assert hasattr(g.efficient, name), name


# ---- op debug configuration, scopes and the fallback policy ---------------------------

def test_op_debug_config_keys_and_tolerances():
    """The reference's keys (op_debug_config.cpp:25-118): tolerances as
    rtol,atol with either part optional, dump folders under dump_path with a
    pid/time suffix unless test_mode."""
    C = torch_gcu._C
    try:
        C._set_op_debug_config("op_check_tol_fp32=1e-4, op_check_tol_fp16=,1e-5 "
                               "op_check_tol_bf16=2e-2,3e-2 dump_path=/tmp/gcu_dbg")
        c = C._op_debug_config()
        assert c["op_check_tol"] == ((1e-4, 1e-6), (1e-3, 1e-5), (2e-2, 3e-2))
        assert c["op_check_dump_dir"].startswith("/tmp/gcu_dbg/op_check_dump_")
        assert c["op_dump_dir"].startswith("/tmp/gcu_dbg/op_dump_")
        assert str(os.getpid()) in c["op_dump_dir"]
        C._set_op_debug_config("dump_path=/tmp/gcu_dbg test_mode=true op_statistics_dump=true")
        c = C._op_debug_config()
        assert c["op_check_dump_dir"] == "/tmp/gcu_dbg/op_check_dump"
        assert c["op_dump_dir"] == "/tmp/gcu_dbg/op_dump"
        assert c["op_statistics"] and c["op_statistics_dump"]
        C._set_op_debug_config("")
        c = C._op_debug_config()
        assert c["dump_path"] == "./torch_gcu_dump_file"
        assert c["op_check_tol"] == ((1e-6, 1e-6), (1e-3, 1e-3), (1e-3, 1e-3))
    finally:
        C._set_op_debug_config("")


def test_op_debug_scopes_and_ctx():
    C = torch_gcu._C
    dbg = torch.gcu.debug
    assert dbg.OpDebugCtx.current_state() == {"dump_op_name": False, "fallback_cpu": False,
                                              "op_check": False}
    with dbg.OpDebugCtx(enable_dump_op_name=False, enable_fallback_cpu=True):
        assert C._get_fallback_cpu_scope_state() and not C._get_dump_op_name_scope_state()
    with dbg.OpDebugCtx(enable_op_check=True):
        assert C._get_op_check_scope_state() and C._get_dump_op_name_scope_state()
    assert not any(dbg.OpDebugCtx.current_state().values())
    pre, post = dbg.get_pre_func(), dbg.get_post_func()
    pre(None)
    assert C._get_dump_op_name_scope_state()
    post(None, None)
    assert not C._get_dump_op_name_scope_state()


def test_fallback_policy_registry():
    """codegen/gcu_op_fallback.yaml's mi355x column is compiled into the
    wrappers and recorded: complex tensors take CPU ATen on the native
    compute ops, fp64 / integer / complex operands on the GEMM family."""
    pol = torch_gcu._C._fallback_policy()
    assert "self::ComplexFloat" in pol["add.out"] and "other::ComplexDouble" in pol["add.out"]
    assert "dtype::ComplexFloat" in pol["sum.dim_IntList"]
    assert {"self::Long", "self::Double", "self::ComplexFloat"} <= set(pol["mm.out"])
    assert "mat1::Int" in pol["addmm"] and "tensors::ComplexFloat" in pol["cat"]
    policy = gen_register.load_policy()
    assert set(pol) == set(policy)
    native = {e.name for e in gen_register.load_entries()}
    assert set(pol) <= native


def test_policy_codegen_rules_and_errors(tmp_path):
    with tempfile.TemporaryDirectory() as d:
        gen_register.generate(d)
        src = open(os.path.join(d, "RegisterGCU.cpp")).read()
    assert ("(self.defined() && (self.scalar_type() == at::ScalarType::ComplexHalf || "
            "self.scalar_type() == at::ScalarType::ComplexFloat") in src
    assert "torch_gcu::any_dtype_in(tensors, {at::ScalarType::ComplexHalf" in src
    assert "(dtype.has_value() && ((*dtype) == at::ScalarType::ComplexHalf" in src
    assert 'torch_gcu::register_fallback_policy("add.out", {"self::ComplexHalf"' in src

    def gen_with(text):
        f = tmp_path / "policy.yaml"
        f.write_text(text)
        old = gen_register.POLICY_YAML
        try:
            gen_register.POLICY_YAML = str(f)
            out = tmp_path / "gen"
            out.mkdir(exist_ok=True)
            gen_register.generate(str(out))
            return (out / "RegisterGCU.cpp").read_text()
        finally:
            gen_register.POLICY_YAML = old

    # "all", a bool rule and an int rule; other hardware keys are ignored
    src = gen_with("fallback:\n- name: _softmax\n  mi355x: all\n"
                   "- name: _log_softmax\n  mi355x:\n    - half_to_float: true\n    - dim: 0,2\n"
                   "- name: cos.out\n  s60: all\n")
    assert "return at::native::call_fallback_fn<&torch_gcu::gcu_cpu_fallback, ATEN_OP(_softmax)>" in src
    assert "(half_to_float == true) || (dim == 0 || dim == 2)" in src
    with pytest.raises(AssertionError, match="without a native kernel"):
        gen_with("fallback:\n- name: cos.out\n  mi355x: all\n")
    with pytest.raises(AssertionError, match="not an argument"):
        gen_with("fallback:\n- name: add.out\n  mi355x:\n    - input: Float\n")
    with pytest.raises(AssertionError, match="not a dtype"):
        gen_with("fallback:\n- name: add.out\n  mi355x:\n    - self: Float32\n")


def test_deregister_skips_native_registration():
    """deregister=<ops> (read when the library loads) leaves those ops to the
    CPU fallback, as the reference's isDeregister guard does
    (codegen/gen_backend_stubs.py:616-642)."""
    import subprocess

    env = dict(os.environ)
    env["ENFLAME_PT_OP_DEBUG_CONFIG"] = "deregister=mul.Tensor,sum"
    env["PYTHONPATH"] = os.pathsep.join([os.path.join(REPO, "torch-gcu_amd"), REPO,
                                         env.get("PYTHONPATH", "")])
    code = ("import torch, torch_gcu\n"
            "print([torch._C._dispatch_has_kernel_for_dispatch_key(o, 'PrivateUse1') for o in "
            "('aten::mul.Tensor', 'aten::mul.out', 'aten::sum.dim_IntList', "
            "'aten::sum.IntList_out', 'aten::add.out')])")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert eval(r.stdout.strip().splitlines()[-1]) == [False, True, False, False, True]
