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
        assert 'm.impl("add.out", TORCH_FN(wrapper_PrivateUse1_add_out));' in src
        assert ('if (torch_gcu::env_true("ENFLAME_PT_ENABLE_LINEAR_OVERRIDE")) '
                'm.impl("linear", TORCH_FN(wrapper_PrivateUse1_linear));') in src
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
