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
        assert torch._C._dispatch_has_kernel_for_dispatch_key(full, "PrivateUse1"), full


def test_generated_sources_are_deterministic():
    with tempfile.TemporaryDirectory() as d1, tempfile.TemporaryDirectory() as d2:
        gen_register.generate(d1)
        gen_register.generate(d2)
        for f in ("RegisterGCU.cpp", "aotops.h"):
            assert open(os.path.join(d1, f)).read() == open(os.path.join(d2, f)).read()
        src = open(os.path.join(d1, "RegisterGCU.cpp")).read()
        assert 'm.impl("add.out", TORCH_FN(wrapper_PrivateUse1_add_out));' in src
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
