"""Generates the PrivateUse1 registrations of the gcu backend.

Input: ``gcu_native_functions.yaml`` (same flags as the reference's
codegen/gcu_native_functions.yaml).  Schemas come from the native_functions.yaml
packaged with torchgen, C++ signatures from torchgen's dispatcher API.

Output (into the build directory):

* ``aotops.h``         -- declarations of the hand-written native kernels
                          ``torch_gcu::aotops::<op>_<overload>``;
* ``RegisterGCU.cpp``  -- one ``wrapper_PrivateUse1_<op>`` per op doing what the
                          reference's generated wrappers do
                          (codegen/wrapper_torch_codegen.py:350-440 and
                          codegen/gen_GCUNativeFunctions_methods.py:145-330):
                          device check, device guard, forced CPU fallback /
                          op_check / statistics under ENFLAME_PT_OP_DEBUG_CONFIG,
                          the native call and the op_sync_mode stream sync;
                          then ``TORCH_LIBRARY_IMPL(aten, PrivateUse1, m)``.
"""
from __future__ import annotations

import os
import sys
from dataclasses import dataclass

import yaml

HERE = os.path.dirname(os.path.abspath(__file__))
OPS_YAML = os.path.join(HERE, "gcu_native_functions.yaml")


@dataclass
class OpEntry:
    name: str  # "add.out"
    device_check: bool = True
    device_guard: bool = True
    fallback_cpu: bool = True
    op_check: bool = True
    env_gate: str | None = None  # registered only when this variable reads "true"


def load_entries(path: str | None = None) -> list[OpEntry]:
    path = path or OPS_YAML
    with open(path) as f:
        doc = yaml.safe_load(f)
    assert doc.get("backend") == "GCU", "backend must be GCU"
    out = []
    for e in doc.get("supported", []):
        out.append(OpEntry(name=e["name"], device_check=e.get("device_check", True),
                           device_guard=e.get("device_guard", True),
                           fallback_cpu=e.get("fallback_cpu", True),
                           op_check=e.get("op_check", True),
                           env_gate=e.get("env_gate")))
    names = [e.name for e in out]
    dup = {n for n in names if names.count(n) > 1}
    assert not dup, f"duplicate ops in {path}: {sorted(dup)}"
    return out


def native_schemas() -> dict[str, tuple[str, bool, bool]]:
    import torchgen

    path = os.path.join(os.path.dirname(torchgen.__file__), "packaged", "ATen", "native",
                        "native_functions.yaml")
    loader = getattr(yaml, "CSafeLoader", yaml.SafeLoader)
    with open(path) as f:
        doc = yaml.load(f, Loader=loader)
    out = {}
    for e in doc:
        func = e["func"]
        head = func.split("(", 1)[0]
        # members of a structured group take Tensor[] as ITensorListRef in
        # the dispatcher's C++ signature (cat, cat.out)
        structured = bool(e.get("structured", False)) or "structured_delegate" in e
        out[head] = (func, bool(e.get("use_const_ref_for_mutable_tensors", False)), structured)
    return out


def cpp_name(opname: str) -> str:
    return opname.replace(".", "_")


def _signature(schema_str: str, const_mut: bool = False, structured: bool = False):
    from torchgen import local
    from torchgen.api.types import DispatcherSignature
    from torchgen.model import FunctionSchema

    with local.parametrize(use_const_ref_for_mutable_tensors=const_mut,
                           use_ilistref_for_tensor_lists=structured):
        schema = FunctionSchema.parse(schema_str)
        sig = DispatcherSignature.from_schema(schema, symint=False)
        args = [(a.type if hasattr(a, "type") else None, a.name) for a in sig.arguments()]
        decl_args = ", ".join(a.decl() for a in sig.arguments())
        ret = sig.returns_type().cpp_type()
        boxed = [a.nctype.cpp_type().replace(" &", "&") for a in sig.arguments()]
    return schema, boxed, decl_args, args, ret


def _tensor_args(schema):
    """(name, kind) of tensor-like arguments: 'tensor', 'opt', 'list'."""
    from torchgen.model import BaseTy, BaseType, ListType, OptionalType

    out = []
    for a in schema.arguments.flat_all:
        t = a.type
        if isinstance(t, BaseType) and t.name == BaseTy.Tensor:
            out.append((a.name, "tensor"))
        elif isinstance(t, OptionalType) and isinstance(t.elem, BaseType) and t.elem.name == BaseTy.Tensor:
            out.append((a.name, "opt"))
        elif isinstance(t, ListType) and isinstance(t.elem, BaseType) and t.elem.name == BaseTy.Tensor:
            out.append((a.name, "list"))
    return out


def _device_arg(schema):
    for a in schema.arguments.flat_all:
        if str(a.type) in ("Device?", "Device"):
            return a.name
    return None


def _aliased_return_arg(schema):
    """Name of the argument a Tensor(a!) return aliases, if any."""
    if len(schema.returns) != 1 or schema.returns[0].annotation is None:
        return None
    ann = schema.returns[0].annotation
    for a in schema.arguments.flat_all:
        if a.annotation is not None and a.annotation.alias_set == ann.alias_set:
            return a.name
    return None


def generate(out_dir: str) -> list[str]:
    entries = load_entries()
    schemas = native_schemas()
    decls, wrappers, regs = [], [], []
    for e in entries:
        if e.name not in schemas:
            raise KeyError(f"{e.name} is not an ATen operator (native_functions.yaml)")
        schema, boxed, decl_args, args, ret = _signature(*schemas[e.name])
        fn = cpp_name(e.name)
        arg_names = ", ".join(n for _, n in args)
        decls.append(f"{ret} {fn}({decl_args});")
        base, _, overload = e.name.partition(".")
        tensors = _tensor_args(schema)
        body = []
        if e.device_check and tensors:
            body.append("  std::optional<at::Device> common_device;")
            for n, kind in tensors:
                if kind == "tensor":
                    body.append(f"  torch_gcu::check_device(common_device, {n}, \"{e.name}\", \"{n}\");")
                elif kind == "opt":
                    body.append(f"  if ({n}.has_value()) torch_gcu::check_device(common_device, *{n}, \"{e.name}\", \"{n}\");")
                else:
                    body.append(f"  for (const auto& t_ : {n}) torch_gcu::check_device(common_device, t_, \"{e.name}\", \"{n}\");")
        if e.device_guard:
            dev = _device_arg(schema)
            if dev is not None:
                body.append(f"  const c10::OptionalDeviceGuard device_guard({dev});")
            else:
                first = [n for n, kind in tensors if kind == "tensor"]
                if first:
                    guard_expr = " , ".join(f"torch_gcu::gcu_device_of({n})" for n in first)
                    body.append(f"  const c10::OptionalDeviceGuard device_guard("
                                f"torch_gcu::first_gcu_device({{{guard_expr}}}));")
        # debug paths (fallback / op_check / statistics)
        dbg = []
        dbg.append(f"    static const std::string kName = \"{e.name}\";")
        dbg.append("    const auto& cfg = torch_gcu::OpDebugConfig::get();")
        if e.fallback_cpu:
            ovl = overload if overload else ""
            dbg.append("    if (cfg.forced_fallback(kName)) {")
            dbg.append(f"      return at::native::call_fallback_fn<&torch_gcu::gcu_cpu_fallback, "
                       f"ATEN_OP2({base}, {ovl})>::call({arg_names});"
                       if overload else
                       f"      return at::native::call_fallback_fn<&torch_gcu::gcu_cpu_fallback, "
                       f"ATEN_OP({base})>::call({arg_names});")
            dbg.append("    }")
        if e.op_check:
            alias = _aliased_return_arg(schema)
            ret_ok = ret in ("at::Tensor",) or alias is not None
            if ret_ok:
                dbg.append("    if (cfg.checked(kName) && !torch_gcu::in_op_check()) {")
                dbg.append("      torch_gcu::OpCheckScope scope_;")
                dbg.append(f"      static const auto op_ = c10::Dispatcher::singleton().findSchemaOrThrow(\"aten::{base}\", \"{overload}\");")
                dbg.append(f"      auto stack_ = c10::impl::boxArgs<{', '.join(boxed)}>({arg_names});")
                dbg.append("      torch_gcu::op_check_boxed(op_, &stack_, c10::DispatchKeySet(c10::DispatchKey::PrivateUse1));")
                if alias is not None:
                    dbg.append(f"      return {alias};")
                else:
                    dbg.append("      return stack_.back().toTensor();")
                dbg.append("    }")
        dbg.append("    if (cfg.statistics) torch_gcu::count_op(kName, false);")
        body.append("  if (C10_UNLIKELY(torch_gcu::op_debug_active())) {")
        body.extend(dbg)
        body.append("  }")
        body.append(f"  RECORD_FUNCTION(\"GCU::{e.name}\", std::vector<c10::IValue>());")
        if ret == "void":
            body.append(f"  torch_gcu::aotops::{fn}({arg_names});")
            body.append("  torch_gcu::after_op();")
        else:
            body.append(f"  {'auto&&' if '&' in ret else 'auto'} r_ = torch_gcu::aotops::{fn}({arg_names});")
            body.append("  torch_gcu::after_op();")
            body.append("  return r_;")
        wrappers.append(f"{ret} wrapper_PrivateUse1_{fn}({decl_args}) {{\n" + "\n".join(body) + "\n}\n")
        reg = f"m.impl(\"{e.name}\", TORCH_FN(wrapper_PrivateUse1_{fn}));"
        if e.env_gate:
            regs.append(f"  if (torch_gcu::env_true(\"{e.env_gate}\")) {reg}")
        else:
            regs.append(f"  {reg}")

    header_text = (
        "// Generated by codegen/gen_register.py from codegen/gcu_native_functions.yaml.\n"
        "// Hand-written native kernels of the gcu backend (csrc/host/ops_*.cpp).\n"
        "#pragma once\n#include <ATen/ATen.h>\n\nnamespace torch_gcu {\nnamespace aotops {\n\n"
        + "\n".join(decls) + "\n\n}  // namespace aotops\n}  // namespace torch_gcu\n")
    src_text = (
        "// Generated by codegen/gen_register.py from codegen/gcu_native_functions.yaml.\n"
        "#include <ATen/ATen.h>\n#include <ATen/Operators.h>\n"
        "#include <ATen/core/boxing/impl/boxing.h>\n#include <ATen/native/CPUFallback.h>\n"
        "#include <ATen/record_function.h>\n#include <c10/core/DeviceGuard.h>\n"
        "#include <torch/library.h>\n\n#include \"aotops.h\"\n#include \"dispatch_util.h\"\n"
        "#include \"op_debug.h\"\n\nnamespace {\n\n"
        + "\n".join(wrappers)
        + "\n}  // namespace\n\nTORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {\n"
        + "\n".join(regs) + "\n}\n")
    src = os.path.join(out_dir, "RegisterGCU.cpp")
    _write_if_changed(os.path.join(out_dir, "aotops.h"), header_text)
    _write_if_changed(src, src_text)
    return [src]


def _write_if_changed(path: str, text: str) -> None:
    if os.path.exists(path) and open(path).read() == text:
        return
    with open(path, "w") as f:
        f.write(text)


if __name__ == "__main__":
    d = sys.argv[1] if len(sys.argv) > 1 else "."
    os.makedirs(d, exist_ok=True)
    print(generate(d))
