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
                          device check, device guard, the fallback policy of
                          ``gcu_op_fallback.yaml``, forced CPU fallback /
                          op_check / input and output dumps / statistics /
                          calltrace under ENFLAME_PT_OP_DEBUG_CONFIG, the
                          native call and the op_sync_mode stream sync; then
                          ``TORCH_LIBRARY_IMPL(aten, PrivateUse1, m)``, which
                          skips ops the configuration deregisters and records
                          the policy for introspection.

The fallback policy (codegen/gcu_op_fallback.yaml, the format of the
reference's file and generator: codegen/gcu_op_fallback.yaml:1-64,
codegen/gen_op_fallback_register.py:112-176, register_fallback_ops.h:88-105)
names, for this hardware (the ``mi355x`` key), native ops that run on CPU
ATen always ("all") or when an argument takes one of the listed values: a
tensor by its dtype ("self: ComplexFloat"), a ScalarType, string, bool or
int argument by its value.  The rules become plain comparisons in the
wrapper, ahead of the native call.
"""
from __future__ import annotations

import os
import sys
from dataclasses import dataclass

import yaml

HERE = os.path.dirname(os.path.abspath(__file__))
OPS_YAML = os.path.join(HERE, "gcu_native_functions.yaml")
POLICY_YAML = os.path.join(HERE, "gcu_op_fallback.yaml")
HARDWARE = "mi355x"

# c10::ScalarType names a policy may list for a tensor or dtype argument
SCALAR_TYPES = {
    "Byte", "Char", "Short", "Int", "Long", "Half", "Float", "Double", "ComplexHalf",
    "ComplexFloat", "ComplexDouble", "Bool", "BFloat16", "UInt16", "UInt32", "UInt64",
    "Float8_e5m2", "Float8_e4m3fn", "Float8_e5m2fnuz", "Float8_e4m3fnuz",
}


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


def load_policy(path: str | None = None) -> dict[str, object]:
    """op name -> "all" or [(arg, [values]), ...] for this hardware."""
    path = path or POLICY_YAML
    with open(path) as f:
        doc = yaml.safe_load(f) or {}
    out: dict[str, object] = {}
    for e in doc.get("fallback", []) or []:
        cfg = e.get(HARDWARE)
        if cfg is None:
            continue
        name = e["name"]
        assert name not in out, f"{path}: {name} listed twice"
        if cfg == "all":
            out[name] = "all"
            continue
        assert isinstance(cfg, list), f"{path}: {name}: expected 'all' or a list of rules"
        rules = []
        for r in cfg:
            assert isinstance(r, dict) and len(r) == 1, f"{path}: {name}: bad rule {r!r}"
            (arg, vals), = r.items()
            values = [v.strip() for v in str(vals).split(",") if v.strip()]
            assert values, f"{path}: {name}: rule for {arg} has no values"
            rules.append((arg, values))
        out[name] = rules
    return out


def _policy_condition(op: str, schema, rules) -> tuple[str, list[str]]:
    """C++ condition that is true when a call must take the CPU fallback, and
    the rules as "arg::value" strings."""
    from torchgen.model import BaseTy, BaseType, ListType, OptionalType

    args = {a.name: a.type for a in schema.arguments.flat_all}
    terms, strings = [], []
    for arg, values in rules:
        assert arg in args, f"fallback policy of {op}: {arg} is not an argument of {schema}"
        t = args[arg]
        strings += [f"{arg}::{v}" for v in values]
        opt = isinstance(t, OptionalType)
        base = t.elem if opt else t

        def dtypes(expr):
            for v in values:
                assert v in SCALAR_TYPES, f"fallback policy of {op}: {v} is not a dtype"
            return " || ".join(f"{expr} == at::ScalarType::{v}" for v in values)

        if isinstance(base, BaseType) and base.name == BaseTy.Tensor:
            if opt:
                terms.append(f"({arg}.has_value() && {arg}->defined() && "
                             f"({dtypes(f'{arg}->scalar_type()')}))")
            else:
                terms.append(f"({arg}.defined() && ({dtypes(f'{arg}.scalar_type()')}))")
        elif isinstance(base, ListType) and isinstance(base.elem, BaseType) and \
                base.elem.name == BaseTy.Tensor:
            lst = ", ".join(f"at::ScalarType::{v}" for v in values)
            for v in values:
                assert v in SCALAR_TYPES, f"fallback policy of {op}: {v} is not a dtype"
            terms.append(f"torch_gcu::any_dtype_in({arg}, {{{lst}}})")
        elif isinstance(base, BaseType) and base.name == BaseTy.ScalarType:
            e = f"(*{arg})" if opt else arg
            cond = f"({dtypes(e)})"
            terms.append(f"({arg}.has_value() && {cond})" if opt else cond)
        elif isinstance(base, BaseType) and base.name == BaseTy.str:
            e = f"(*{arg})" if opt else arg
            cond = "(" + " || ".join(f'{e} == "{v}"' for v in values) + ")"
            terms.append(f"({arg}.has_value() && {cond})" if opt else cond)
        elif isinstance(base, BaseType) and base.name == BaseTy.bool:
            e = f"(*{arg})" if opt else arg
            vs = {"true": "true", "1": "true", "false": "false", "0": "false"}
            cond = "(" + " || ".join(f"{e} == {vs[v.lower()]}" for v in values) + ")"
            terms.append(f"({arg}.has_value() && {cond})" if opt else cond)
        elif isinstance(base, BaseType) and base.name in (BaseTy.int, BaseTy.SymInt):
            e = f"(*{arg})" if opt else arg
            cond = "(" + " || ".join(f"{e} == {int(v)}" for v in values) + ")"
            terms.append(f"({arg}.has_value() && {cond})" if opt else cond)
        elif isinstance(base, BaseType) and base.name == BaseTy.Scalar:
            e = f"{arg}->type()" if opt else f"{arg}.type()"
            cond = f"({dtypes(e)})"
            terms.append(f"({arg}.has_value() && {cond})" if opt else cond)
        else:
            raise AssertionError(f"fallback policy of {op}: argument {arg} of type {t} "
                                 "cannot carry a rule")
    return " || ".join(terms), strings


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
    policy = load_policy()
    used_policy: set[str] = set()
    schemas = native_schemas()
    decls, wrappers, regs, policy_regs = [], [], [], []
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
        ovl = overload if overload else ""
        fallback_call = (f"at::native::call_fallback_fn<&torch_gcu::gcu_cpu_fallback, "
                         f"ATEN_OP2({base}, {ovl})>::call({arg_names})" if overload else
                         f"at::native::call_fallback_fn<&torch_gcu::gcu_cpu_fallback, "
                         f"ATEN_OP({base})>::call({arg_names})")
        # the fallback policy of this hardware (gcu_op_fallback.yaml)
        pol = policy.get(e.name)
        if pol is not None:
            assert e.fallback_cpu, f"{e.name} has a fallback policy but fallback_cpu: false"
            if pol == "all":
                body.append(f"  return {fallback_call};  // fallback policy: all")
                policy_regs.append(f'  torch_gcu::register_fallback_policy("{e.name}", {{"all"}});')
            else:
                cond, strings = _policy_condition(e.name, schema, pol)
                body.append(f"  if ({cond}) return {fallback_call};  // fallback policy")
                lst = ", ".join(f'"{x}"' for x in strings)
                policy_regs.append(f'  torch_gcu::register_fallback_policy("{e.name}", {{{lst}}});')
            used_policy.add(e.name)
        # debug paths: names / calltrace, forced fallback, op_check,
        # statistics, input and output dumps
        boxed_args = f"c10::impl::boxArgs<{', '.join(boxed)}>({arg_names})" if boxed else \
            "torch::jit::Stack()"
        dbg = []
        dbg.append(f"    static const std::string kName = \"{e.name}\", kCpp = \"{fn}\";")
        dbg.append("    const auto& cfg = torch_gcu::OpDebugConfig::get();")
        dbg.append("    if (!torch_gcu::in_op_check()) torch_gcu::trace_call(kName, kCpp);")
        if e.fallback_cpu:
            dbg.append("    if (torch_gcu::forced_fallback(kName, kCpp)) {")
            dbg.append(f"      return {fallback_call};")
            dbg.append("    }")
        dbg.append(f"    static const auto op_ = c10::Dispatcher::singleton().findSchemaOrThrow(\"aten::{base}\", \"{overload}\");")
        if e.op_check:
            alias = _aliased_return_arg(schema)
            ret_ok = ret in ("at::Tensor",) or alias is not None
            if ret_ok:
                dbg.append("    if (!torch_gcu::in_op_check() && torch_gcu::checked(kName, kCpp)) {")
                dbg.append("      torch_gcu::OpCheckScope scope_;")
                dbg.append(f"      auto stack_ = {boxed_args};")
                # the native run inside re-enters this wrapper, which records
                # the call's statistics and dumps
                dbg.append("      torch_gcu::op_check_boxed(op_, &stack_, c10::DispatchKeySet(c10::DispatchKey::PrivateUse1), kCpp);")
                if alias is not None:
                    dbg.append(f"      return {alias};")
                else:
                    dbg.append("      return stack_.back().toTensor();")
                dbg.append("    }")
        dbg.append("    if (cfg.statistics) {")
        dbg.append(f"      const auto args_ = {boxed_args};")
        dbg.append("      torch_gcu::count_op(kName, false, &args_, &op_.schema());")
        dbg.append("    }")
        dbg.append("    const bool din_ = torch_gcu::dump_inputs(kName, kCpp);")
        dbg.append("    const bool dout_ = torch_gcu::dump_outputs(kName, kCpp);")
        dbg.append("    if (din_ || dout_) {")
        dbg.append(f"      if (din_) torch_gcu::dump_call(kCpp, \"input\", {boxed_args});")
        if ret == "void":
            dbg.append(f"      torch_gcu::aotops::{fn}({arg_names});")
            dbg.append("      torch_gcu::after_op();")
            dbg.append(f"      if (dout_) torch_gcu::dump_call(kCpp, \"output\", {boxed_args});")
            dbg.append("      return;")
        else:
            dbg.append(f"      {'auto&&' if '&' in ret else 'auto'} d_ = torch_gcu::aotops::{fn}({arg_names});")
            dbg.append("      torch_gcu::after_op();")
            dbg.append("      if (dout_) torch_gcu::dump_call(kCpp, \"output\", {c10::IValue(d_)});")
            dbg.append("      return d_;")
        dbg.append("    }")
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
        reg = (f"if (!torch_gcu::deregistered(\"{e.name}\", \"{fn}\")) "
               f"m.impl(\"{e.name}\", TORCH_FN(wrapper_PrivateUse1_{fn}));")
        if e.env_gate:
            regs.append(f"  if (torch_gcu::env_true(\"{e.env_gate}\")) {{ {reg} }}")
        else:
            regs.append(f"  {reg}")
    unused = set(policy) - used_policy
    assert not unused, (f"fallback policy names ops without a native kernel "
                        f"(they run on CPU anyway): {sorted(unused)}")

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
        + "\n".join(policy_regs + regs) + "\n}\n")
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
