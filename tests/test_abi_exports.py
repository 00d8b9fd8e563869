"""The kernel library loads and exports every entry point its header declares
(CPU only: no compute call is made)."""
import os
import re
import subprocess

from torch_gcu import _abi

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER_DIR = os.path.join(REPO, "include")


def declared_in_headers():
    names = set()
    decl = re.compile(r"^\s*(?:const\s+)?\w+\**\s+\**(mi_\w+)\s*\(", re.M)
    for f in os.listdir(HEADER_DIR):
        if f.endswith(".h"):
            names.update(decl.findall(open(os.path.join(HEADER_DIR, f)).read()))
    return names


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", _abi.library_path()],
                         capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_header_declares_entry_points():
    names = declared_in_headers()
    assert {"mi_add", "mi_mul", "mi_index_select", "mi_log_softmax", "mi_rms_norm"} <= names


def test_library_exports_every_declared_symbol():
    missing = declared_in_headers() - exported()
    assert not missing, f"declared but not exported: {sorted(missing)}"


def test_ctypes_binding_covers_header():
    assert set(_abi.declared_symbols()) == declared_in_headers()


def test_library_loads_and_reports_version():
    lib = _abi.lib()
    v = lib.mi_abi_version()
    assert v >> 16 == 1
    assert lib.mi_last_error() == b""


def test_invalid_arguments_fail_without_gpu():
    # argument validation runs before any device call
    import torch
    t = _abi.MiTensor()
    t.ndim = 99
    st = _abi.lib().mi_copy(t, t, None)
    assert st == 1
    assert b"ndim" in _abi.lib().mi_last_error()
    x = _abi.desc(torch.empty(0))
    st = _abi.lib().mi_index_select(x, x, 0, _abi.desc(torch.empty(2, 2, dtype=torch.int64)), None)
    assert st == 1 and b"vector" in _abi.lib().mi_last_error()
