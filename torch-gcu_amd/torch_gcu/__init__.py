"""torch_gcu for MI355X: the "gcu" PrivateUse1 device, backed by hand-written
gfx950 HIP kernels.

``import torch_gcu`` loads the C++ host (``torch_gcu._C``: runtime, caching
allocator, GCUGraph, the generated aten registrations and the efficient ops)
and the kernel library it links, renames PrivateUse1 to "gcu" and installs
``torch.gcu`` -- the same steps as the reference's package init
(torch_gcu/__init__.py:11-16 and :79-106).  There is no fallback when the
extension is missing: the import fails.
"""
import os as _os

import torch as _torch

from . import _abi  # noqa: F401  (kernel library; loaded first)

try:
    from . import _C  # noqa: F401
except ImportError as _e:  # pragma: no cover - exercised only on a broken install
    raise ImportError(
        "torch_gcu._C is not built (run `python torch-gcu_amd/build.py`): " + str(_e)) from _e

_torch.utils.rename_privateuse1_backend("gcu")

from . import gcu  # noqa: E402

_torch._register_device_module("gcu", gcu)
_torch.utils.generate_methods_for_privateuse1_backend(for_tensor=True, for_module=True,
                                                      for_storage=True)
_C._init()

from .gcu import efficient  # noqa: E402,F401

if _C._op_debug_config()["op_statistics_dump"]:
    # op_statistics_dump=true: the statistics are written at exit
    # (the reference dumps them when its statistics object is destroyed)
    import atexit as _atexit

    _atexit.register(_C._dump_op_statistics_to_json)

__all__ = ["gcu", "efficient"]
