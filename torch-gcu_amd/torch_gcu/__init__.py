"""torch_gcu for MI355X: the "gcu" PrivateUse1 device backed by hand-written
gfx950 HIP kernels.

Importing the package loads the kernel library (``torch_gcu._abi``).  The
PrivateUse1 host extension (``torch_gcu._C``) is loaded by
``torch_gcu._backend``.
"""
from . import _abi  # noqa: F401

__all__ = ["_abi"]
