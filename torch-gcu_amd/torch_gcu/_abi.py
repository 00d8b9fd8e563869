"""ctypes view of the gfx950 kernel library's C ABI (``include/mi355x_ops.h``).

This is the binding a Python caller of the library uses directly (the tests
and the benchmark call through it); the PrivateUse1 host in ``torch_gcu._C``
links the same library from C++.  Tensors handed to it must live on the GPU;
here that memory comes from any torch device tensor (``data_ptr``), and the
stream is passed explicitly.

Loading fails loudly when the library has not been built: there is no CPU
fallback behind this module.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Iterable, Optional, Sequence

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libmi355x_ops.so")

MI_MAX_DIMS = 8

MI_OK = 0
STATUS_NAMES = {0: "MI_OK", 1: "MI_ERR_INVALID", 2: "MI_ERR_UNSUPPORTED",
                3: "MI_ERR_WORKSPACE", 4: "MI_ERR_LAUNCH", 5: "MI_ERR_TOO_LARGE"}

# dtype codes equal c10::ScalarType's
DTYPE_CODES = {
    torch.uint8: 0, torch.int8: 1, torch.int16: 2, torch.int32: 3, torch.int64: 4,
    torch.float16: 5, torch.float32: 6, torch.float64: 7, torch.bool: 11,
    torch.bfloat16: 15,
}
MI_F64, MI_I64, MI_BOOL = 7, 4, 11


class MiTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("sizes", ctypes.c_int64 * MI_MAX_DIMS),
                ("strides", ctypes.c_int64 * MI_MAX_DIMS)]


class MiScalar(ctypes.Structure):
    _fields_ = [("f", ctypes.c_double), ("i", ctypes.c_int64), ("dtype", ctypes.c_int32),
                ("wrapped", ctypes.c_int32)]


class MiAdamwHparams(ctypes.Structure):
    _fields_ = [("lr", ctypes.c_double), ("beta1", ctypes.c_double), ("beta2", ctypes.c_double),
                ("weight_decay", ctypes.c_double), ("eps", ctypes.c_double),
                ("amsgrad", ctypes.c_int32), ("maximize", ctypes.c_int32)]


class MiError(RuntimeError):
    """A kernel-library call returned a status other than MI_OK."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} failed with {STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


_ALLOC_FN = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p)
_FREE_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p)

_T = ctypes.POINTER(MiTensor)
_S = ctypes.c_void_p
_SIGNATURES = {
    "mi_abi_version": ([], ctypes.c_int32),
    "mi_last_error": ([], ctypes.c_char_p),
    "mi_set_workspace_allocator": ([_ALLOC_FN, _FREE_FN, ctypes.c_void_p], ctypes.c_int),
    "mi_device_cu_count": ([], ctypes.c_int32),
    "mi_copy": ([_T, _T, _S], ctypes.c_int),
    "mi_fill": ([_T, MiScalar, _S], ctypes.c_int),
    "mi_cat": ([_T, ctypes.POINTER(_T), ctypes.c_int32, ctypes.c_int32, _S], ctypes.c_int),
    "mi_silu": ([_T, _T, _S], ctypes.c_int),
    "mi_silu_backward": ([_T, _T, _T, _S], ctypes.c_int),
    "mi_foreach_add_scalar": ([ctypes.POINTER(_T), ctypes.c_int32, ctypes.c_double, _S], ctypes.c_int),
    "mi_foreach_mul_scalar": ([ctypes.POINTER(_T), ctypes.c_int32, ctypes.c_double, _T, _S],
                              ctypes.c_int),
    "mi_amp_unscale": ([ctypes.POINTER(_T), ctypes.c_int32, _T, _T, _S], ctypes.c_int),
    "mi_amp_update_scale": ([_T, _T, _T, ctypes.c_double, ctypes.c_double, ctypes.c_int64, _S],
                            ctypes.c_int),
    "mi_log_softmax_backward": ([_T, _T, _T, ctypes.c_int64, _S], ctypes.c_int),
    "mi_softmax_backward": ([_T, _T, _T, ctypes.c_int64, _S], ctypes.c_int),
    "mi_layer_norm_backward": ([_T] * 8 + [ctypes.c_int64, _S], ctypes.c_int),
    "mi_layer_norm": ([_T] * 6 + [ctypes.c_int64, ctypes.c_double, _S], ctypes.c_int),
    "mi_fused_adamw": ([ctypes.POINTER(_T)] * 6 + [ctypes.c_int32, _T, ctypes.POINTER(MiAdamwHparams),
                                                   _T, _T, _S], ctypes.c_int),
    "mi_add": ([_T, _T, _T, MiScalar, _S], ctypes.c_int),
    "mi_sub": ([_T, _T, _T, MiScalar, _S], ctypes.c_int),
    "mi_mul": ([_T, _T, _T, _S], ctypes.c_int),
    "mi_div": ([_T, _T, _T, _S], ctypes.c_int),
    "mi_add_scalar": ([_T, _T, MiScalar, MiScalar, _S], ctypes.c_int),
    "mi_mul_scalar": ([_T, _T, MiScalar, _S], ctypes.c_int),
    "mi_div_scalar": ([_T, _T, MiScalar, _S], ctypes.c_int),
    "mi_index_select": ([_T, _T, ctypes.c_int64, _T, _S], ctypes.c_int),
    "mi_index": ([_T, _T, ctypes.POINTER(_T), ctypes.c_int32, _S], ctypes.c_int),
    "mi_index_fault_take": ([ctypes.c_int32, ctypes.POINTER(ctypes.c_int64),
                             ctypes.POINTER(ctypes.c_int64)], ctypes.c_int32),
    "mi_sum": ([_T, _T, ctypes.POINTER(ctypes.c_int64), ctypes.c_int32, ctypes.c_int32, _S],
               ctypes.c_int),
    "mi_amax": ([_T, _T, ctypes.POINTER(ctypes.c_int64), ctypes.c_int32, ctypes.c_int32, _S],
                ctypes.c_int),
    "mi_mean": ([_T, _T, ctypes.POINTER(ctypes.c_int64), ctypes.c_int32, ctypes.c_int32, _S],
                ctypes.c_int),
    "mi_mean_noalloc": ([_T, _T, ctypes.POINTER(ctypes.c_int64), ctypes.c_int32, ctypes.c_int32,
                         _S], ctypes.c_int),
    "mi_softmax": ([_T, _T, ctypes.c_int64, _S], ctypes.c_int),
    "mi_log_softmax": ([_T, _T, ctypes.c_int64, _S], ctypes.c_int),
    "mi_rms_norm": ([_T, _T, _T, ctypes.c_double, _S], ctypes.c_int),
    "mi_rope": ([_T, _T, _T, _T, _T, ctypes.c_double, _S], ctypes.c_int),
    "mi_silu_mul": ([_T, _T, _T, _S], ctypes.c_int),
    "mi_addmm": ([_T, _T, _T, _T, ctypes.c_double, ctypes.c_double, _S], ctypes.c_int),
    "mi_addmv": ([_T, _T, _T, _T, ctypes.c_double, ctypes.c_double, _S], ctypes.c_int),
    "mi_mm": ([_T, _T, _T, _S], ctypes.c_int),
    "mi_bmm": ([_T, _T, _T, _S], ctypes.c_int),
    "mi_baddbmm": ([_T, _T, _T, _T, ctypes.c_double, ctypes.c_double, _S], ctypes.c_int),
    "mi_int8_linear": ([_T, _T, _T, _T, _T, _S], ctypes.c_int),
    "mi_linear_residual": ([_T, _T, _T, _T, _S], ctypes.c_int),
    "mi_linear_silu_mul": ([_T, _T, _T, _T, _S], ctypes.c_int),
    "mi_flash_attention_fwd": ([_T, _T, _T, _T, _T, ctypes.c_int32, ctypes.c_double, _S],
                               ctypes.c_int),
}

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()


def library_path() -> str:
    return _LIB_PATH


def declared_symbols() -> list[str]:
    return sorted(_SIGNATURES)


def lib() -> ctypes.CDLL:
    """Loads the kernel library (torch is imported first so that the HIP
    runtime torch ships is the one the library binds to)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise RuntimeError(
                    f"kernel library not built: {_LIB_PATH} is missing "
                    "(run `python torch-gcu_amd/build.py`)")
            handle = ctypes.CDLL(_LIB_PATH, mode=ctypes.RTLD_GLOBAL)
            for name, (args, res) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.argtypes = args
                fn.restype = res
            _lib = handle
        return _lib


def runtime_info() -> dict:
    """Which HIP runtime the loaded kernel library resolved: the paths of
    every libamdhip64 mapped into this process (torch's bundled copy and the
    library share one when they bind to the same file) and that runtime's
    hipRuntimeGetVersion."""
    lib()
    with open("/proc/self/maps") as f:
        paths = sorted({line.split()[-1] for line in f
                        if "libamdhip64" in line and line.split()[-1].startswith("/")})
    version = None
    if paths:
        v = ctypes.c_int(0)
        if ctypes.CDLL(paths[0]).hipRuntimeGetVersion(ctypes.byref(v)) == 0:
            version = v.value
    return {"libamdhip64": paths, "hip_runtime_version": version}


# ---- descriptors ---------------------------------------------------------------

def desc(t: Optional[torch.Tensor]) -> MiTensor:
    d = MiTensor()
    if t is None:
        return d
    if t.dim() > MI_MAX_DIMS:
        raise ValueError(f"tensor rank {t.dim()} exceeds {MI_MAX_DIMS}")
    d.data = t.data_ptr() if t.numel() > 0 else None
    d.dtype = DTYPE_CODES[t.dtype]
    d.ndim = t.dim()
    for i, (s, st) in enumerate(zip(t.shape, t.stride())):
        d.sizes[i] = s
        d.strides[i] = st
    return d


def scalar(v, dtype: Optional[torch.dtype] = None, wrapped: bool = True) -> MiScalar:
    s = MiScalar()
    if dtype is None:
        if isinstance(v, bool):
            dtype = torch.bool
        elif isinstance(v, int):
            dtype = torch.int64
        else:
            dtype = torch.float64
    s.dtype = DTYPE_CODES[dtype]
    if dtype.is_floating_point:
        s.f = float(v)
    else:
        s.i = int(v)
    s.wrapped = 1 if wrapped else 0
    return s


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def check(fn: str, status: int) -> None:
    if status != MI_OK:
        raise MiError(fn, status, lib().mi_last_error().decode(errors="replace"))


# ---- workspace ------------------------------------------------------------------

def install_workspace() -> None:
    """Registers the gcu caching allocator (torch_gcu._C) as the library's
    stream-ordered workspace allocator; direct C-ABI callers need it for the
    entry points that take temporary memory (split reductions)."""
    from . import _C

    _C._init()


# ---- thin op wrappers (out tensors are preallocated by the caller) --------------

def _dims(dims: Sequence[int]):
    arr = (ctypes.c_int64 * max(1, len(dims)))(*dims)
    return arr, len(dims)


def copy_(out, src):
    check("mi_copy", lib().mi_copy(desc(out), desc(src), stream_of(out)))
    return out


def cat(out, inputs, dim):
    """out = cat(inputs, dim) through mi_cat; every input has out's rank."""
    descs = [desc(t) for t in inputs]  # kept alive for the call
    arr = (_T * max(1, len(descs)))(*[ctypes.pointer(d) for d in descs])
    check("mi_cat", lib().mi_cat(desc(out), arr, len(descs), dim, stream_of(out)))
    return out


def fused_adamw(params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, *, lr,
                beta1, beta2, weight_decay, eps, amsgrad=False, maximize=False, grad_scale=None,
                found_inf=None):
    """One AdamW step in place through mi_fused_adamw; lr is a float or a
    one-element device tensor."""
    n = len(params)

    def arr(lst):
        if lst is None or len(lst) == 0:
            return None, []
        ds = [desc(t) for t in lst]
        return (_T * len(ds))(*[ctypes.pointer(d) for d in ds]), ds

    keep = []
    arrays = []
    for lst in (params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs if amsgrad else None,
                state_steps):
        a, ds = arr(lst)
        keep.append(ds)
        arrays.append(a)
    hp = MiAdamwHparams(lr if not isinstance(lr, torch.Tensor) else 0.0, beta1, beta2,
                        weight_decay, eps, int(amsgrad), int(maximize))
    lr_d = desc(lr) if isinstance(lr, torch.Tensor) else None
    gs_d = desc(grad_scale) if grad_scale is not None else None
    fi_d = desc(found_inf) if found_inf is not None else None
    check("mi_fused_adamw", lib().mi_fused_adamw(
        *arrays, n, lr_d, ctypes.byref(hp), gs_d, fi_d,
        stream_of(params[0]) if n else torch.cuda.current_stream().cuda_stream))


def foreach_add_scalar_(tensors, value):
    """Every tensor += value, in place, through mi_foreach_add_scalar."""
    ds = [desc(t) for t in tensors]
    arr = (_T * max(1, len(ds)))(*[ctypes.pointer(d) for d in ds])
    check("mi_foreach_add_scalar", lib().mi_foreach_add_scalar(
        arr, len(ds), value, stream_of(tensors[0]) if tensors else torch.cuda.current_stream().cuda_stream))
    return tensors


def foreach_mul_scalar_(tensors, value=0.0, scalar=None):
    """Every tensor *= value (or the one-element fp32 device tensor `scalar`)."""
    ds = [desc(t) for t in tensors]
    arr = (_T * max(1, len(ds)))(*[ctypes.pointer(d) for d in ds])
    sd = desc(scalar) if scalar is not None else None
    check("mi_foreach_mul_scalar", lib().mi_foreach_mul_scalar(
        arr, len(ds), float(value), sd, stream_of(tensors[0]) if tensors else None))
    return tensors


def amp_unscale_(tensors, found_inf, inv_scale):
    """GradScaler's unscale and inf / NaN check through mi_amp_unscale."""
    ds = [desc(t) for t in tensors]
    arr = (_T * max(1, len(ds)))(*[ctypes.pointer(d) for d in ds])
    check("mi_amp_unscale", lib().mi_amp_unscale(arr, len(ds), desc(found_inf), desc(inv_scale),
                                                 stream_of(found_inf)))
    return tensors


def amp_update_scale_(scale, growth_tracker, found_inf, growth_factor, backoff_factor, interval):
    """GradScaler's scale update through mi_amp_update_scale."""
    check("mi_amp_update_scale", lib().mi_amp_update_scale(
        desc(scale), desc(growth_tracker), desc(found_inf), float(growth_factor),
        float(backoff_factor), int(interval), stream_of(scale)))
    return scale


def silu(out, self):
    check("mi_silu", lib().mi_silu(desc(out), desc(self), stream_of(out)))
    return out


def silu_backward(grad_input, grad_output, self):
    check("mi_silu_backward", lib().mi_silu_backward(desc(grad_input), desc(grad_output), desc(self),
                                                     stream_of(grad_input)))
    return grad_input


def log_softmax_backward(grad_input, grad_output, output, dim):
    check("mi_log_softmax_backward", lib().mi_log_softmax_backward(
        desc(grad_input), desc(grad_output), desc(output), dim, stream_of(grad_input)))
    return grad_input


def softmax_backward(grad_input, grad_output, output, dim):
    check("mi_softmax_backward", lib().mi_softmax_backward(
        desc(grad_input), desc(grad_output), desc(output), dim, stream_of(grad_input)))
    return grad_input


def layer_norm(out, mean, rstd, x, weight, bias, normalized_numel, eps):
    """weight and bias may be None."""
    check("mi_layer_norm", lib().mi_layer_norm(
        desc(out), desc(mean), desc(rstd), desc(x), desc(weight) if weight is not None else None,
        desc(bias) if bias is not None else None, normalized_numel, eps, stream_of(x)))
    return out


def layer_norm_backward(grad_input, grad_weight, grad_bias, grad_out, x, mean, rstd, weight,
                        normalized_numel):
    """Any of grad_input / grad_weight / grad_bias / weight may be None."""
    opt = [desc(t) if t is not None else None for t in (grad_input, grad_weight, grad_bias)]
    check("mi_layer_norm_backward", lib().mi_layer_norm_backward(
        *opt, desc(grad_out), desc(x), desc(mean), desc(rstd),
        desc(weight) if weight is not None else None, normalized_numel, stream_of(x)))


def fill_(out, value, dtype=None):
    check("mi_fill", lib().mi_fill(desc(out), scalar(value, dtype), stream_of(out)))
    return out


def add(out, a, b, alpha=1):
    if isinstance(b, torch.Tensor):
        check("mi_add", lib().mi_add(desc(out), desc(a), desc(b), scalar(alpha), stream_of(out)))
    else:
        check("mi_add_scalar",
              lib().mi_add_scalar(desc(out), desc(a), scalar(b), scalar(alpha), stream_of(out)))
    return out


def sub(out, a, b, alpha=1):
    if isinstance(b, torch.Tensor):
        check("mi_sub", lib().mi_sub(desc(out), desc(a), desc(b), scalar(alpha), stream_of(out)))
    else:
        check("mi_add_scalar",
              lib().mi_add_scalar(desc(out), desc(a), scalar(b), scalar(-alpha), stream_of(out)))
    return out


def mul(out, a, b):
    if isinstance(b, torch.Tensor):
        check("mi_mul", lib().mi_mul(desc(out), desc(a), desc(b), stream_of(out)))
    else:
        check("mi_mul_scalar", lib().mi_mul_scalar(desc(out), desc(a), scalar(b), stream_of(out)))
    return out


def div(out, a, b):
    if isinstance(b, torch.Tensor):
        check("mi_div", lib().mi_div(desc(out), desc(a), desc(b), stream_of(out)))
    else:
        check("mi_div_scalar", lib().mi_div_scalar(desc(out), desc(a), scalar(b), stream_of(out)))
    return out


def index_select(out, self, dim, index):
    check("mi_index_select",
          lib().mi_index_select(desc(out), desc(self), dim, desc(index), stream_of(out)))
    return out


def index(out, self, indices):
    """out = self[indices] through mi_index; indices is a list (one entry per
    leading dim of self, None for a dim taken whole) of int32/int64 device
    tensors already broadcast to one shape."""
    descs = [None if t is None else desc(t) for t in indices]
    arr = (_T * max(1, len(descs)))(*[None if d is None else ctypes.pointer(d) for d in descs])
    check("mi_index", lib().mi_index(desc(out), desc(self), arr, len(descs), stream_of(out)))
    return out


def _reduce(name, out, self, dims, keepdim):
    arr, n = _dims(list(dims))
    check(name, getattr(lib(), name)(desc(out), desc(self), arr, n, int(keepdim),
                                     stream_of(out)))
    return out


def sum_(out, self, dims: Iterable[int] = (), keepdim=False):
    return _reduce("mi_sum", out, self, dims, keepdim)


def amax(out, self, dims: Iterable[int] = (), keepdim=False):
    return _reduce("mi_amax", out, self, dims, keepdim)


def mean(out, self, dims: Iterable[int] = (), keepdim=False):
    return _reduce("mi_mean", out, self, dims, keepdim)


def mean_noalloc(out, self, dims: Iterable[int] = (), keepdim=False):
    """mi_mean_noalloc: mean with its temporary memory in the library's
    static per-GPU scratch (no allocation)."""
    return _reduce("mi_mean_noalloc", out, self, dims, keepdim)


def index_fault_take(device: int = 0):
    """mi_index_fault_take: (index, dim size) of an out-of-range index the
    gather kernels met on `device` since the last call, or None; clears it.
    Call after synchronising with the work."""
    idx, size = ctypes.c_int64(0), ctypes.c_int64(0)
    if lib().mi_index_fault_take(device, ctypes.byref(idx), ctypes.byref(size)):
        return idx.value, size.value
    return None


def softmax(out, self, dim):
    check("mi_softmax", lib().mi_softmax(desc(out), desc(self), dim, stream_of(out)))
    return out


def log_softmax(out, self, dim):
    check("mi_log_softmax", lib().mi_log_softmax(desc(out), desc(self), dim, stream_of(out)))
    return out


def rms_norm(out, x, weight, eps):
    check("mi_rms_norm", lib().mi_rms_norm(desc(out), desc(x), desc(weight), eps, stream_of(out)))
    return out


def rope(q_out, k_out, q, k, positions, theta):
    check("mi_rope", lib().mi_rope(desc(q_out), desc(k_out), desc(q), desc(k), desc(positions),
                                   theta, stream_of(q_out)))
    return q_out, k_out


def silu_mul(out, gate, up):
    check("mi_silu_mul", lib().mi_silu_mul(desc(out), desc(gate), desc(up), stream_of(out)))
    return out


def addmm(out, bias, a, b, beta=1.0, alpha=1.0):
    check("mi_addmm", lib().mi_addmm(desc(out), desc(bias), desc(a), desc(b), beta, alpha,
                                     stream_of(out)))
    return out


def addmv(out, bias, mat, vec, beta=1.0, alpha=1.0):
    check("mi_addmv", lib().mi_addmv(desc(out), desc(bias), desc(mat), desc(vec), beta, alpha,
                                     stream_of(out)))
    return out


def mm(out, a, b):
    check("mi_mm", lib().mi_mm(desc(out), desc(a), desc(b), stream_of(out)))
    return out


def bmm(out, a, b):
    check("mi_bmm", lib().mi_bmm(desc(out), desc(a), desc(b), stream_of(out)))
    return out


def baddbmm(out, bias, a, b, beta=1.0, alpha=1.0):
    check("mi_baddbmm", lib().mi_baddbmm(desc(out), desc(bias), desc(a), desc(b), beta, alpha,
                                         stream_of(out)))
    return out


def int8_linear(out, x, weight, scales, bias=None):
    check("mi_int8_linear", lib().mi_int8_linear(desc(out), desc(x), desc(weight), desc(scales),
                                                 desc(bias), stream_of(out)))
    return out


def linear_residual(out, x, weight, residual):
    check("mi_linear_residual", lib().mi_linear_residual(desc(out), desc(x), desc(weight),
                                                         desc(residual), stream_of(out)))
    return out


def linear_silu_mul(out, x, w_gate, w_up):
    check("mi_linear_silu_mul", lib().mi_linear_silu_mul(desc(out), desc(x), desc(w_gate),
                                                         desc(w_up), stream_of(out)))
    return out


def flash_attention_fwd(out, lse, q, k, v, is_causal=True, scale=None):
    if scale is None:
        scale = q.shape[-1] ** -0.5
    check("mi_flash_attention_fwd",
          lib().mi_flash_attention_fwd(desc(out), desc(lse), desc(q), desc(k), desc(v),
                                       int(is_causal), float(scale), stream_of(out)))
    return out
