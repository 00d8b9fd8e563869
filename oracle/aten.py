"""The reference's own CPU path for each op: CPU ATen.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Each function takes CPU tensors and returns CPU tensors; the caller copies
device inputs to the host first, exactly as the boxed fallback does
(torch_gcu/csrc/aten/aten_cpu_fallback.cpp:342-411 -> at::native::cpu_fallback
at :390, results copied back by copy_back_to_org_device).  For the fused ops
that have no reference counterpart (RMSNorm, RoPE, SiLU-mul, int8
weight-only linear) the oracle is the fp32 closed form built from CPU ATen
ops, as the north_star defines them.
"""
from __future__ import annotations

import torch


# ---- config 1: elementwise and indexing ---------------------------------------

def mul(a: torch.Tensor, b) -> torch.Tensor:
    """aten::mul.out -> topsatenMul (codegen/gcu_native_functions.yaml:461).
    Pinned by numpy float32 multiply (bit-exact) in tests/test_oracle.py."""
    return torch.mul(a, b)


def add(a: torch.Tensor, b, alpha=1) -> torch.Tensor:
    """aten::add.out -> topsatenAdd (yaml :202); a CPU scalar operand takes the
    RHS_IS_SCALAR branch (codegen/gen_backend_stubs.py:1061-1078).
    Pinned by numpy float32 add (bit-exact)."""
    return torch.add(a, b, alpha=alpha)


def sub(a, b, alpha=1):
    """aten::sub.out (sub is add with -alpha).  Pinned by numpy."""
    return torch.sub(a, b, alpha=alpha)


def div(a, b):
    """aten::div.out, true division.  Pinned by numpy float32 divide."""
    return torch.div(a, b)


def index_select(self: torch.Tensor, dim: int, index: torch.Tensor) -> torch.Tensor:
    """aten::index_select -> topsatenIndexSelect (yaml :377-380; shape rules
    torch_gcu/csrc/aten/shape_inference/indexing.cpp:20-69).
    Pinned by numpy.take (bit-exact) and brute force on tiny inputs."""
    return torch.index_select(self, dim, index)


# ---- copy and transfer -----------------------------------------------------------

def copy(dst: torch.Tensor, src: torch.Tensor) -> torch.Tensor:
    """aten::copy_ into a tensor shaped and typed like dst: src broadcast to
    dst's shape and cast to its dtype (the reference's _copy_from,
    torch_gcu/csrc/aten/aot_ops/gcu_copy.cpp:279-386, device side topsatenCopy
    :116-150).  Pinned by numpy astype / broadcast_to (bit-exact)."""
    out = torch.empty_like(dst)
    out.copy_(src)
    return out


def cat(tensors, dim: int = 0) -> torch.Tensor:
    """aten::cat.out -> topsatenCat (codegen/gcu_native_functions.yaml:263):
    result_type promotion, legacy 1-D empty inputs skipped.  Pinned by
    numpy.concatenate and a brute-force walk over output positions."""
    return torch.cat(list(tensors), dim)


# ---- config 2: reductions and softmax --------------------------------------

def sum_(x: torch.Tensor, dim=None, keepdim=False, dtype=None) -> torch.Tensor:
    """aten::sum.IntList_out -> topsatenSum (yaml :576), fp32 accumulation for
    bf16.  Pinned by float64 numpy sums within the fp32/bf16 bars and by the
    constant-row closed form N*c."""
    if dim is None:
        return torch.sum(x, dtype=dtype)
    return torch.sum(x, dim=dim, keepdim=keepdim, dtype=dtype)


def amax(x: torch.Tensor, dim=(), keepdim=False) -> torch.Tensor:
    """aten::amax.out -> topsatenAmax (yaml :209).  Order independent, so
    exact.  Pinned by numpy.max (bit-exact) and the single-spike row."""
    return torch.amax(x, dim=dim, keepdim=keepdim)


def mean(x: torch.Tensor, dim=None, keepdim=False) -> torch.Tensor:
    """aten::mean.out -> topsatenMean (yaml :445).  Pinned by float64 numpy."""
    if dim is None:
        return torch.mean(x)
    return torch.mean(x, dim=dim, keepdim=keepdim)


def log_softmax(x: torch.Tensor, dim: int, half_to_float: bool = False) -> torch.Tensor:
    """aten::_log_softmax.out -> topsatenLogSoftmaxForward (yaml :155-156).
    Pinned by a float64 numpy log-sum-exp, the constant-row value -ln(N) and
    the invariant logsumexp(out) == 0."""
    if half_to_float:  # CPU ATen has no half_to_float kernel; the upcast is exact
        return torch._log_softmax(x.float(), dim, False)
    return torch._log_softmax(x, dim, half_to_float)


def softmax(x: torch.Tensor, dim: int, half_to_float: bool = False) -> torch.Tensor:
    """aten::_softmax.out -> topsatenSoftmaxForward (yaml :182-183).
    Pinned by float64 numpy and the invariant sum(out) == 1."""
    if half_to_float:
        return torch._softmax(x.float(), dim, False)
    return torch._softmax(x, dim, half_to_float)


# ---- config 3: fused efficient ops (fp32 closed forms) -------------------------

def rms_norm(x: torch.Tensor, w, eps: float) -> torch.Tensor:
    """y = x * rsqrt(mean(x^2) + eps) * w in fp32, one cast to x.dtype.
    torch.rms_norm's CPU kernel computes exactly this for bf16 (checked
    bit-exact in tests/test_oracle.py).  Pinned by float64 numpy and the
    golden fixture tests/golden/rms_norm.npz."""
    xf = x.float()
    r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    y = xf * r
    if w is not None:
        y = y * w.float()
    return y.to(x.dtype)


def rope_tables(positions: torch.Tensor, head_dim: int, theta: float):
    """fp32 cos/sin of pos * inv_freq, inv_freq = 1 / theta^(2i/d), i < d/2
    (the rotate-half convention used by HF/NeoX Llama)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = positions.float()[:, None] * inv_freq[None, :]
    return freqs.cos(), freqs.sin()


def rope(x: torch.Tensor, positions: torch.Tensor, theta: float) -> torch.Tensor:
    """Rotate-half RoPE on [tokens, heads, head_dim] in fp32:
    out[..., :h] = x1*cos - x2*sin, out[..., h:] = x2*cos + x1*sin.
    Pinned by the invariants (position 0 is the identity, pair norms are
    preserved), float64 numpy and tests/golden/rope.npz."""
    d = x.shape[-1]
    h = d // 2
    cos, sin = rope_tables(positions, d, theta)
    cos = cos[:, None, :]
    sin = sin[:, None, :]
    xf = x.float()
    x1, x2 = xf[..., :h], xf[..., h:]
    out = torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)
    return out.to(x.dtype)


def addmm(bias, a, b, beta=1.0, alpha=1.0):
    """aten::addmm.out -> topsatenAddmm (yaml :205), as the fp32 closed form
    beta*bias + alpha*(a @ b) over upcast inputs with one cast to a.dtype
    (CPU ATen's bf16 addmm accumulates in fp32 too).  Pinned by float64
    numpy matmul and the row-sampling identity C[rows] = A[rows] @ B."""
    out = (a.float() @ b.float()) * alpha
    if bias is not None and beta != 0:
        out = out + beta * bias.float()
    return out.to(a.dtype)


def addmv(bias, mat, vec, beta=1.0, alpha=1.0):
    """aten::addmv.out -> topsatenAddmv (yaml :206): CPU ATen's addmv (the
    reference's fallback path), fp32 for bf16/fp16 inputs then one cast, as
    its bf16 gemv accumulates in fp32.  bias None means beta = 0 (mv).
    Pinned by a float64 numpy product, alpha = 0 and beta = 0 ignoring NaN
    operands, and mv == addmv with beta = 0."""
    lowp = mat.dtype in (torch.bfloat16, torch.float16)
    m, v = (mat.float(), vec.float()) if lowp else (mat, vec)
    b = torch.zeros(mat.shape[0], dtype=m.dtype) if bias is None else bias.to(m.dtype)
    out = torch.addmv(b, m, v, beta=beta if bias is not None else 0.0, alpha=alpha)
    return out.to(mat.dtype)


def bmm(a, b):
    """aten::bmm.out -> topsatenBmm (yaml :260), fp32 closed form."""
    return torch.bmm(a.float(), b.float()).to(a.dtype)


def sdpa(q, k, v, is_causal=False, scale=None):
    """Scaled dot-product attention as CPU ATen runs it for [B, H, S, D]
    inputs: _scaled_dot_product_flash_attention_for_cpu (the CPU kernel
    F.scaled_dot_product_attention selects; for bf16 it rounds the softmax
    weights to bf16 before the P V product, as GPU flash kernels do).  k/v
    heads are repeated to the query heads when fewer.  Returns (out, lse).
    The reference reaches attention through _scaled_dot_product_flash_attention
    (torch_gcu/csrc/aten/GCUNativeFunctions.cpp:49-102).  Pinned by the fp32
    closed form softmax(scale q k^T + mask) v in tests/test_oracle.py."""
    H, Hk = q.shape[1], k.shape[1]
    if Hk != H:
        k = k.repeat_interleave(H // Hk, dim=1)
        v = v.repeat_interleave(H // Hk, dim=1)
    out, lse = torch.ops.aten._scaled_dot_product_flash_attention_for_cpu(
        q, k, v, 0.0, is_causal, scale=scale)
    return out, lse


def int8_linear(x, w, scales, bias=None):
    """int8 weight-only linear, fp32 closed form (x @ W^T) * scales (+ bias)
    with one cast; new efficient op, no reference counterpart.  Pinned by
    float64 numpy and by aten::_weight_int8pack_mm with bf16 scales."""
    y = (x.float() @ w.float().t()) * scales.float()
    if bias is not None:
        y = y + bias.float()
    return y.to(x.dtype)


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up in fp32, one cast (the reference would run silu.out,
    yaml :561, then mul.out).  Pinned by float64 numpy and
    tests/golden/silu_mul.npz."""
    return (torch.nn.functional.silu(gate.float()) * up.float()).to(gate.dtype)


# ---- training-side neighbours -------------------------------------------------------

def fused_adamw(params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, *, lr,
                beta1, beta2, weight_decay, eps, amsgrad, maximize, grad_scale=None,
                found_inf=None):
    """aten::_fused_adamw_ -> topsatenFusedAdamw (codegen/gcu_native_functions.yaml:144-145,
    torch_gcu/csrc/aten/aot_ops/_fused_adamw_.cpp:15-52): CPU ATen's fused AdamW
    run on clones.  Returns the updated (params, grads, exp_avgs, exp_avg_sqs,
    max_exp_avg_sqs).  Pinned by the float64 AdamW closed form
    (numpy_ref.adamw64) and its planted-mistake variant."""
    c = [[t.clone() for t in lst] for lst in (params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs)]
    torch._fused_adamw_(*c, [s.clone() for s in state_steps], lr=lr, beta1=beta1, beta2=beta2,
                        weight_decay=weight_decay, eps=eps, amsgrad=amsgrad, maximize=maximize,
                        grad_scale=grad_scale, found_inf=found_inf)
    return c


def silu_backward(grad_output, x):
    """aten::silu_backward -> topsatenSiluBackward (yaml silu_backward.grad_input :563),
    sent to CPU on s60 (codegen/gcu_op_fallback.yaml:22-25).  Pinned by the
    float64 closed form s * (1 + x * (1 - s)) and a central difference of silu."""
    return torch.ops.aten.silu_backward(grad_output, x)


def log_softmax_backward(grad_output, output, dim, input_dtype):
    """aten::_log_softmax_backward_data (yaml :157; s60 fallback list).  Pinned
    by float64 dy - exp(y) * sum(dy) and a central difference of log_softmax."""
    return torch.ops.aten._log_softmax_backward_data(grad_output, output, dim, input_dtype)


def softmax_backward(grad_output, output, dim, input_dtype):
    """aten::_softmax_backward_data (yaml :184; s60 fallback list).  Pinned by
    float64 y * (dy - sum(dy * y))."""
    return torch.ops.aten._softmax_backward_data(grad_output, output, dim, input_dtype)


def layer_norm_forward(x, normalized_shape, weight, bias, eps):
    """aten::native_layer_norm on CPU: (out, mean, rstd), the inputs of the backward."""
    return torch.native_layer_norm(x, normalized_shape, weight, bias, eps)


def layer_norm_backward(grad_out, x, normalized_shape, mean, rstd, weight, bias, mask):
    """aten::native_layer_norm_backward -> topsatenNativeLayerNormBackward
    (yaml :483; s60 fallback list).  Pinned by the float64 closed form of
    numpy_ref.layer_norm_backward64 and central differences of layer norm."""
    return torch.ops.aten.native_layer_norm_backward(grad_out, x, normalized_shape, mean, rstd,
                                                     weight, bias, mask)


def foreach_add_scalar(tensors, value):
    """aten::_foreach_add_.Scalar -> the generated foreach add
    (codegen/gcu_native_functions.yaml:47): CPU ATen on clones; each element
    plus the scalar in the op-math type (float for 16-bit inputs), rounded
    once.  Pinned by the numpy float32 sum rounded to the dtype and by
    x + 0 == x."""
    c = [t.clone() for t in tensors]
    torch._foreach_add_(c, value)
    return c


def foreach_mul(tensors, other):
    """aten::_foreach_mul_.Scalar / .Tensor (codegen/gcu_native_functions.yaml:131,
    :133): CPU ATen on clones.  Pinned by the numpy float32 product rounded to
    the dtype, x * 1 == x and x * -1 == -x."""
    c = [t.clone() for t in tensors]
    torch._foreach_mul_(c, other)
    return c


def amp_unscale(grads, found_inf, inv_scale):
    """aten::_amp_foreach_non_finite_check_and_unscale_
    (codegen/gcu_native_functions.yaml:15): CPU ATen on clones; returns
    (unscaled grads, found_inf).  Pinned by the numpy float32 product
    rounded to the dtype, the inv_scale == 1 identity, and found_inf being 1
    exactly when some element is inf or NaN."""
    c = [t.clone() for t in grads]
    fi = found_inf.clone()
    torch._amp_foreach_non_finite_check_and_unscale_(c, fi, inv_scale)
    return c, fi


def amp_update_scale(scale, growth_tracker, found_inf, growth_factor, backoff_factor,
                     growth_interval):
    """aten::_amp_update_scale_ (codegen/gcu_native_functions.yaml:16): CPU ATen
    on clones; returns (scale, growth_tracker).  Pinned by the state machine
    of numpy_ref.amp_update_scale_ref and hand-worked step sequences."""
    s, t = scale.clone(), growth_tracker.clone()
    torch._amp_update_scale_(s, t, found_inf, growth_factor, backoff_factor, growth_interval)
    return s, t


def int32_indices_index(self, indices):
    """The efficient op device_int32_indices_index
    (torch_gcu/csrc/efficient_ops/ops.cpp:335-342; gcu/efficient/op.py:8-16):
    CPU ATen's aten::index with the int32 indices widened to int64 (the same
    values).  Pinned by numpy advanced indexing (which places the broadcast
    index dims by the same adjacent / non-adjacent rule) and by a brute-force
    walk over output positions."""
    return torch.ops.aten.index(self, [None if i is None else i.long() for i in indices])


def widened_fallback(fn, *args, **kwargs):
    """The CPU fallback of an op whose CPU kernel lacks a 16-bit float dtype
    (torch_gcu/csrc/aten/aten_cpu_fallback.cpp:193-340): every tensor of that
    dtype widened to float32, the op run on CPU ATen, and the tensor results
    rounded back to the 16-bit dtype.  Pinned by float64 closed forms (a
    diagonal sum, scipy's erfcx) rounded to the 16-bit dtype."""
    low = next(a.dtype for a in args
               if isinstance(a, torch.Tensor) and a.dtype in (torch.float16, torch.bfloat16))
    wide = [a.float() if isinstance(a, torch.Tensor) and a.dtype == low else a for a in args]
    out = fn(*wide, **kwargs)
    if isinstance(out, torch.Tensor):
        return out.to(low) if out.dtype == torch.float32 else out
    return type(out)(o.to(low) if isinstance(o, torch.Tensor) and o.dtype == torch.float32 else o
                     for o in out)
