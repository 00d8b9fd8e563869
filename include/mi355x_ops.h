/*
 * mi355x_ops.h -- C ABI of the gfx950 (MI355X) kernel library behind the
 * torch_gcu PrivateUse1 op path.
 *
 * This library takes the place of the closed TopsAten kernel library that the
 * reference reaches through its bridge templates
 * (torch_gcu/csrc/aten/aot_ops/topsaten_bridge_define.h:323-427): every entry
 * point receives preallocated outputs, borrowed inputs, scalar parameters by
 * value and the stream to enqueue on, and returns a status.  The descriptor
 * replaces topsatenTensor (built by createTopsatenTensor,
 * torch_gcu/csrc/gcu/gcu_utils.cpp:79-108) and the scalar replaces
 * topsatenScalar_t (gcu_utils.cpp:322-430).
 *
 * Rules every entry point keeps:
 *   - plain C types only: no torch, no C++ exceptions across the boundary;
 *   - outputs are preallocated by the caller and never resized here;
 *   - enqueue-only on `stream`: no hipMalloc, no synchronous copy and no
 *     stream synchronisation, so every call can be captured in a hipGraph;
 *   - temporary device memory comes only from the allocator registered with
 *     mi_set_workspace_allocator (the reference registers its caching
 *     allocator with the kernel library the same way,
 *     torch_gcu/csrc/gcu/gcu_custom_api.cpp:23-31);
 *   - on failure a status other than MI_OK is returned and mi_last_error()
 *     gives a message for the calling thread.
 *   - 64-bit integer and floating types stay 64-bit on the device (the
 *     reference narrows them, torch_gcu/csrc/gcu/gcu_hardware.h:38-101; this
 *     library does not).
 */
#ifndef MI355X_OPS_H
#define MI355X_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling in HIP headers; 0 is the null stream. */
typedef void* mi_stream_t;

typedef enum {
  MI_OK = 0,
  MI_ERR_INVALID = 1,      /* bad shape, stride, dtype or parameter */
  MI_ERR_UNSUPPORTED = 2,  /* valid request this library does not implement */
  MI_ERR_WORKSPACE = 3,    /* no workspace allocator, or it returned NULL */
  MI_ERR_LAUNCH = 4,       /* the HIP runtime reported an error */
  MI_ERR_TOO_LARGE = 5     /* a size exceeds a documented maximum */
} mi_status_t;

/* Data types.  The numeric codes equal c10::ScalarType's so the host passes
 * tensor.scalar_type() through unchanged. */
typedef enum {
  MI_U8 = 0,
  MI_I8 = 1,
  MI_I16 = 2,
  MI_I32 = 3,
  MI_I64 = 4,
  MI_F16 = 5,
  MI_F32 = 6,
  MI_F64 = 7,
  MI_BOOL = 11,
  MI_BF16 = 15
} mi_dtype_t;

#define MI_MAX_DIMS 8

/* Strided tensor view.  Sizes and strides are in elements; ndim 0 is a
 * scalar (one element).  Replaces topsatenTensor(dims, strides, dtype, data)
 * (gcu_utils.cpp:79-108), which caps rank at 8 as this does. */
typedef struct {
  void* data;
  int32_t dtype;
  int32_t ndim;
  int64_t sizes[MI_MAX_DIMS];
  int64_t strides[MI_MAX_DIMS];
} mi_tensor_t;

/* A host scalar.  dtype is the scalar's own type: a floating dtype selects
 * f, any other selects i (bools are 0/1).  wrapped != 0 marks a Python
 * number (ATen's "wrapped number", which takes part in type promotion only
 * by category and as the default dtype); wrapped == 0 marks the value of a
 * 0-dim tensor.  Replaces topsatenScalar_t (gcu_utils.cpp:322-430); the CPU
 * 0-dim operand rule (codegen/gen_backend_stubs.py:1061-1078) hands values
 * over this way. */
typedef struct {
  double f;
  int64_t i;
  int32_t dtype;
  int32_t wrapped;
} mi_scalar_t;

/* ---- library state ---------------------------------------------------- */

/* Version of this ABI, (major << 16) | minor. */
int32_t mi_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* mi_last_error(void);

/* Stream-ordered workspace allocator used by entry points that need
 * temporary device memory.  Replaces topsatenMallocAsyncFuncRegister /
 * topsatenFreeAsyncFuncRegister (torch_gcu/csrc/gcu/gcu_custom_api.cpp:23-31,
 * implemented at gcu_caching_allocator.cpp:2956-3000).  free_fn is called with
 * the stream the memory was last used on. */
typedef void* (*mi_alloc_fn)(size_t bytes, mi_stream_t stream, void* ctx);
typedef void (*mi_free_fn)(void* ptr, mi_stream_t stream, void* ctx);
mi_status_t mi_set_workspace_allocator(mi_alloc_fn alloc_fn, mi_free_fn free_fn,
                                       void* ctx);

/* Number of compute units of the current device (used for launch sizing);
 * negative on error. */
int32_t mi_device_cu_count(void);

/* Out-of-range indices met by mi_index_select and mi_index on `device`
 * since the last call: returns 1 and stores one offending index and the size
 * of the dimension it indexed, or returns 0; clears the record.  The kernels
 * write the record into pinned host-coherent memory, so this reads host
 * memory only and must follow a synchronisation with the work it covers.
 * No counterpart in the reference's TopsAten seam, whose index kernels check
 * their indices themselves; the host layer raises the IndexError that CPU
 * ATen would, at the next synchronisation. */
int32_t mi_index_fault_take(int32_t device, int64_t* index, int64_t* dim_size);

/* ---- copies and fills --------------------------------------------------- */

/* out[...] = (out.dtype) src[...]; src broadcasts to out.  Same-dtype
 * contiguous copies become one D2D memcpy.  Replaces topsatenCopy
 * (torch_gcu/csrc/aten/aot_ops/gcu_copy.cpp:116-150). */
mi_status_t mi_copy(const mi_tensor_t* out, const mi_tensor_t* src,
                    mi_stream_t stream);

/* out = cat(inputs[0..n_inputs), dim): every input has out's rank and sizes
 * except along `dim`, where they add up to out's.  Dense inputs of out's
 * dtype with a dense out take one batched-row-copy launch (32 inputs per
 * launch); other layouts and dtype casts copy input by input (mi_copy).
 * ATen's shape rules (the skipped legacy 1-D empty inputs, dtype promotion,
 * memory format of out) are the host layer's.  Replaces topsatenCat
 * (codegen/gcu_native_functions.yaml cat.out :263). */
mi_status_t mi_cat(const mi_tensor_t* out, const mi_tensor_t* const* inputs,
                   int32_t n_inputs, int32_t dim, mi_stream_t stream);

/* out[...] = value.  Replaces topsatenFill_ (yaml fill_.Scalar :316). */
mi_status_t mi_fill(const mi_tensor_t* out, mi_scalar_t value,
                    mi_stream_t stream);

/* ---- binary elementwise (TensorIterator semantics) ----------------------
 * Inputs broadcast to out.  The common dtype follows ATen's result_type
 * (dimensioned tensors over 0-dim tensors over wrapped scalars, by
 * category); the op computes in float for f16/bf16, in the common type
 * otherwise, and casts to out.dtype on store.
 * Replace topsatenAdd / topsatenSub / topsatenMul / topsatenDiv
 * (codegen/gcu_native_functions.yaml add.out :202, mul.out :461; the
 * scalar forms are the RHS_IS_SCALAR branch,
 * codegen/gen_backend_stubs.py:1061-1078). */
mi_status_t mi_add(const mi_tensor_t* out, const mi_tensor_t* self,
                   const mi_tensor_t* other, mi_scalar_t alpha,
                   mi_stream_t stream);
mi_status_t mi_sub(const mi_tensor_t* out, const mi_tensor_t* self,
                   const mi_tensor_t* other, mi_scalar_t alpha,
                   mi_stream_t stream);
mi_status_t mi_mul(const mi_tensor_t* out, const mi_tensor_t* self,
                   const mi_tensor_t* other, mi_stream_t stream);
/* True division: integer inputs compute in float32. */
mi_status_t mi_div(const mi_tensor_t* out, const mi_tensor_t* self,
                   const mi_tensor_t* other, mi_stream_t stream);
/* out = self + alpha * other_scalar, other a wrapped number. */
mi_status_t mi_add_scalar(const mi_tensor_t* out, const mi_tensor_t* self,
                          mi_scalar_t other, mi_scalar_t alpha,
                          mi_stream_t stream);
/* out = self * other_scalar, other a wrapped number. */
mi_status_t mi_mul_scalar(const mi_tensor_t* out, const mi_tensor_t* self,
                          mi_scalar_t other, mi_stream_t stream);
/* out = self / other_scalar (true division), other a wrapped number. */
mi_status_t mi_div_scalar(const mi_tensor_t* out, const mi_tensor_t* self,
                          mi_scalar_t other, mi_stream_t stream);

/* ---- optimizer ---------------------------------------------------------- */

/* Hyper-parameters of one fused AdamW step (the float arguments of
 * torch._fused_adamw_). */
typedef struct {
  double lr; /* used when the lr tensor is NULL */
  double beta1, beta2, weight_decay, eps;
  int32_t amsgrad, maximize;
} mi_adamw_hparams_t;

/* One AdamW step over n_tensors parameters, in place: params, grads,
 * exp_avgs, exp_avg_sqs (and max_exp_avg_sqs with amsgrad) are arrays of
 * n_tensors descriptors of one dtype (f32, bf16, f16 or f64), each tensor
 * dense and laid out like its param; state_steps are one-element f32 step
 * counts (read, not advanced).  lr_tensor (one f32/f64 element) overrides
 * hp->lr when not NULL; grad_scale unscales the grads (written back) and
 * found_inf = 1 skips the step (both one-element f32, optional).  Every
 * scalar tensor is read on the device, so the call can be captured.
 * Replaces topsatenFusedAdamw (torch_gcu/csrc/aten/aot_ops/_fused_adamw_.cpp:
 * 15-52; yaml _fused_adamw_ :144-145). */
mi_status_t mi_fused_adamw(const mi_tensor_t* const* params,
                           const mi_tensor_t* const* grads,
                           const mi_tensor_t* const* exp_avgs,
                           const mi_tensor_t* const* exp_avg_sqs,
                           const mi_tensor_t* const* max_exp_avg_sqs,
                           const mi_tensor_t* const* state_steps,
                           int32_t n_tensors, const mi_tensor_t* lr_tensor,
                           const mi_adamw_hparams_t* hp,
                           const mi_tensor_t* grad_scale,
                           const mi_tensor_t* found_inf, mi_stream_t stream);

/* Every tensor of the list += value, in place (the sum in fp32, fp64 for
 * f64, rounded once): n_tensors dense tensors of one dtype (f32, bf16, f16,
 * f64).  The optimizer's step-count advance before a fused step.  Replaces
 * topsatenForeachAdd (yaml _foreach_add_.Scalar :47). */
mi_status_t mi_foreach_add_scalar(const mi_tensor_t* const* tensors,
                                  int32_t n_tensors, double value,
                                  mi_stream_t stream);

/* Every tensor of the list *= one value, in place: `scalar` (a one-element
 * float32 device tensor read by the kernel) when it is non-NULL, else
 * `value`.  The list is dense tensors of one float dtype, as for
 * mi_foreach_add_scalar.  Replaces the generated _foreach_mul_.Scalar and
 * _foreach_mul_.Tensor (yaml :131, :133). */
mi_status_t mi_foreach_mul_scalar(const mi_tensor_t* const* tensors, int32_t n_tensors,
                                  double value, const mi_tensor_t* scalar, mi_stream_t stream);

/* Mixed-precision grad unscaling: every element of the n_tensors dense
 * tensors (one dtype: f32, bf16, f16, f64) *= inv_scale in place (left as it
 * is when inv_scale is 1), and found_inf is set to 1 when any element is inf
 * or NaN (it is never cleared here).  found_inf and inv_scale are one-element
 * float32 tensors read on the device.  Replaces the generated
 * _amp_foreach_non_finite_check_and_unscale_ (yaml :15). */
mi_status_t mi_amp_unscale(const mi_tensor_t* const* tensors, int32_t n_tensors,
                           const mi_tensor_t* found_inf,
                           const mi_tensor_t* inv_scale, mi_stream_t stream);

/* GradScaler's scale update in place: when found_inf is nonzero the scale is
 * multiplied by backoff_factor and growth_tracker set to 0; otherwise
 * growth_tracker counts up, and on reaching growth_interval the scale is
 * multiplied by growth_factor (kept only if finite) and the count restarts.
 * scale and found_inf are one-element float32, growth_tracker one-element
 * int32, all device tensors.  Replaces the generated _amp_update_scale_
 * (yaml :16). */
mi_status_t mi_amp_update_scale(const mi_tensor_t* scale, const mi_tensor_t* growth_tracker,
                                const mi_tensor_t* found_inf, double growth_factor,
                                double backoff_factor, int64_t growth_interval,
                                mi_stream_t stream);

/* ---- indexing ---------------------------------------------------------- */

/* out = self.index_select(dim, index); index is 1-D (or 0-D) int32/int64;
 * negative indices are not wrapped (as in ATen).  The kernel never reads
 * outside self: a row whose index is out of range is written as zeros and
 * recorded for mi_index_fault_take (the reference validates shapes in
 * torch_gcu/csrc/aten/shape_inference/indexing.cpp:20-69).  Replaces
 * topsatenIndexSelect (yaml index_select.out :379). */
mi_status_t mi_index_select(const mi_tensor_t* out, const mi_tensor_t* self,
                            int64_t dim, const mi_tensor_t* index,
                            mi_stream_t stream);

/* out = self[indices] (advanced indexing, ATen's index.Tensor rules).
 * indices has n_indices <= self.ndim entries, one per leading dim of self:
 * NULL takes that dim whole, otherwise an int32 or int64 index tensor.  The
 * defined index tensors must already be broadcast to one shape B (stride 0
 * where broadcast).  When the indexed dims are adjacent,
 * out.shape = self.shape[:first] + B + self.shape[last+1:]; otherwise
 * out.shape = B + the other dims of self in order.  out is contiguous, of
 * self's dtype.  int32 indices are read as int32 (no widening to int64).
 * Negative indices count from the end of their dim; an index still out of
 * range writes its out row as zeros (the kernel never reads outside self)
 * and is recorded for mi_index_fault_take.  Replaces
 * topsatenIndex behind device_int32_indices_index
 * (torch_gcu/csrc/efficient_ops/ops.cpp:335-342, bridge_topsatenIndex_out1). */
mi_status_t mi_index(const mi_tensor_t* out, const mi_tensor_t* self,
                     const mi_tensor_t* const* indices, int32_t n_indices,
                     mi_stream_t stream);

/* ---- reductions ----------------------------------------------------------
 * dims lists the reduced dimensions of self (empty = all).  out holds
 * self's shape with reduced dims removed (keepdim=0) or set to 1
 * (keepdim=1).  Floating inputs accumulate in float (double for f64);
 * integer sums in int64.  Replace topsatenSum (sum.IntList_out :576),
 * topsatenAmax (amax.out :209), topsatenMean (mean.out :445). */
mi_status_t mi_sum(const mi_tensor_t* out, const mi_tensor_t* self,
                   const int64_t* dims, int32_t ndims, int32_t keepdim,
                   mi_stream_t stream);
mi_status_t mi_amax(const mi_tensor_t* out, const mi_tensor_t* self,
                    const int64_t* dims, int32_t ndims, int32_t keepdim,
                    mi_stream_t stream);
mi_status_t mi_mean(const mi_tensor_t* out, const mi_tensor_t* self,
                    const int64_t* dims, int32_t ndims, int32_t keepdim,
                    mi_stream_t stream);

/* Size of the static device scratch of mi_mean_noalloc (per GPU). */
#define MI_MEAN_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)

/* mi_mean that allocates nothing.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under hipGraph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results as mi_mean; the temporary memory mi_mean
 * takes from the workspace allocator (split-reduction partials; staging
 * copies for a reduced block that is not dense or an out that is not dense)
 * comes instead from a static device array of MI_MEAN_NOALLOC_SCRATCH_BYTES
 * per GPU, held until the process ends.  The call makes no hipMalloc /
 * hipFree and never calls the registered workspace allocator; a call that
 * would need more scratch than that returns MI_ERR_TOO_LARGE before it
 * writes out.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (on two streams, or from two threads) race. */
mi_status_t mi_mean_noalloc(const mi_tensor_t* out, const mi_tensor_t* self,
                            const int64_t* dims, int32_t ndims,
                            int32_t keepdim, mi_stream_t stream);

/* ---- softmax family -------------------------------------------------------
 * out = softmax / log_softmax of self along dim, computed in float; out may
 * be float when self is f16/bf16 (half_to_float).  Replace
 * topsatenSoftmaxForward (_softmax.out :182) and topsatenLogSoftmaxForward
 * (_log_softmax.out :155). */
mi_status_t mi_softmax(const mi_tensor_t* out, const mi_tensor_t* self,
                       int64_t dim, mi_stream_t stream);
mi_status_t mi_log_softmax(const mi_tensor_t* out, const mi_tensor_t* self,
                           int64_t dim, mi_stream_t stream);

/* Gradients of the two, from the forward output y and grad_output dy (one
 * dtype; grad_input may be f16/bf16 when they are float, the half_to_float
 * case), row sums in float:
 *   log_softmax: grad_input = dy - exp(y) * sum(dy)
 *   softmax:     grad_input = y * (dy - sum(dy * y))
 * Contiguous operands.  Replace topsatenLogSoftmaxBackward
 * (_log_softmax_backward_data.out :157) and topsatenSoftmaxBackward
 * (_softmax_backward_data.out :184). */
mi_status_t mi_log_softmax_backward(const mi_tensor_t* grad_input,
                                    const mi_tensor_t* grad_output,
                                    const mi_tensor_t* output, int64_t dim,
                                    mi_stream_t stream);
mi_status_t mi_softmax_backward(const mi_tensor_t* grad_input,
                                const mi_tensor_t* grad_output,
                                const mi_tensor_t* output, int64_t dim,
                                mi_stream_t stream);

/* ---- dense contractions ------------------------------------------------------
 * bf16 / fp16 operands run on MFMA (v_mfma_f32_32x32x16) with fp32
 * accumulation and one rounding of the result; fp32 operands on the VALU.
 * mat1, mat2 and out share a dtype.  A layout the MFMA kernel cannot read
 * directly (mat1 not K-contiguous, mat2 not K-contiguous as [N, K] rows, a
 * leading dim that is not a multiple of 8) is first copied densely into
 * workspace.  Replace topsatenAddmm (addmm.out :205), topsatenMm (mm.out
 * :452) and topsatenBmm (bmm.out :260); baddbmm.out is yaml :238. */

/* out = beta * self + alpha * (mat1 @ mat2); mat1 [M, K], mat2 [K, N], self
 * broadcasts to [M, N] and is ignored when beta == 0. */
mi_status_t mi_addmm(const mi_tensor_t* out, const mi_tensor_t* self,
                     const mi_tensor_t* mat1, const mi_tensor_t* mat2,
                     double beta, double alpha, mi_stream_t stream);
/* out = self @ mat2, [M, K] x [K, N]. */
mi_status_t mi_mm(const mi_tensor_t* out, const mi_tensor_t* self,
                  const mi_tensor_t* mat2, mi_stream_t stream);
/* out = beta * self + alpha * (mat @ vec); mat [M, K], vec [K], out [M]
 * (all one dtype: bf16, fp16 or fp32, fp32 accumulation, one rounding);
 * self is 0-D or [M] (the output's dtype or fp32) and is ignored when
 * beta == 0; mat and vec are ignored when alpha == 0.  Replaces
 * topsatenAddmv (addmv.out, codegen/gcu_native_functions.yaml:206); mv is
 * addmv with beta = 0. */
mi_status_t mi_addmv(const mi_tensor_t* out, const mi_tensor_t* self,
                     const mi_tensor_t* mat, const mi_tensor_t* vec,
                     double beta, double alpha, mi_stream_t stream);
/* out[b] = self[b] @ mat2[b], [B, M, K] x [B, K, N]. */
mi_status_t mi_bmm(const mi_tensor_t* out, const mi_tensor_t* self,
                   const mi_tensor_t* mat2, mi_stream_t stream);
/* out[b] = beta * self[b] + alpha * (batch1[b] @ batch2[b]). */
mi_status_t mi_baddbmm(const mi_tensor_t* out, const mi_tensor_t* self,
                       const mi_tensor_t* batch1, const mi_tensor_t* batch2,
                       double beta, double alpha, mi_stream_t stream);

/* int8 weight-only linear: out[m, n] = scales[n] * sum_k x[m, k] * w[n, k]
 * (+ bias[n]); x and out bf16 or fp16 [M, K] / [M, N], w int8 [N, K], scales
 * fp32 [N], bias (optional, NULL data for none) broadcast to [M, N].  The
 * weight is widened to bf16/fp16 exactly on its way into LDS and multiplied
 * on MFMA with fp32 accumulation.  For 64 < M <= 512 with too few 256 x 256
 * tiles to fill the CUs, K is split and the fp32 partial sums (S x M x N
 * floats, S = CUs / tiles, at most 16) come from the workspace allocator;
 * they are added in a fixed slice order, so results do not depend on
 * scheduling.  New efficient op: no TopsAten counterpart. */
mi_status_t mi_int8_linear(const mi_tensor_t* out, const mi_tensor_t* x,
                           const mi_tensor_t* weight, const mi_tensor_t* scales,
                           const mi_tensor_t* bias, mi_stream_t stream);

/* ---- attention ------------------------------------------------------------------
 * Flash-attention forward: out = softmax(scale * q k^T [+ causal mask]) v.
 * q [B, H, Sq, D], k and v [B, Hk, Sk, D] with H a multiple of Hk (query
 * heads share k/v heads in groups), D = 64 or 128, bf16 or fp16, head_dim
 * contiguous and rows 16-byte aligned; out like q.  is_causal masks key j
 * for query i when j > i.  lse (optional, NULL data for none) receives the
 * fp32 [B, H, Sq] log-sum-exp of the scaled scores.  Replaces
 * topsatenScaledDotProductFlashAttention
 * (torch_gcu/csrc/aten/aot_ops/gcu_attention.cpp:59-70). */
mi_status_t mi_flash_attention_fwd(const mi_tensor_t* out, const mi_tensor_t* lse,
                                   const mi_tensor_t* q, const mi_tensor_t* k,
                                   const mi_tensor_t* v, int32_t is_causal,
                                   double scale, mi_stream_t stream);

/* ---- fused efficient ops ---------------------------------------------------
 * The reference's efficient_ops entry point pattern
 * (torch_gcu/csrc/efficient_ops/ops.h:14-93, pybind at
 * torch_gcu/csrc/python/efficient_ops.cpp:12-26) holds one op; these are
 * new fused ops on the same surface and have no TopsAten counterpart. */

/* out[r, :] = x[r, :] * rsqrt(mean(x[r, :]^2) + eps) * weight, fp32 math,
 * over the last dim; weight a dense vector of the last dim's size, or NULL
 * data (no scale). */
mi_status_t mi_rms_norm(const mi_tensor_t* out, const mi_tensor_t* x,
                        const mi_tensor_t* weight, double eps,
                        mi_stream_t stream);

/* Rotate-half RoPE on [tokens, heads, head_dim] q and k (k may be NULL data)
 * with per-token int64/int32 positions:
 *   inv_freq[i] = theta^(-2i/head_dim), angle = pos * inv_freq[i],
 *   out[..., i]      = x[i] * cos - x[i + d/2] * sin
 *   out[..., i+d/2]  = x[i + d/2] * cos + x[i] * sin,   i < d/2.
 * Outputs may alias inputs (in place). */
mi_status_t mi_rope(const mi_tensor_t* q_out, const mi_tensor_t* k_out,
                    const mi_tensor_t* q, const mi_tensor_t* k,
                    const mi_tensor_t* positions, double theta,
                    mi_stream_t stream);

/* out = silu(gate) * up, fp32 math: silu(g) = g / (1 + exp(-g)). */
mi_status_t mi_silu_mul(const mi_tensor_t* out, const mi_tensor_t* gate,
                        const mi_tensor_t* up, mi_stream_t stream);

/* Fused matmul epilogues of a decoder layer.  No counterpart in the
 * reference (new efficient ops, like rms_norm, rope and silu_mul above); each
 * gives, bit for bit, what the unfused ops give:
 *   mi_linear_residual: out = residual + x @ weight^T, the product rounded to
 *     out's dtype first, then added in fp32 and rounded (linear, then add);
 *   mi_linear_silu_mul: out = silu(x @ w_gate^T) * (x @ w_up^T), both
 *     products rounded first (two linears, then silu_mul).
 * x [M, K], weights [N, K] (w_gate and w_up with one row stride), residual
 * and out [M, N]; bf16 or f16, unit column strides for the fused kernel (any
 * strides otherwise); out may be the residual itself.  The large-tile matmul
 * kernel applies the epilogue while its output tile is in LDS when there are
 * tiles enough to fill the CUs; other shapes run the matmul(s) into
 * workspace and then add / silu_mul. */
mi_status_t mi_linear_residual(const mi_tensor_t* out, const mi_tensor_t* x,
                               const mi_tensor_t* weight, const mi_tensor_t* residual,
                               mi_stream_t stream);
mi_status_t mi_linear_silu_mul(const mi_tensor_t* out, const mi_tensor_t* x,
                               const mi_tensor_t* w_gate, const mi_tensor_t* w_up,
                               mi_stream_t stream);

/* out = silu(self) = self / (1 + exp(-self)), fp32 math, one rounding; self
 * broadcast to out, one dtype (bf16, f16, f32).  Replaces topsatenSilu
 * (yaml silu.out :561). */
mi_status_t mi_silu(const mi_tensor_t* out, const mi_tensor_t* self, mi_stream_t stream);

/* grad_input = dy * s * (1 + x * (1 - s)), s = sigmoid(x), fp32 math; dy and
 * x broadcast to grad_input, all one dtype.  Replaces topsatenSiluBackward
 * (yaml silu_backward.grad_input :563). */
mi_status_t mi_silu_backward(const mi_tensor_t* grad_input,
                             const mi_tensor_t* grad_output,
                             const mi_tensor_t* self, mi_stream_t stream);

/* native_layer_norm over rows of normalized_numel elements: mean, biased
 * variance and rstd = 1 / sqrt(var + eps) in fp32 (stored in mean / rstd,
 * fp32 or the input's dtype, one element per row), out = (x - mean) * rstd *
 * weight + bias with the fp32 statistics; weight and bias optional, fp32 or
 * the input's dtype.  Contiguous f32 / bf16 / f16 input and out.  Replaces
 * topsatenNativeLayerNorm (yaml native_layer_norm :481). */
mi_status_t mi_layer_norm(const mi_tensor_t* out, const mi_tensor_t* mean,
                          const mi_tensor_t* rstd, const mi_tensor_t* input,
                          const mi_tensor_t* weight, const mi_tensor_t* bias,
                          int64_t normalized_numel, double eps, mi_stream_t stream);

/* native_layer_norm_backward over rows of normalized_numel elements: with
 * xh = (x - mean) * rstd and gw = dy * weight,
 *   grad_input  = rstd * (gw - mean_row(gw) - xh * mean_row(gw * xh))
 *   grad_weight = sum_rows(dy * xh),  grad_bias = sum_rows(dy)
 * in fp32; any of the three outputs may be NULL (not computed).  input and
 * grad_out contiguous of one dtype (f32/bf16/f16); mean and rstd one element
 * per row, fp32 or the input's dtype; weight fp32 or the input's dtype, or
 * NULL.  The column sums are added in a fixed order (workspace of at most
 * 2048 x 2 x normalized_numel floats).  Replaces
 * topsatenNativeLayerNormBackward (yaml native_layer_norm_backward :483). */
mi_status_t mi_layer_norm_backward(const mi_tensor_t* grad_input,
                                   const mi_tensor_t* grad_weight,
                                   const mi_tensor_t* grad_bias,
                                   const mi_tensor_t* grad_out,
                                   const mi_tensor_t* input,
                                   const mi_tensor_t* mean,
                                   const mi_tensor_t* rstd,
                                   const mi_tensor_t* weight,
                                   int64_t normalized_numel, mi_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MI355X_OPS_H */
