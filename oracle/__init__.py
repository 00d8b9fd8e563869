"""CPU oracle for the torch_gcu PrivateUse1 op path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this package: only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker / the CPU baseline, never as the
thing measured or shipped.

The reference computes every op of this path in the closed TopsAten library
(torch_gcu/csrc/aten/aot_ops/topsaten_bridge_define.h:323-427); its own
oracle is PyTorch CPU ATen, reached by the boxed CPU fallback
(torch_gcu/csrc/aten/aten_cpu_fallback.cpp:342-411, at::native::cpu_fallback
at :390) and by op_check's CPU redispatch
(torch_gcu/csrc/aten/aot_ops/gcu_op_check.cpp:202-229).  This package
restates that path in two independent forms:

* ``oracle.aten``  -- the op run on CPU ATen exactly as the reference's
  fallback runs it (device inputs copied to CPU, the CPU kernel, the result
  copied back), plus the fp32 closed forms the fused ops are defined by;
* ``oracle.numpy_ref`` -- numpy restatements of the same arithmetic (IEEE
  float32 elementwise, integer gathers, float64 reductions, closed forms),
  used to pin ``oracle.aten`` before it is trusted.

``oracle.tolerance`` holds the parity bars (exact for integer, index and
single-rounding float ops; fp32 rel 1e-5; bf16 rel 1e-2 with fp32
accumulation) with their absolute floors written out.

Pinning status of each function is recorded in its docstring; every
function here is pinned by at least one check in ``tests/test_oracle.py``
(numpy restatement, closed form, invariant or committed golden fixture).
"""
