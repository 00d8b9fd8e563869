"""Parity bars of the path, with the absolute floors written out.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* integer, index, bool and amax results, and fp32 single-rounding
  elementwise ops: bit-exact (NaNs compare equal);
* fp32 reductions / normalisations: |d| <= 1e-5*|ref| + 1e-5*max|ref|;
* bf16 / fp16 outputs with fp32 accumulation:
  |d| <= 1e-2*|ref| + 1e-2*rms(ref).

The relative parts are the north_star's; the floors make the bar meaningful
for references near zero.
"""
from __future__ import annotations

import torch

FP32_RTOL = 1e-5
BF16_RTOL = 1e-2


def assert_exact(actual: torch.Tensor, expected: torch.Tensor, what: str = "") -> None:
    a, e = actual.cpu(), expected.cpu()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    assert a.dtype == e.dtype, f"{what}: dtype {a.dtype} != {e.dtype}"
    if a.dtype.is_floating_point:
        same = (a == e) | (torch.isnan(a) & torch.isnan(e))
    else:
        same = a == e
    if not bool(same.all()):
        bad = (~same).nonzero()[:5].tolist()
        raise AssertionError(f"{what}: {int((~same).sum())} of {a.numel()} elements differ; "
                             f"first at {bad}: got {a[tuple(bad[0])].item()} "
                             f"expected {e[tuple(bad[0])].item()}")


def bar(expected: torch.Tensor, kind: str):
    """(rtol, atol) of the bar `kind` ('fp32' or 'bf16') for this reference."""
    e = expected.double()
    finite = e[torch.isfinite(e)]
    if kind == "fp32":
        scale = finite.abs().max().item() if finite.numel() else 0.0
        return FP32_RTOL, FP32_RTOL * scale
    if kind == "bf16":
        scale = finite.pow(2).mean().sqrt().item() if finite.numel() else 0.0
        return BF16_RTOL, BF16_RTOL * scale
    raise ValueError(kind)


def assert_close(actual: torch.Tensor, expected: torch.Tensor, kind: str, what: str = "") -> None:
    a, e = actual.cpu(), expected.cpu()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    assert a.dtype == e.dtype, f"{what}: dtype {a.dtype} != {e.dtype}"
    rtol, atol = bar(e, kind)
    ad, ed = a.double(), e.double()
    nan_ok = torch.isnan(ad) & torch.isnan(ed)
    inf_ok = torch.isinf(ad) & torch.isinf(ed) & (ad == ed)
    err = (ad - ed).abs()
    ok = (err <= rtol * ed.abs() + atol) | nan_ok | inf_ok
    if not bool(ok.all()):
        bad = (~ok).nonzero()[:3].tolist()
        i = tuple(bad[0])
        raise AssertionError(
            f"{what}: {int((~ok).sum())} of {a.numel()} outside |d| <= {rtol}*|ref| + {atol:.3g}; "
            f"first at {bad}: got {ad[i].item()} expected {ed[i].item()}")


def bar_ratio(actual: torch.Tensor, expected: torch.Tensor, kind: str) -> float:
    """max over finite elements of |d| / (rtol*|ref| + atol) under the bar
    `kind`: assert_close passes exactly when this is <= 1 (and the non-finite
    elements agree), so it shows the margin a passing result has."""
    a, e = actual.cpu().double(), expected.cpu().double()
    rtol, atol = bar(e, kind)
    fin = torch.isfinite(e) & torch.isfinite(a)
    if not bool(fin.any()):
        return 0.0
    r = (a - e).abs()[fin] / (rtol * e.abs()[fin] + atol).clamp_min(1e-300)
    return float(r.max())


def max_rel_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    a, e = actual.cpu().double(), expected.cpu().double()
    return float(((a - e).abs() / e.abs().clamp_min(1e-30)).max())


def rel_l2(actual: torch.Tensor, expected: torch.Tensor) -> float:
    a, e = actual.cpu().double(), expected.cpu().double()
    return float((a - e).norm() / e.norm().clamp_min(1e-30))


def assert_composed_close(actual: torch.Tensor, cpu: torch.Tensor, truth: torch.Tensor,
                          what: str = "", factor: float = 1.25) -> None:
    """Bar for a chain of bf16 ops (a whole decoder layer), where per-op
    roundings compound and residual sums cancel, so no single elementwise
    bound of the op bar holds near zero.  `cpu` is CPU ATen's result in the
    same dtype, `truth` the same chain in fp32.  The device result must be
    no further from the fp32 truth than CPU ATen is (relative L2, within
    `factor`), and within 1e-2 relative L2 of CPU ATen itself."""
    e_dev, e_cpu = rel_l2(actual, truth), rel_l2(cpu, truth)
    assert e_dev <= factor * e_cpu + 1e-4, (
        f"{what}: relative L2 error vs fp32 {e_dev:.3g} exceeds {factor} x CPU ATen's {e_cpu:.3g}")
    d = rel_l2(actual, cpu)
    assert d <= BF16_RTOL, f"{what}: relative L2 distance to CPU ATen {d:.3g} > {BF16_RTOL}"
