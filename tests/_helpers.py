"""Shared test utilities: seeded inputs and the dtype-aware tolerance."""

from __future__ import annotations

import torch

DEV = "cuda"

# Tolerances: fp32 atol = rtol = 1e-5; fp16/bf16 2e-2
# absolute against the oracle rounded to the output dtype, where a result
# may also differ from the rounded oracle by one unit in the last place of
# that dtype (a float32 result and a float64 result can round to
# neighbouring 16-bit values; for |x| >= 4 in bf16 one ulp exceeds 2e-2).
LOWP_ATOL = 2e-2
FP32_TOL = 1e-5


def randn(shape, dtype=torch.float32, seed=0, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * std).to(dtype)


def ulp(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """One unit in the last place of ``dtype`` at |x| (float64 result)."""
    mant = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}[dtype]
    tiny = torch.finfo(dtype).tiny
    ax = x.abs().to(torch.float64).clamp_min(tiny)
    return torch.exp2(torch.floor(torch.log2(ax)) - mant)


def assert_close(ours: torch.Tensor, ref: torch.Tensor, dtype: torch.dtype, what: str = "",
                 scale_tol: float = 1.0):
    """Compare a device result with a float64 oracle value."""
    o = ours.detach().to("cpu", torch.float64)
    r = ref.detach().to("cpu", torch.float64)
    assert o.shape == r.shape, f"{what}: shape {tuple(o.shape)} vs {tuple(r.shape)}"
    fin = torch.isfinite(r)
    assert torch.equal(torch.isfinite(o), fin), f"{what}: finite pattern differs"
    assert torch.equal(o[~fin], r[~fin]), f"{what}: non-finite values differ"
    o, r = o[fin], r[fin]
    if o.numel() == 0:
        return
    if dtype == torch.float32:
        tol = FP32_TOL * scale_tol * (1 + r.abs())
        err = (o - r).abs()
    else:
        rr = r.to(dtype).to(torch.float64)
        tol = torch.maximum(torch.full_like(rr, LOWP_ATOL * scale_tol), ulp(rr, dtype))
        err = (o - rr).abs()
    bad = err > tol
    if bad.any():
        i = int(torch.argmax((err - tol)))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{o.numel()} elements out of tolerance; worst "
            f"|diff|={float(err[i]):.3e} (tol {float(tol[i]):.3e}) ours={float(o[i]):.6f} "
            f"ref={float(r[i]):.6f}")
