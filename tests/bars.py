"""Parity bars shared by the GPU tests (north star: bf16 max-abs 2e-2 against fp32 ground truth).

A bf16 result of magnitude x is stored with a rounding error of up to 2^-8 x, which already
exceeds 2e-2 above |x| ~ 5, so the absolute bar is asserted where max |ref| <= 4 and the
relative bar (2e-2 of max |ref|) everywhere.
"""
TOL = 2e-2
ABS_LIMIT = 4.0


def bar(scale: float) -> float:
    """Largest admissible max |x - ref| for a tensor whose reference has max |ref| = scale."""
    rel = TOL * scale
    return min(rel, TOL) if scale <= ABS_LIMIT else rel


def check(name: str, err: float, scale: float) -> None:
    assert err <= bar(scale), f"{name}: max err {err:.3e} > bar {bar(scale):.3e} (max|ref| {scale:.3e})"

# fp32 inputs (north star: rel 1e-4): max |x - ref| <= 1e-4 * max |ref| for every tensor
TOL_F32 = 1e-4


def check_f32(name: str, err: float, scale: float) -> None:
    assert err <= TOL_F32 * scale, f"{name}: max err {err:.3e} > {TOL_F32:.0e} * max|ref| {scale:.3e}"
