"""Shared comparison helpers for the parity tests."""
from __future__ import annotations

import numpy as np

from peregrine_amd.synth import bf16_to_f32

# Tolerance stated by the north star for bf16 outputs with fp32 accumulation.
BF16_RTOL = 1e-2


def assert_bf16_close(got_bits, ref_bits, rtol: float = BF16_RTOL, atol_frac: float = 1e-2,
                      min_exact: float | None = None, what: str = "") -> dict:
    """|got - ref| <= rtol*|ref| + atol_frac*rms(ref), elementwise.

    bf16 keeps 8 significant bits, so one output ulp is ~0.4-0.8% relative;
    rtol 1e-2 admits a one-ulp rounding flip caused by a different fp32
    summation order and nothing larger. The absolute floor (1% of the RMS of
    the reference) covers outputs that cancel to near zero.
    """
    g = bf16_to_f32(np.asarray(got_bits)).astype(np.float64)
    r = bf16_to_f32(np.asarray(ref_bits)).astype(np.float64)
    assert g.shape == r.shape, (g.shape, r.shape)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    rms = float(np.sqrt(np.mean(r * r))) if r.size else 0.0
    err = np.abs(g - r)
    bound = rtol * np.abs(r) + atol_frac * rms
    bad = err > bound
    exact = float(np.mean(np.asarray(got_bits) == np.asarray(ref_bits)))
    stats = {"max_abs": float(err.max(initial=0)), "exact_frac": exact, "rms": rms, "bad": int(bad.sum())}
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.size} outside tolerance; {stats}"
    if min_exact is not None:
        assert exact >= min_exact, f"{what}: bit-exact fraction {exact:.4f} < {min_exact}; {stats}"
    return stats
