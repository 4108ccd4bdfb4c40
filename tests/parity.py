"""The parity bar of BASELINE.json's north_star, shared by the GPU tests.

float32: every element within |got - ref| <= atol + rtol * |ref|, rtol 1e-4, atol 1e-5 (no
scaling by the tensor's magnitude); bf16 inputs with a float32 state: rtol 2e-2, the same
atol 1e-5 (16-bit results: their rounding is relative, so the float32 atol applies).  `close`
prints the per-tensor count of elements outside the bar and fails when it exceeds `allow`
(0 unless a test states a measured exception).
"""

import numpy as np
import torch

RTOL, ATOL = 1e-4, 1e-5            # float32 parity bar
RTOL_BF16, ATOL_BF16 = 2e-2, 1e-5  # bf16 inputs, float32 state


def _np(v):
    if isinstance(v, torch.Tensor):
        return v.detach().to("cpu", torch.float64).numpy()
    return np.asarray(v, dtype=np.float64)


def outside(got, ref, rtol=RTOL, atol=ATOL):
    """Number of elements of `got` outside atol + rtol |ref| (NaN counts as outside)."""
    g, r = _np(got), _np(ref)
    ok = np.abs(g - r) <= atol + rtol * np.abs(r)
    return int(g.size - np.count_nonzero(ok))


def close(got, ref, rtol=RTOL, atol=ATOL, name="", allow=0):
    g, r = _np(got), _np(ref)
    n = outside(g, r, rtol, atol)
    print(f"parity {name or 'tensor'}: {n} of {g.size} elements outside rtol {rtol:g} / atol {atol:g}", flush=True)
    if n > allow:
        np.testing.assert_allclose(g, r, rtol=rtol, atol=atol, err_msg=f"{name}: {n} outside (allowed {allow})")


F32_TERMS = 2.0 ** -16   # float32 resolution of a sum of terms: a few ulps of their magnitudes


def close_or_cancelled(got, ref, mag, name="", allow=0, rtol=RTOL, atol=ATOL, unit=F32_TERMS):
    """The bar for a gradient summed from float32 terms that can cancel (dA over batch and
    time, ddelta over the states): an element outside the bar passes only when its error is
    within float32 resolution of the sum of its terms' magnitudes `mag` (the oracle's), and at
    most `allow` elements may sit outside the bar at all.  `unit` is that resolution (2^-16 for
    float32 terms; a sum of 16-bit rounded terms passes its own, e.g. 2^-7 for bf16)."""
    g, r, m = _np(got), _np(ref), _np(mag)
    err = np.abs(g - r)
    bad = ~(err <= atol + rtol * np.abs(r))
    worst = float((err[bad] / m[bad]).max()) if bad.any() else 0.0
    print(f"parity {name or 'tensor'}: {int(bad.sum())} of {g.size} elements outside rtol {rtol:g} / "
          f"atol {atol:g}; largest error / term magnitude among them {worst:.2e}", flush=True)
    assert np.all(err[bad] <= unit * m[bad]), f"{name}: an outlier exceeds the resolution of its terms"
    assert bad.sum() <= allow, f"{name}: {int(bad.sum())} outside (allowed {allow})"
