"""Tolerance rules used by the parity tests.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* ``check_result`` / ``check_lse``: the reference's acceptance rule
  (test_sparse_attn_sharedkv.py:394-481, sparse_flash_mla_golden.py:606-663):
  >= 99.5 % of elements pass ``np.isclose`` at the dtype's tolerance and the
  worst failing element's normalised relative error stays below 10.
* ``check_vs_exact``: the kernel is at least as close to the exact float64
  answer as golden is: max |out - exact| <= 2 max |golden - exact| + 2^-9 max|exact|
  (2^-9 = half a bf16 ULP at the data scale).
* ``check_strict``: every element within ``atol + rtol*|ref|`` for the output
  (atol = rtol = 2e-2 for bf16/fp16) and ``|lse - ref| <= 1e-3*|ref| + 1e-5``
  for finite LSE values (non-finite values must match exactly).
"""

from __future__ import annotations

import numpy as np
import torch

OUT_ATOL = 2e-2
OUT_RTOL = 2e-2
LSE_RTOL = 1e-3
LSE_ATOL_FLOOR = 1e-5


def _as_np(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        return x.detach().cpu().to(torch.float32).numpy().ravel()
    return np.asarray(x, dtype=np.float32).ravel()


def _reference_rule(real, expt, rtol, atol, what):
    assert real.size == expt.size, f"{what}: size mismatch {real.size} vs {expt.size}"
    ok = np.isclose(real, expt, rtol=rtol, atol=atol, equal_nan=True)
    n_err = int((~ok).sum())
    pct = (real.size - n_err) / max(real.size, 1) * 100.0
    floor = (1.0 / (1 << 14)) / 0.005
    denom = np.maximum(np.maximum(np.abs(real), np.abs(expt)), floor) + 1e-9
    with np.errstate(invalid="ignore"):
        rel = np.abs(real - expt) / denom
    worst = float(np.nanmax(rel[~ok])) if n_err else 0.0
    assert pct >= 99.5, f"{what}: {pct:.4f}% within tol (rtol={rtol}, atol={atol}); " \
                        f"{n_err}/{real.size} failing, worst rel {worst:.4f}"
    assert worst < 10.0, f"{what}: worst normalised rel err {worst:.4f} >= 10"


def check_result(out, ref) -> None:
    """Reference output rule (bf16: rtol 2^-7, atol 1e-4; fp16: 0.005 / 2.5e-5)."""
    dt = out.dtype if isinstance(out, torch.Tensor) else torch.bfloat16
    rtol, atol = (0.0078125, 0.0001) if dt == torch.bfloat16 else (0.005, 0.000025)
    _reference_rule(_as_np(out), _as_np(ref), rtol, atol, "out")


def check_lse(lse, ref, q_dtype) -> None:
    """Reference LSE rule (bf16: rtol 0.015, atol 0.005; fp16: 0.01 / 0.001)."""
    rtol, atol = (0.015, 0.005) if q_dtype == torch.bfloat16 else (0.01, 0.001)
    _reference_rule(_as_np(lse), _as_np(ref), rtol, atol, "lse")


def check_strict(out, ref, lse=None, lse_ref=None) -> dict:
    """Per-element bound on every output and LSE value; returns the worst errors."""
    a, b = _as_np(out), _as_np(ref)
    assert a.size == b.size
    assert np.isfinite(a).all(), "non-finite output"
    err = np.abs(a - b)
    bound = OUT_ATOL + OUT_RTOL * np.abs(b)
    worst_i = int(np.argmax(err - bound)) if a.size else 0
    assert (err <= bound).all(), \
        f"out: {int((err > bound).sum())} elements beyond atol=rtol=2e-2; worst at {worst_i}: " \
        f"{a[worst_i]} vs {b[worst_i]}"
    res = dict(out_max_abs=float(err.max()) if a.size else 0.0)
    if lse is not None:
        x, y = _as_np(lse), _as_np(lse_ref)
        fin = np.isfinite(y)
        assert (np.isfinite(x) == fin).all(), "lse: finiteness differs"
        assert (x[~fin] == y[~fin]).all(), "lse: non-finite values differ"
        e = np.abs(x[fin] - y[fin])
        bnd = LSE_RTOL * np.abs(y[fin]) + LSE_ATOL_FLOOR
        assert (e <= bnd).all(), f"lse: {int((e > bnd).sum())} values beyond 1e-3 relative; " \
                                 f"max abs err {float(e.max())}"
        res["lse_max_abs"] = float(e.max()) if e.size else 0.0
    return res


def check_vs_exact(out, golden, exact) -> dict:
    """Accuracy against the float64 closed form, relative to golden's own accuracy."""
    a, g = _as_np(out).astype(np.float64), _as_np(golden).astype(np.float64)
    e = np.asarray(exact, dtype=np.float64).ravel()
    keep = np.isfinite(e)
    a, g, e = a[keep], g[keep], e[keep]
    ours = float(np.abs(a - e).max()) if e.size else 0.0
    gold = float(np.abs(g - e).max()) if e.size else 0.0
    scale = float(np.abs(e).max()) if e.size else 0.0
    bound = 2.0 * gold + scale * 2.0 ** -9
    assert ours <= bound, f"max|out-exact| {ours:.3e} > 2*max|golden-exact| ({gold:.3e}) + " \
                          f"2^-9*{scale:.3e}"
    return dict(ours=ours, golden=gold, scale=scale)
