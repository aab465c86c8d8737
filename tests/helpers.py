"""Shared test helpers."""
import numpy as np


def maxabs_rel(got: np.ndarray, want: np.ndarray) -> float:
    """max |got - want| / max |want| (outputs must agree to 1e-5 by this measure)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.max(np.abs(want))
    return float(np.max(np.abs(got - want)) / (den if den > 0 else 1.0))


def within(name: str, got: np.ndarray, want: np.ndarray, bar: float) -> float:
    """Assert maxabs_rel(got, want) < bar, printing the measured value (the
    bars of whole-model comparisons are set from these measurements)."""
    err = maxabs_rel(got, want)
    print(f"[bar] {name}: {err:.3e} (bar {bar:.0e})", flush=True)
    assert err < bar, f"{name}: {err:.3e} >= {bar:.0e}"
    return err


def near_max_steps(logits, want_tokens, want_logits, tol: float) -> list:
    """The steps at which token want_tokens[i] is not within `tol` (relative
    to the range of want_logits[i]) of the maximum of logits[i]: those where
    an implementation could not have picked it up to a rounding drift of
    that size."""
    bad = []
    for i, (lg, t, wl) in enumerate(zip(logits, want_tokens, want_logits)):
        rng = float(np.max(wl) - np.min(wl))
        if (float(np.max(lg)) - float(lg[int(t)])) > tol * rng:
            bad.append(i)
    return bad
