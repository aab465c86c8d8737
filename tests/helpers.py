"""Shared test helpers."""
import numpy as np


def maxabs_rel(got: np.ndarray, want: np.ndarray) -> float:
    """max |got - want| / max |want| (outputs must agree to 1e-5 by this measure)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.max(np.abs(want))
    return float(np.max(np.abs(got - want)) / (den if den > 0 else 1.0))
