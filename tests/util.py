"""Shared test helpers."""
import numpy as np


def rel_err(y, ref) -> float:
    """max |y - ref| / max |ref| over the whole output (norm-wise relative error).

    This is the relative tolerance the parity tests state: per-element
    relative error is meaningless for outputs near zero, whose absolute error
    is set by the magnitude of the other terms of the dot product."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(y - ref)) / (den if den > 0 else 1.0))
