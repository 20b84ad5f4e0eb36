"""bench.py's host-side helpers (no GPU): the parity block of the bench line."""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402


def test_parity_normwise_and_per_element():
    y_ref = np.array([10.0, -5.0, 0.001, 2.0], np.float64)
    y = y_ref.copy()
    y[1] += 1e-4  # abs error 1e-4 on |y| = 5: rel 2e-5, normwise 1e-5
    y[2] += 1.0   # |y_ref| = 1e-3 < 1e-3 * 10: excluded from the per-element figure
    p = bench.parity_vs(y, y_ref, exact=True)
    assert abs(p["normwise_err"] - 0.1) < 1e-6  # the excluded element dominates the normwise error
    assert abs(p["per_element_rel_err_max"] - 2e-5) < 1e-8
    assert p["elements_compared"] == 3 and p["outputs"] == 4
    assert p["bit_exact"] is False
    assert bench.parity_vs(y_ref, y_ref, exact=True)["bit_exact"] is True


def test_parity_zero_reference():
    p = bench.parity_vs(np.zeros(3), np.zeros(3), exact=False)
    assert p["normwise_err"] == 0.0 and p["elements_compared"] == 0 and "bit_exact" not in p
