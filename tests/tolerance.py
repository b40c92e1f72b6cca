"""FP32-vs-double comparison used by every numeric parity test.

An output passes when ANY of these holds (plus a
condition-aware bound for outputs that are near zero because of cancellation):
  |a - e| <= 1e-4 * |e|             relative error 1e-4
  |a - e| <= 1e-5                   absolute error near zero
  |a - e| <= 16 * 2^-24 * m         m = sum_k |a_k * b_k|, i.e. "near zero" means
                                    |e| is small next to the magnitudes summed;
                                    a correct FP32 sum in any order stays below
                                    ~ (terms * 2^-24) * m, and a dropped or doubled
                                    term of a d-term row moves the result by ~m/d,
                                    far above 16 * 2^-24 * m for d < 1e6.
check() returns the error maxima and `only_cond`, the number of outputs that
pass by the third bound alone (beyond both 1e-4 relative and 1e-5 absolute).
"""
import numpy as np

RTOL = 1e-4
ATOL = 1e-5
COND = 16 * 2.0 ** -24


def check(actual, expected, mag, what=""):
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    mag = np.asarray(mag, dtype=np.float64)
    err = np.abs(actual - expected)
    ok = (err <= RTOL * np.abs(expected)) | (err <= ATOL) | (err <= COND * mag)
    ok &= np.isfinite(actual)
    if not ok.all():
        bad = np.flatnonzero(~ok.ravel())
        i = bad[0]
        raise AssertionError(
            f"{what}: {bad.size} of {ok.size} outputs out of tolerance; first at flat index "
            f"{i}: got {actual.ravel()[i]!r}, expected {expected.ravel()[i]!r}, "
            f"sum|ab| {mag.ravel()[i]!r}")
    rel = err / np.maximum(np.abs(expected), 1e-30)
    # outputs that pass neither the 1e-4 relative nor the 1e-5 absolute bound,
    # only the condition-aware one
    only_cond = ~((err <= RTOL * np.abs(expected)) | (err <= ATOL))
    n_cond = int(only_cond.sum())
    return {"n": int(err.size), "max_abs": float(err.max(initial=0)),
            "max_rel": float(rel.max(initial=0)),
            "max_cond": float((err / np.maximum(mag, 1e-30)).max(initial=0)),
            "only_cond": n_cond,
            "only_cond_max_abs": float(err[only_cond].max(initial=0)),
            "only_cond_max_abs_over_mag": float(
                (err[only_cond] / np.maximum(mag[only_cond], 1e-30)).max(initial=0))}
