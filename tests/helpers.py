"""Shared test helpers: fp16 comparison at the path's tolerance."""
import numpy as np


def fp16_ulp(x):
    """Spacing of fp16 at |x| (subnormal spacing near zero)."""
    x = np.abs(np.asarray(x, dtype=np.float16))
    return np.spacing(x).astype(np.float64)


def assert_fp16_close(got, want, what="", max_ulp=1, rtol=1e-3):
    """|got - want| <= max(max_ulp fp16 ulps of want, rtol * |want|), elementwise.

    This is the output tolerance of the W8A8 path: the int32 partials are
    exact, and fp16 outputs may differ by the order of the fp32 sum over
    K-groups (the reference itself sums in different orders on its N == 1
    and N > 4 paths)."""
    got = np.asarray(got, dtype=np.float16).astype(np.float64)
    want = np.asarray(want, dtype=np.float16).astype(np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), "%s: non-finite output" % what
    tol = np.maximum(max_ulp * fp16_ulp(want), rtol * np.abs(want))
    err = np.abs(got - want)
    bad = err > tol
    if bad.any():
        i = np.argmax(err - tol)
        raise AssertionError("%s: %d/%d outside tolerance; worst at %s: got %r want %r" % (
            what, int(bad.sum()), bad.size, np.unravel_index(i, got.shape),
            got.flat[i], want.flat[i]))
