"""Collected after the other GPU tests (file name): no decode plan made
through the entry points during the suite failed the kernels' grid and
shape assumptions.  plan_gemv drops such a plan and the call takes its other
path, so a planner bug would not fail any parity test; this counter is
where it shows."""
import pytest

from fish_amd import _lib

pytestmark = pytest.mark.gpu


def test_no_decode_plan_was_dropped():
    assert _lib.lib().fa_debug_gemv_plan_rejects() == 0
