"""The synchronisation probes (mkx_probe) on the GPU: they finish without a timed-out wait and report
plausible costs for the grid barrier and a stage hand-off (the reference prices its grid barrier the same
way, src/tune_mk.py:28-33, :66-68)."""
import ctypes

import pytest

from mkx import _lib

pytestmark = pytest.mark.gpu


def _probe(**kw):
    L = _lib.lib()
    a = _lib.MkxProbeArgs(**kw)
    _lib.check(L.mkx_probe(ctypes.byref(a), None), "mkx_probe")
    return a


def test_barrier_probe_runs_and_is_microseconds():
    a = _probe(kind=_lib.PROBE_BARRIER, n=200, bytes=0, fan=0, reps=3)
    print(f"grid barrier: {a.us_median:.3f} us (min {a.us_min:.3f})")
    assert not a.timed_out
    assert 0.1 < a.us_median < 50.0


@pytest.mark.parametrize("nbytes,fan", [(4096, 1), (24576, 24), (73728, 128)])
def test_handoff_probe_runs_across_xcds(nbytes, fan):
    a = _probe(kind=_lib.PROBE_HANDOFF, n=100, bytes=nbytes, fan=fan, reps=3)
    print(f"hand-off {nbytes} B x {fan}: {a.us_median:.3f} us (min {a.us_min:.3f}), XCDs {a.xcd_first[0]} -> {a.xcd_first[1]}")
    assert not a.timed_out
    assert 0.1 < a.us_median < 50.0
    assert a.xcd_first[0] != a.xcd_first[1]  # producer and first consumer on different XCDs
