"""The denoise schedule (schedule_sigmas, ming-generator.cc:158-174) on the
host: the library's against the oracle's (pinned to the closed form of
ming-config-test.cc:45-59) bit for bit, and its refusals."""
import numpy as np
import pytest

import oracle as orc
import ming_dit_amd as m


@pytest.mark.parametrize("steps", [1, 2, 11, 30])
@pytest.mark.parametrize("shift", [1.0, 3.0, 6.0])
def test_schedule_sigmas_matches_the_oracle(steps, shift):
    got = m.schedule_sigmas(steps, shift)
    want = np.asarray(orc.schedule_sigmas(steps, shift), np.float32)
    assert got.shape == (steps + 1,) and np.array_equal(got, want)
    assert got[0] == 1.0 and got[-1] == 0.0 and np.all(np.diff(got) < 0)


def test_the_default_schedule_closed_form():
    """11 steps at shift 6: sigma_k = 6m / (11 + 5m), m = 11 - k."""
    got = m.schedule_sigmas(11, 6.0)
    mm = 11 - np.arange(11)
    assert np.array_equal(got[:11], (6.0 * mm / (11.0 + 5.0 * mm)).astype(np.float32))


def test_schedule_refusals():
    out = (np.zeros(8, np.float32))
    ptr = out.ctypes.data_as(m.C.POINTER(m.C.c_float))
    for steps, shift in ((0, 6.0), (-1, 6.0), (4, 0.0), (4, float("nan"))):
        assert m.lib().ming_schedule_sigmas(steps, shift, ptr) == 1
    assert m.lib().ming_schedule_sigmas(4, 6.0, None) == 1
