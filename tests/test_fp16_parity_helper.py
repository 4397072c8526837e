"""The FP16 output bar used by the GPU parity tests (``helpers.fp16_parity``)
on hand-made cases whose answer follows from the FP16 grid alone."""

import numpy as np

from tests.helpers import fp16_parity


def _check(got, ref64):
    ref64 = np.asarray(ref64, dtype=np.float64)
    return fp16_parity(np.asarray(got, dtype=np.float16), ref64.astype(np.float16), ref64)


def test_midpoint_flip_passes():
    # -7.689451837 lies 1.3e-6 from the midpoint of -7.6875 and -7.69140625
    # (one ulp = 2**-8 apart): either neighbour is a correct rounding
    r = _check([-7.69140625], [-7.689451837480545])
    assert r["ok"] and r["boundary_flips"] == 1 and r["max_interval_gap"] < 2e-6
    r = _check([-7.6875], [-7.689451837480545])
    assert r["ok"] and r["boundary_flips"] == 0


def test_two_ulps_off_fails_past_four():
    # 7.6875 is exact in FP16; 7.6953125 (two ulps up) rounds only from
    # [7.69336, 7.69727], at least 5.9e-3 away
    r = _check([7.6953125], [7.6875])
    assert not r["ok"] and r["max_interval_gap"] > 5.8e-3


def test_one_ulp_off_an_exact_value_is_the_tolerance_edge():
    # 7.69140625 rounds from [7.689453125, 7.693359375]: 1.953e-3 from 7.6875
    assert _check([7.69140625], [7.6875])["ok"]
    assert not fp16_parity(np.float16([7.69140625]), np.float16([7.6875]),
                           np.float64([7.6875]), tol=1.9e-3)["ok"]


def test_small_values_use_the_plain_bar():
    r = _check([0.5, -0.0019], [0.5015, 0.0])
    assert r["ok"] and r["boundary_flips"] == 0 and r["max_fp16_diff"] <= 2e-3
    assert not _check([0.5], [0.5025])["ok"]


def test_binade_edge_uses_the_narrower_half_interval():
    # 8.0's reals reach down only to 8 - 2**-9 (the ulp below 8 is 2**-8)
    # and up to 8 + 2**-8 (the ulp above is 2**-7)
    r = _check([8.0], [8.0 + 5.9e-3])
    assert r["ok"] and abs(r["max_interval_gap"] - (5.9e-3 - 2 ** -8)) < 1e-9
    # 4.0e-3 below 8 is 2.05e-3 outside; the upper half-interval would wrongly admit it
    r = _check([8.0], [8.0 - 4.0e-3])
    assert not r["ok"] and abs(r["max_interval_gap"] - (4.0e-3 - 2 ** -9)) < 1e-9
