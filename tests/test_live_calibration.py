"""The live runners' two-point clock calibration (ssla_hip/live.py), on the
CPU: handshake points are preferred; the kernel's start / exit stamps are
the fallback."""
from ssla_hip import live as LV


def test_calibration_prefers_handshakes():
    # two handshakes 2 s apart at exactly 10 ns per tick
    h_ref, k_ref, npt = LV._calibration((5_000_000, 1000, 2000), (2_005_000_000, 200_001_000, 2500),
                                        900, 4_000_000, 200_002_000, 2_008_000_000)
    assert (h_ref, k_ref) == (5_000_000, 1000) and abs(npt - 10.0) < 1e-12


def test_calibration_falls_back_to_stamps():
    h_ref, k_ref, npt = LV._calibration(None, (1, 2, 3), 100, 1_000, 1_100, 11_000)
    assert (h_ref, k_ref) == (1_000, 100) and npt == 10.0
    # no exit stamp: nominal 100 MHz
    assert LV._calibration(None, None, 100, 1_000, 0, 0)[2] == 10.0
