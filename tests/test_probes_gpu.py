"""The calibration probes behind the roofline notes (tsl_probe_mfma,
tsl_probe_mfma16, tsl_probe_stream): they run, give rates in a physically possible range
(at most the published peaks), and reject bad arguments."""

import pytest

import tessel_amd as T

pytestmark = pytest.mark.gpu


def test_mfma_probe_is_below_the_dense_peak(gpu):
    for rnd in (False, True):
        tf = T.probe_mfma(rnd, True, iters=200)
        assert 100.0 < tf <= 2500.0 * 1.01, tf


def test_mfma16_probe_is_below_the_dense_peak(gpu):
    tf = T.probe_mfma16(True, iters=200)
    assert 100.0 < tf <= 2500.0 * 1.01, tf
    with pytest.raises(T.TesselError):
        T.probe_mfma16(True, iters=0)


def test_stream_probe_is_below_the_hbm_peak(gpu):
    buf = T.alloc(64 << 20)
    gbs = T.probe_stream(buf, 16 << 20, iters=8)
    assert 100.0 < gbs, gbs
    with pytest.raises(T.TesselError):
        T.probe_stream(buf, 128 << 20)
    T.free(buf)
