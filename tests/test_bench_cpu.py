"""bench.py's host-side helpers on the CPU: the roofline's counter traffic
comes from the committed rocprofv3 summary, and the GB/s arithmetic."""
import bench


def test_measured_traffic_reads_the_committed_counter_summary():
    traffic = bench.measured_traffic()
    assert isinstance(traffic, int)
    # HBM bytes per decode launch at the headline shape: within a few
    # percent of the algorithmic 544.8 MB (no re-reads).
    assert 0.9 * 544.8e6 < traffic < 1.1 * 544.8e6


def test_hbm_fraction_arithmetic():
    r = bench._hbm(544_800_000, 90e-6)  # the headline kernel's bytes in 90 us
    assert r["GB/s"] == 6053.3 and r["frac"] == round(6053.33 / 8000, 4) and r["us"] == 90.0
