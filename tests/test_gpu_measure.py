"""The achievable-peak kernels (obs_measure_read, obs_measure_mfma) that the
bench reads its roofline fractions against. No reference counterpart: the
reference's harness is a wall-clock token timer (main.rs:99-116).

Checks that both launch and finish, report what they claim (the flop count
of the launch, a core clock between 0.5 and 3 GHz) and land below the
published peaks (8 TB/s HBM, 2.5 PFLOP/s dense bf16), with argument errors
refused on the host."""
import numpy as np
import pytest

import obsidian_hip as oh

pytestmark = pytest.mark.gpu


def test_read_peak_is_below_the_published_hbm_peak(exe):
    nbytes = 512 << 20
    buf = exe.alloc(nbytes, np.uint8)
    sink = exe.alloc(4, np.uint32)
    exe.measure_read(buf, nbytes, sink)
    exe.timer_start()
    exe.measure_read(buf, nbytes, sink)
    ms = exe.timer_stop()
    exe.device_status()
    gbs = nbytes / (ms * 1e-3) / 1e9
    print(f"read {nbytes >> 20} MiB in {ms * 1e3:.1f} us = {gbs:.0f} GB/s")
    assert 500.0 < gbs < 8000.0


def test_mfma_peak_reports_its_flops_and_clock(exe):
    sink = exe.alloc(4, np.float32)
    clocks = exe.alloc(2, np.uint64)
    iters = 20000
    exe.timer_start()
    flops = exe.measure_mfma(iters, sink, clocks)
    ms = exe.timer_stop()
    exe.device_status()
    n_cus, _, _ = exe.dispatch_info()
    assert flops == 2 * n_cus * 4 * 4 * iters * (2 * 32 * 32 * 16)
    cyc, ticks = (int(v) for v in clocks.download())
    ghz = cyc / (ticks / 1e8) / 1e9
    tf = flops / (ms * 1e-3) / 1e12
    print(f"mfma {tf:.0f} TFLOP/s at {ghz:.3f} GHz")
    assert 0.5 < ghz < 3.0
    assert 100.0 < tf < 2600.0


def test_measure_rejects_bad_arguments(exe):
    buf = exe.alloc(64, np.uint8)
    sink = exe.alloc(4, np.uint32)
    with pytest.raises(oh.ObsError):
        exe.measure_read(buf, 24, sink)
    with pytest.raises(oh.ObsError):
        exe.measure_read(buf, 0, sink)
    with pytest.raises(oh.ObsError):
        exe.measure_mfma(0, sink, sink)
    with pytest.raises(oh.ObsError):
        exe.measure_mfma((1 << 24) + 1, sink, sink)
