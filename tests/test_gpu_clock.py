"""The engine-clock probe (t2t_clock_probe) on the GPU: a plausible MI355X
engine clock under MFMA load, and the bench helper's peak at that clock."""
import pytest
import torch

import bench

pytestmark = pytest.mark.gpu


def test_engine_clock_is_plausible(gpu_device):
    clk = bench.engine_clock(gpu_device, iters=5000, reps=3)
    # gfx950 engine clocks lie between a few hundred MHz and the 2.4 GHz peak
    assert 300.0 < clk["engine_mhz_under_mfma_load"] <= 2500.0, clk
    assert clk["wall_clock_khz"] > 0
    cus = torch.cuda.get_device_properties(gpu_device).multi_processor_count
    expect = cus * 4096 * clk["engine_mhz_under_mfma_load"] * 1e6 / 1e12
    assert abs(clk["bf16_peak_at_clock_tflops"] - expect) < 0.2
