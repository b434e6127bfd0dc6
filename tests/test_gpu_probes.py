"""The ceiling probes bench.py reports (sglang.cpp_amd/csrc/probes/ceilings.hip)
run on the GPU and return plausible figures: the reads move their bytes at
a positive rate no faster than a generous bound on HBM3E, the MFMA probe's
clock readings are physical, constant operands are not slower than random
ones by more than noise, and an empty launch costs microseconds, not
milliseconds. These are measurement tools, not the product; the bounds only
catch a broken probe (a wrong byte or flop count, a clock ratio off by a
unit)."""
import importlib.util
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu

REPO = Path(__file__).resolve().parents[1]


def test_ceiling_probes_report_plausible_figures(dev):
    print("[case] ceiling probes", flush=True)
    spec = importlib.util.spec_from_file_location("_bench", REPO / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    c = bench.measure_ceilings(torch, dev, min_warm_s=0.1)
    for key in ("stream_read", "page_read_32k"):
        assert 500.0 < c[key]["GB/s"] < 12000.0, (key, c[key])
    for key in ("k_operand_cached", "k_rows_nt"):
        assert 500.0 < c["decode_read_pattern"]["GB/s"][key] < 12000.0, key
    for key in ("mfma_random", "mfma_const"):
        assert 100.0 < c[key]["TFLOP/s"] < 3000.0, (key, c[key])
        assert 500.0 < c[key]["shader_clock_MHz"] < 3500.0, (key, c[key])
    assert c["mfma_const"]["TFLOP/s"] > 0.9 * c["mfma_random"]["TFLOP/s"]
    assert 0.1 < c["empty_launch_us"]["graph"] < 100.0
