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
    for key in ("stream_read", "page_read_32k", "stream_copy", "stream_copy_inplace",
                "stream_write"):
        assert 500.0 < c[key]["GB/s"] < 12000.0, (key, c[key])
    for key in ("k_operand_cached", "k_rows_nt"):
        assert 500.0 < c["decode_read_pattern"]["GB/s"][key] < 12000.0, key
    for key in ("mfma_random", "mfma_const"):
        assert 100.0 < c[key]["TFLOP/s"] < 3000.0, (key, c[key])
        assert 500.0 < c[key]["shader_clock_MHz"] < 3500.0, (key, c[key])
    assert c["mfma_const"]["TFLOP/s"] > 0.9 * c["mfma_random"]["TFLOP/s"]
    assert 0.1 < c["empty_launch_us"]["graph"] < 100.0


def test_copy_probe_moves_the_bytes(dev):
    """The copy probe's destination holds the source with bit 0 of every
    16-byte word's first lane flipped, for copies and in place, every
    variant, and a tail that is not a multiple of the unrolled step."""
    print("[case] copy probe contents", flush=True)
    spec = importlib.util.spec_from_file_location("_bench", REPO / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    lib = bench.load_probes()
    n = (1 << 20) + 48  # bytes
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    src = torch.randint(0, 1 << 30, (n // 4,), device=dev, generator=g, dtype=torch.int32)
    flip = torch.zeros_like(src)
    flip[0::4] = 1
    for variant in range(8):
        dst = torch.zeros_like(src)
        assert lib.sgl_probe_stream_copy(src.data_ptr(), dst.data_ptr(), n, 37, variant,
                                         torch.cuda.current_stream().cuda_stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(dst, src ^ flip), variant
    inplace = src.clone()
    assert lib.sgl_probe_stream_copy(inplace.data_ptr(), inplace.data_ptr(), n, 37, 3,
                                     torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(inplace, src ^ flip)
