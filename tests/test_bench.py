"""Host-side checks of bench.py's contract (no GPU): the one-GPU refusal, the roofline fields of a memory-bound and
an MFMA-bound line, and the workload list the default run measures."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


class _WL:
    def __init__(self, name, bound, flops, nbytes):
        self.name, self.bound, self.flops, self.algo_bytes = name, bound, flops, nbytes


def test_roofline_hbm_line():
    wl = _WL("decode_q4_swiglu_M1", "hbm", 2.0 * 28672 * 4096, 73437184)
    rf = bench.roofline(wl, 0.0131)                        # 13.1 us per call
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert rf["achieved"] == pytest.approx(73437184 / 13.1e-6 / 1e9, rel=1e-3)
    assert rf["frac"] == pytest.approx(rf["achieved"] / 8000.0, abs=1e-4)
    fetch, write = bench.TRAFFIC_KIB["decode_q4_swiglu_M1"]
    assert rf["traffic"] == int((bench.FETCH_FACTOR * fetch + bench.WRITE_FACTOR * write) * 1024)
    assert 1.0 <= rf["traffic"] / wl.algo_bytes < 1.05     # the stream reads each weight byte once


def test_roofline_mfma_line():
    flops = 2.0 * 2048 * 4096 * 4096
    wl = _WL("prefill_q8_rms_resadd", "mfma", flops, 1)
    rf = bench.roofline(wl, 0.0913)
    assert rf["bound"] == "mfma" and rf["unit"] == "TFLOP/s" and rf["peak"] == 2500.0
    assert rf["achieved"] == pytest.approx(flops / 91.3e-6 / 1e12, rel=1e-3)
    assert rf["frac"] == pytest.approx(rf["achieved"] / 2500.0, abs=1e-4)


def test_default_run_measures_every_config():
    # configs[1] (decode M = 1 / 4 / 16), configs[2] (q8 prefill), configs[3] a / b (DiT QKV, up), configs[4] (conv3)
    for name in ("decode1", "decode4", "decode16", "prefill", "prefill_f16res", "dit_qkv", "dit_up", "conv3",
                 "hbm_ceiling"):
        assert name in bench.BUILDERS
    assert bench.HBM_SECONDARY_CALLS >= 1000
