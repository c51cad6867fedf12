"""The JavaScript CPU restatement (oracle/cpu_ref.mjs, the timed CPU baseline) agrees with the C oracle — no GPU.
Both are CPU restatements of the reference path; this pins the one bench.py times to the one the parity tests use."""
import ctypes as C
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle
import p0k
from cases import assert_close, make_case, make_conv3_case

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which("node")
pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


def run_js(case, tmp_path):
    s = p0k.gemm_args(case.args(lambda n: case.bufs[n]), p0k.numpy_resolve)
    spec = {name: getattr(s, name) for name, t in p0k.GemmArgs._fields_ if not name.endswith("_buf")}
    (tmp_path / "spec.json").write_text(json.dumps(spec))
    for k, v in case.bufs.items():
        v.tofile(str(tmp_path / f"{k}.bin"))
    subprocess.run([NODE, os.path.join(ROOT, "oracle", "cpu_ref.mjs"), "check", str(tmp_path)], check=True, timeout=120)
    return np.fromfile(str(tmp_path / "y_js.bin"), dtype=case.bufs["y"].dtype)


@pytest.mark.parametrize("kw", [
    dict(enc="q4g32a.t64", epi="swiglu", M=2, N=256, K=128),
    dict(enc="q4g32a.t64", epi="swiglu", M=2, N=256, K=128, act="gelu", bias=True),
    dict(enc="q8g64s.t64", xmode="rms", epi="resadd", M=3, N=128, K=128, bias=True, gate=True),
    dict(enc="q4g32a.t64", xmode="lnmod", epi="heads", M=3, N=384, K=64, Hq=1, Hkv=1, rope_mode="half", row_off=2, Ltot=8),
    dict(enc="f16", epi="heads", M=3, N=384, K=64, Hq=1, Hkv=1),
    dict(enc="f16", xmode="lnmod", epi="bias", M=3, N=64, K=64, res=True),
    dict(enc="q8g64s.t64", epi="f16", M=5, N=64, K=128),
    dict(enc="q4g32a.t64", epi="onormgate", M=2, N=128, K=64),
], ids=lambda k: f"{k['enc']}-{k.get('xmode', 'f16')}-{k['epi']}")
def test_js_port_matches_oracle(kw, tmp_path):
    case = make_case(seed=4, **kw)
    got = run_js(case, tmp_path)
    want = case.run_oracle(weights=oracle.CPU_WEIGHTS)          # both restate cpuGemm's fp32 dequantised weights
    assert_close(got, want, fp16=want.dtype == np.uint16, what="cpu_ref.mjs vs oracle")


def test_js_port_conv3_matches_oracle(tmp_path):
    case = make_conv3_case(T=3, H=4, W=5, C=32, N=64, pn=True)
    assert_close(run_js(case, tmp_path), case.run_oracle(weights=oracle.CPU_WEIGHTS), what="cpu_ref.mjs conv3")


def test_js_bench_runs():
    out = subprocess.run([NODE, os.path.join(ROOT, "oracle", "cpu_ref.mjs"), "bench", "conv3", "2"], capture_output=True,
                         text=True, timeout=120, check=True)
    r = json.loads(out.stdout.strip().splitlines()[-1])
    assert r["rows"] == 2 and r["ms_per_row"] > 0
