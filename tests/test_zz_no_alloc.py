"""p0k_gemm_noalloc: the allocation-free gemm (workspaces from the device's static scratch array) gives the same bits
as p0k_gemm on the calls that use a workspace — the split decode (partials + arrival counters), the rms / lnmod X'
pass, conv3 with PixelNorm (X' + the zero block of the padding taps) — on two calls in a row, the second smaller,
and refuses a call whose workspace would not fit."""
import numpy as np
import pytest

import oracle
import p0k
from cases import assert_close, make_case, make_conv3_case

pytestmark = pytest.mark.gpu


def run(dev, case, fn):
    d = {k: dev.upload(v) for k, v in case.bufs.items()}
    try:
        fn(case.args(lambda n: d[n]))
        out = case.bufs[case.out]
        return dev.read(d[case.out], out.dtype, out.size)
    finally:
        for b in d.values():
            dev.free(b)


PAIRS = {
    "split_decode": (dict(enc="q4g32a.t64", epi="swiglu", M=4, N=1024, K=4096, seed=81, wscale=0.02),
                     dict(enc="q4g32a.t64", epi="swiglu", M=2, N=512, K=2048, seed=82, wscale=0.02)),
    "split_decode_q8_rms": (dict(enc="q8g64s.t64", xmode="rms", epi="resadd", M=3, N=768, K=2048, seed=83),
                            dict(enc="q8g64s.t64", xmode="rms", epi="resadd", M=1, N=256, K=1024, seed=84)),
    "prefill_lnmod": (dict(enc="q4g32a.t64", xmode="lnmod", epi="bias", M=300, N=256, K=512, seed=85),
                      dict(enc="q4g32a.t64", xmode="lnmod", epi="bias", M=100, N=128, K=256, seed=86)),
}


@pytest.mark.parametrize("name", list(PAIRS))
def test_noalloc_matches_gemm(dev, name, monkeypatch):
    monkeypatch.setenv("P0K_GEMV_SN", "0")                  # the split decode, not the 16-row items (no workspace)
    for i, kw in enumerate(PAIRS[name]):
        print(f"[no-alloc] {name} call {i} {kw}", flush=True)
        c = make_case(**kw)
        kern = dev.select_tile(c.args(lambda n: c.bufs[n]))
        if kw["M"] <= 16:
            assert kern["kernel"].startswith("gemv")
        else:
            assert kern["kernel"] == "mfma_dma"
        want = run(dev, c, dev.gemm)
        got = run(dev, c, dev.gemm_noalloc)
        assert np.array_equal(got, want), f"{name} call {i}: noalloc differs from gemm"
        assert_close(got, c.run_oracle(), fp16=got.dtype == np.uint16, what=f"{name} call {i}")


def test_noalloc_conv3_pixelnorm(dev):
    for i, (T, H, W) in enumerate([(3, 10, 12), (2, 6, 8)]):
        print(f"[no-alloc] conv3 pn call {i}", flush=True)
        c = make_conv3_case(T=T, H=H, W=W, C=64, N=128, pn=True)
        assert dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"] == "mfma_dma"
        want = run(dev, c, dev.gemm)
        got = run(dev, c, dev.gemm_noalloc)
        assert np.array_equal(got, want)


def test_noalloc_refuses_oversized_workspace(dev):
    cap = p0k.lib().p0k_gemm_noalloc_scratch_bytes()
    M, K = 4096, 4096                                   # X' of M * K * 2 = 32 MiB > the scratch array
    assert M * K * 2 > cap
    c = make_case(enc="q8g64s.t64", xmode="rms", epi="f16", M=M, N=128, K=K, seed=87)
    with pytest.raises(p0k.P0kError, match="scratch array holds"):
        run(dev, c, dev.gemm_noalloc)


def test_noalloc_refuses_a_second_context(dev):
    """the first context to call p0k_gemm_noalloc holds the device's scratch array; another live context on the same
    device is refused (its stream could overlap the holder's calls), and may take it once the holder is gone"""
    c = make_case(enc="q4g32a.t64", epi="swiglu", M=2, N=512, K=2048, seed=88, wscale=0.02)
    run(dev, c, dev.gemm_noalloc)                       # dev holds the array from here on
    other = p0k.Device(0)
    try:
        with pytest.raises(p0k.P0kError, match="held by another live context"):
            run(other, c, other.gemm_noalloc)
        assert np.array_equal(run(other, c, other.gemm), run(dev, c, dev.gemm_noalloc))   # plain gemm is unaffected
    finally:
        other.close()
