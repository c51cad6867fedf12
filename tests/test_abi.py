"""The C ABI without a GPU: the library loads, exports every entry point include/p0k.h declares, the struct layout
matches, and every argument error the reference throws (src/ops/gemm.js:31,271,283,313) — plus this build's bounds
and alignment checks — is reported on the host before anything could launch."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import p0k
from cases import make_case, make_conv3_case

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    txt = open(os.path.join(ROOT, "include", "p0k.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(p0k_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_declared_symbol():
    L = p0k.lib()
    names = declared_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), f"{n} is declared in include/p0k.h but not exported"
    assert set(names) == set(p0k.EXPORTS)
    assert L.p0k_abi_version() == 4


def test_struct_layout_matches():
    a = p0k.GemmArgs()
    a.struct_size = 7
    assert p0k.lib().p0k_gemm_check(C.byref(a)) == p0k.E_ARG
    msg = p0k.lib().p0k_last_error().decode()
    want = int(re.search(r"expects (\d+)", msg).group(1))
    assert want == C.sizeof(p0k.GemmArgs)


def host_args(case):
    return case.args(lambda n: case.bufs[n])


def expect_error(a, pattern):
    with pytest.raises(p0k.P0kError, match=pattern) as e:
        p0k.check(a)
    assert e.value.code == p0k.E_ARG


def test_valid_cases_pass_check():
    for kw in [dict(), dict(enc="q4g32a.t64", epi="swiglu", N=256), dict(enc="q8g64s.t64", xmode="rms", epi="resadd"),
               dict(epi="heads", N=384, Hq=1, Hkv=1), dict(xmode="lnmod", epi="bias", res=True)]:
        p0k.check(host_args(make_case(**kw)))
    p0k.check(host_args(make_conv3_case()))


def test_empty_calls_pass_check():
    """M = 0 or N = 0: the reference makes zero tiles and dispatches nothing (src/ops/gemm.js:312-319); the checks of
    the other arguments still apply"""
    for M, N in [(0, 256), (4, 0), (0, 0)]:
        a = host_args(make_case(enc="q4g32a.t64", M=4, N=256, K=256))
        a.update(M=M, N=N)
        p0k.check(a)
    a = host_args(make_case(enc="q4g32a.t64", M=4, N=256, K=256))
    a.update(M=0, K=48)
    expect_error(a, "K must be a multiple of 32")


def test_reference_errors():
    c = make_case()
    a = host_args(c)
    a["w"]["enc"] = "q3"
    expect_error(a, "unsupported weight encoding")
    a = host_args(c)
    a["K"] = 100
    expect_error(a, "K must be a multiple of 32")
    a = host_args(c)
    a["tile"] = {"BM": 48, "BN": 128}
    expect_error(a, "bad tile 48x128")
    a["tile"] = {"BM": 256, "BN": 128}
    expect_error(a, "bad tile")
    a = host_args(make_case(epi="heads", N=384, Hq=1, Hkv=1))
    a["tile"] = {"BM": 64, "BN": 64}                       # heads forces BN = 128: no error
    p0k.check(a)


def test_missing_bindings():
    a = host_args(make_case(xmode="rms"))
    del a["stats"]
    expect_error(a, "missing binding ST")
    a = host_args(make_case(xmode="lnmod"))
    del a["pv"]
    expect_error(a, "missing binding PV")
    a = host_args(make_case(epi="bias"))
    del a["ev"]
    expect_error(a, "missing binding EV")
    a = host_args(make_case(epi="heads", N=384, Hq=1, Hkv=1))
    del a["heads"]["rope"]
    expect_error(a, "missing binding RP")
    a = host_args(make_case(epi="onormgate", N=256))
    del a["gt"]
    expect_error(a, "missing binding GT")


def test_bounds_and_shapes():
    a = host_args(make_case(M=8))
    a["M"] = 9                                              # one row more than x holds
    expect_error(a, "x needs")
    a = host_args(make_case(M=8))
    a["y"]["size"] = 100
    expect_error(a, "y needs")
    a = host_args(make_case(enc="q4g32a.t64"))
    a["w"]["bytes"] -= 16
    expect_error(a, "w needs")
    a = host_args(make_case(enc="q4g32a.t64"))
    a["wk0"] = 32
    expect_error(a, "exceeds w.cols")
    a = host_args(make_case(epi="swiglu", N=256))
    a["N"] = 255
    expect_error(a, "swiglu")
    a = host_args(make_case(epi="heads", N=384, Hq=1, Hkv=1))
    a["N"] = 320
    expect_error(a, "heads needs N")
    a = host_args(make_case(xmode="f16"))
    a["x"]["ld"] = 258
    expect_error(a, "multiples of 4")


def test_conv3_frame_window_checked():
    c = make_conv3_case()
    a = host_args(c)
    a["conv"]["padT"], a["conv"]["padL"] = 2, 2           # frame 1 is read but the buffer starts at frame 2
    a["M"] = 36
    expect_error(a, "starts at frame padL")
    a = host_args(c)
    a["conv"]["Ci"] = 16
    expect_error(a, "Ci % 32")


def test_kernel_choice():
    assert p0k.select_tile(host_args(make_case(M=1, enc="q4g32a.t64")))["kernel"] == "gemv_short"   # short call
    assert p0k.select_tile(host_args(make_case(M=1)))["kernel"] == "gemv_short"             # f16 rows, 1..4: short call
    assert p0k.select_tile(host_args(make_case(M=4)))["kernel"] == "gemv_short"
    assert p0k.select_tile(host_args(make_case(M=5)))["kernel"] == "gemv_mfma"              # 5..16: matrix cores
    assert p0k.select_tile(host_args(make_case(M=2, K=96)))["kernel"] != "gemv_short"       # K % 64 != 0
    assert p0k.select_tile(host_args(make_case(M=2, enc="q4g32a.t64")))["kernel"] == "gemv_short"
    assert p0k.select_tile(host_args(make_case(M=3, enc="q4g32a.t64")))["kernel"] == "gemv"   # q4, 3..4 rows: stream
    assert p0k.select_tile(host_args(make_case(M=4, enc="q4g32a.t64")))["kernel"] == "gemv"
    assert p0k.select_tile(host_args(make_case(M=5, enc="q4g32a.t64")))["kernel"] == "gemv_mfma"
    assert p0k.select_tile(host_args(make_case(M=16)))["kernel"] == "gemv_mfma"
    assert p0k.select_tile(host_args(make_case(M=17)))["kernel"] == "mfma_dma"          # fp16 rows, K % 64 == 0
    assert p0k.select_tile(host_args(make_case(M=17, K=96)))["kernel"] == "mfma"         # K % 64 != 0
    c = make_conv3_case(T=1, H=2, W=2)                     # M = 4, a convolution: always the MFMA kernel
    assert p0k.select_tile(host_args(c))["kernel"] == "mfma"
    assert p0k.lib().p0k_gemm_flops(C.byref(p0k.gemm_args(host_args(make_case(M=3, N=64, K=32)), p0k.numpy_resolve))) == 2 * 3 * 64 * 32


@pytest.mark.parametrize("M,N,tile", [(4096, 24576, (128, 256)), (2048, 4096, (128, 128)), (4096, 9216, (128, 256)),
                                      (191360, 128, (128, 128)), (20000, 128, (128, 128)), (100, 128, (128, 128)),
                                      (64, 2048, (128, 128)), (8192, 8192, (128, 256))])
def test_mfma_tile_choice(M, N, tile):
    """Large tiles when the grid still fills the 256 CUs; smaller ones when it would leave them idle."""
    t = p0k.select_tile(host_args(make_case(M=M, N=N, K=32)))
    assert t["kernel"] == "mfma" and (t["BM"], t["BN"]) == tile


@pytest.mark.parametrize("enc,rows,K", [("q4g32a.t64", 128, 256), ("q8g64s.t64", 192, 128), ("f16", 64, 96)])
def test_product_encoders_match_the_oracle(enc, rows, K):
    """libp0k's host encoders (the converter side of FORMAT.md) produce the oracle's bytes exactly."""
    import oracle
    W = oracle.randn(rows * K, 77, 0.05)
    W[5] = 0.0                                      # an all-zero group: scale 0 -> 1
    if enc == "f16":
        assert np.array_equal(p0k.pack(enc, W, rows, K), oracle.f16_bits(W).view(np.uint8))
        return
    got, gdeq = p0k.pack(enc, W, rows, K, want_deq=True)
    want, wdeq = (oracle.pack_q4 if enc.startswith("q4") else oracle.pack_q8)(W, rows, K, want_deq=True)
    assert np.array_equal(got, want) and np.array_equal(gdeq, wdeq)
    with pytest.raises(p0k.P0kError):
        p0k.pack(enc, W[: 32 * K], 32, K)


@pytest.mark.parametrize("enc,M,N,tile", [("f16", 4096, 4096, (256, 256)), ("q8g64s.t64", 2048, 4096, (256, 128)),
                                          ("q4g32a.t64", 4096, 9216, (256, 256)), ("q4g32a.t64", 2048, 4096, (256, 128)),
                                          ("q8g64s.t64", 8192, 8192, (256, 256)), ("f16", 17, 256, (128, 256)),
                                          ("q4g32a.t64", 1024, 4096, (128, 128))])
def test_dma_tile_choice(enc, M, N, tile):
    """The load-to-LDS kernel's tile: 256-row tiles for quantised weights while the grid fills the CUs (a decoded
    weight feeds four 32-row blocks), smaller tiles when the grid would leave CUs idle."""
    t = p0k.select_tile(host_args(make_case(enc=enc, M=M, N=N, K=64)))
    assert t["kernel"] == "mfma_dma" and (t["BM"], t["BN"]) == tile


def test_conv3_gather_tile_choice():
    """conv3 with Ci % 64 == 0 takes the load-to-LDS gather, 256 x 128 tiles (8 waves: the per-step tap addressing
    runs under the other wave's MFMAs); Ci = 32 keeps the register-staged kernel."""
    t = p0k.select_tile(host_args(make_conv3_case(T=13, H=92, W=160, C=128, N=128)))
    assert t["kernel"] == "mfma_dma" and (t["BM"], t["BN"]) == (256, 128)
    assert p0k.select_tile(host_args(make_conv3_case(T=4, H=6, W=8, C=32, N=128)))["kernel"] == "mfma"


def test_tuning_switches_read_per_call_without_a_context(monkeypatch):
    """p0k_select_tile (no context) reads the P0K_* switches when called; a context reads them once and again on
    p0k_ctx_reload_env (the Python Device does that when this process changed them)."""
    a = host_args(make_case(enc="q4g32a.t64", M=2048, N=4096, K=64))
    base = p0k.select_tile(a)
    monkeypatch.setenv("P0K_MFMA_TILE", "128x128")
    t = p0k.select_tile(a)
    assert (t["BM"], t["BN"]) == (128, 128)
    monkeypatch.setenv("P0K_MFMA_TILE", "100x7")                  # not a tile: ignored
    assert p0k.select_tile(a) == base
    monkeypatch.setenv("P0K_MFMA_KERNEL", "reg")
    assert p0k.select_tile(a)["kernel"] == "mfma"
    monkeypatch.delenv("P0K_MFMA_KERNEL")
    monkeypatch.delenv("P0K_MFMA_TILE")
    assert p0k.select_tile(a) == base


def test_decode_row_routing_switch(monkeypatch):
    """P0K_GEMV_MX=n sends q4 decode calls with 2..n rows to the stream kernel's matrix-core form (kernel "gemv");
    the default is 4, beyond it the q4 matrix-core decode (k_gemv_mq4, "gemv_mfma") takes the call."""
    q4 = lambda M: p0k.select_tile(host_args(make_case(M=M, enc="q4g32a.t64", N=256, K=512)))["kernel"]   # noqa: E731
    monkeypatch.setenv("P0K_GEMV_SN", "0")                        # (these short calls would take the 16-row items)
    assert [q4(M) for M in (1, 2, 3, 4, 5, 16)] == ["gemv"] * 4 + ["gemv_mfma"] * 2
    monkeypatch.setenv("P0K_GEMV_MX", "0")
    assert [q4(M) for M in (1, 2, 3, 4)] == ["gemv", "gemv", "gemv_mfma", "gemv_mfma"]
    monkeypatch.setenv("P0K_GEMV_MX", "16")
    assert [q4(M) for M in (5, 8, 16)] == ["gemv"] * 3
    # q8 / f16 weights never take it
    assert p0k.select_tile(host_args(make_case(M=4, enc="q8g64s.t64", N=256, K=512)))["kernel"] == "gemv_mfma"


def test_short_decode_routing(monkeypatch):
    """q4 decode with one or two rows whose 16-row items number at most about one per CU (1.5 per CU at one row), K up to
    8192 and an element-wise epilogue takes the short-call kernel; q8 decode at one row, and with up to 2 / 1 items per CU at
    2 / 3..4 rows and K up to 8192 as well; P0K_GEMV_SN=0 / 1 switch it off / on wherever it can run (up to 4
    rows, K up to 16384 for q4 and 8192 for q8 / f16, X' in 64 KB of LDS); f16 weights with 16-byte rows take it at 1..4
    rows whenever it can run."""
    q4 = lambda M, N, K, **kw: p0k.select_tile(host_args(make_case(M=M, enc="q4g32a.t64", N=N, K=K, **kw)))["kernel"]   # noqa: E731
    assert q4(1, 4096, 4096) == "gemv_short" and q4(2, 4096, 4096) == "gemv_short"
    assert q4(1, 6144, 4096) == "gemv_short" and q4(2, 6144, 4096) == "gemv"
    assert q4(1, 14336, 4096) == "gemv" and q4(4, 4096, 4096) == "gemv" and q4(1, 4096, 16384) == "gemv"
    assert q4(1, 2048, 1024, epi="swiglu") == "gemv_short"
    assert q4(1, 384, 256, epi="heads", Hq=1, Hkv=1) != "gemv_short"
    q8 = lambda M, N, K, **kw: p0k.select_tile(host_args(make_case(M=M, enc="q8g64s.t64", N=N, K=K, **kw)))["kernel"]   # noqa: E731
    assert q8(1, 256, 512) == "gemv_short" and q8(1, 14336, 4096) == "gemv_short" and q8(2, 8192, 4096) == "gemv_short"
    assert q8(4, 4096, 4096) == "gemv_short" and q8(1, 4096, 8192) == "gemv_short"
    assert q8(2, 10240, 4096) == "gemv_mfma" and q8(4, 6144, 4096) == "gemv_mfma" and q8(1, 4096, 8704) != "gemv_short"
    assert q8(1, 28672, 4096) == "gemv_short" and q8(2, 28672, 4096) == "gemv_mfma"   # 1792 items: 7 per CU
    f16 = lambda M, N, K, **kw: p0k.select_tile(host_args(make_case(M=M, enc="f16", N=N, K=K, **kw)))["kernel"]   # noqa: E731
    assert f16(1, 256, 512) == "gemv_short" and f16(4, 14336, 4096) == "gemv_short" and f16(4, 256, 8192) == "gemv_short"
    assert f16(1, 256, 8256) != "gemv_short" and f16(1, 256, 544) != "gemv_short" and f16(5, 256, 512) != "gemv_short"
    monkeypatch.setenv("P0K_GEMV_SN", "0")
    assert q4(1, 4096, 4096) == "gemv" and q8(1, 4096, 4096) == "gemv_mfma"
    monkeypatch.setenv("P0K_GEMV_SN", "1")
    assert q4(1, 14336, 4096) == "gemv_short" and q4(1, 4096, 16384) == "gemv_short" and q4(4, 4096, 4096) == "gemv_short" and q4(3, 520, 96) == "gemv_short"
    assert q4(1, 4096, 16416) != "gemv_short" and q4(4, 4096, 8192) != "gemv_short"   # past the longest K an item stages
    assert q8(4, 4096, 4096) == "gemv_short" and q8(3, 6144, 8192) != "gemv_short"   # 3..4 rows x 8192 k: past 64 KB
    assert q8(2, 40960, 8192) == "gemv_short" and q8(1, 4096, 16384) != "gemv_short"


def test_null_context_calls_are_refused():
    L = p0k.lib()
    assert L.p0k_ctx_reload_env(None) == p0k.E_ARG
    assert L.p0k_ctx_cus(None) == 0
    assert L.p0k_alloc(None, 16, C.byref(C.c_void_p())) == p0k.E_ARG
