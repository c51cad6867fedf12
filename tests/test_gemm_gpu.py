"""GPU parity of the HIP `gemm` path against the CPU oracle, through the C ABI (libp0k.so).

Mirrors the reference's own GPU cases (test/kernels.test.js:71-145) — three encodings x two accumulate modes, partial
tiles, the 3x3x3 convolution whole / per tile / in 2-frame chunks / from a 3-frame ring — and extends them to every
prologue and epilogue of gemm.js on both kernels (the decode GEMV for M <= 16 and the MFMA GEMM above). Pass bars:
the reference's cosine > 0.9995 against its fp32-weight cpuGemm, the per-element tolerance of cases.assert_close
against the oracle, bit-identity where the reference demands it (conv3 chunks / ring), and bit-exact dequantised
weights.
"""
import numpy as np
import pytest

import oracle
import p0k
from cases import Case, assert_close, cos_maxerr, make_case, make_conv2d_case, make_conv3_case, to_float

pytestmark = pytest.mark.gpu


def banner(msg):
    print(f"[p0k-test] {msg}", flush=True)


# ------------------------------------------------------------------------------------------------ reference suite
@pytest.mark.parametrize("enc", ["f16", "q4g32a.t64", "q8g64s.t64"])
@pytest.mark.parametrize("acc", ["f32", "f16"])
def test_reference_gemm_cases(dev, enc, acc):
    """test/kernels.test.js:72-84: M 32, N 128, K 256, X = f16(randn seed 7), W = randn(seed 11, 0.05)."""
    M, N, K = 32, 128, 256
    banner(f"reference gemm {enc} acc={acc}")
    X = oracle.h2f(oracle.f16_bits(oracle.randn(M * K, 7)))
    W0 = oracle.randn(N * K, 11, 0.05)
    if enc == "f16":
        Wd = oracle.h2f(oracle.f16_bits(W0))
        wb = oracle.f16_bits(W0).view(np.uint8).copy()
    else:
        wb, Wd = (oracle.pack_q4 if enc.startswith("q4") else oracle.pack_q8)(W0, N, K, want_deq=True)
    bufs = {"w": wb, "x": oracle.f16_bits(X), "y": np.zeros(M * N, np.uint16)}
    spec = {"w": {"enc": enc, "buf": "w", "off": 0, "bytes": wb.nbytes, "rows": N, "cols": K}, "x": {"buf": "x"},
            "y": {"buf": "y"}, "M": M, "N": N, "K": K, "acc": acc}
    c = Case(spec, bufs)
    got = c.run_device(dev)
    cos, _ = cos_maxerr(to_float(got), oracle.cpu_gemm(X, Wd, M, N, K))
    assert cos > 0.9995
    assert_close(got, c.run_oracle(), what=f"{enc}/{acc}")


def test_reference_partial_tiles(dev):
    """test/kernels.test.js:85-92: M 33, N 192 (partial tiles), fp16 weights."""
    M, N, K = 33, 192, 256
    X = oracle.h2f(oracle.f16_bits(oracle.randn(M * K, 17)))
    Wd = oracle.h2f(oracle.f16_bits(oracle.randn(N * K, 19, 0.05)))
    bufs = {"w": oracle.f16_bits(Wd).view(np.uint8).copy(), "x": oracle.f16_bits(X), "y": np.zeros(M * N, np.uint16)}
    spec = {"w": {"enc": "f16", "buf": "w", "off": 0, "bytes": bufs["w"].nbytes, "rows": N, "cols": K},
            "x": {"buf": "x"}, "y": {"buf": "y"}, "M": M, "N": N, "K": K}
    c = Case(spec, bufs)
    got = c.run_device(dev)
    cos, _ = cos_maxerr(to_float(got), oracle.cpu_gemm(X, Wd, M, N, K))
    assert cos > 0.9995
    assert_close(got, c.run_oracle())


def test_config0_plain_f16_gemm(dev):
    """BASELINE configs[0], the reference's own correctness shape class (test/kernels.test.js:72-92) at M 64, N 256,
    K 512: x fp16 U[-1, 1], w fp16 N(0, 0.02). The reference's bar (cos > 0.9995 against the float64 cpuGemm) and the
    per-element tolerance against the oracle."""
    M, N, K = 64, 256, 512
    banner("configs[0] plain f16 GEMM")
    c = make_case(enc="f16", M=M, N=N, K=K, seed=64, wscale=0.02, x_uniform=True)
    X = oracle.h2f(c.bufs["x"])
    Wd = oracle.h2f(c.bufs["w"].view(np.uint16))
    assert X.min() >= -1.0 and X.max() <= 1.0
    got = c.run_device(dev)
    cos, _ = cos_maxerr(to_float(got), oracle.cpu_gemm(X, Wd, M, N, K))
    assert cos > 0.9995
    assert_close(got, c.run_oracle(), what="configs[0]")


# ------------------------------------------------------------------------------------------------ all prologues/epilogues
EPIS = [
    ("f16", "f16", {}),
    ("f16", "f32", {"ld_pad": 8, "k0": 32, "n0": 8}),
    ("rms", "resadd", {"bias": True, "gate": True}),
    ("lnmod", "resadd", {"store": True}),
    ("f16", "resadd", {}),
    ("lnmod", "bias", {"res": True}),
    ("rms", "bias", {}),
    ("f16", "swiglu", {}),
    ("f16", "swiglu", {"act": "gelu", "bias": True}),
    ("lnmod", "heads", {"Hq": 1, "Hkv": 1, "rope_mode": "half", "row_off": 3, "Ltot": 80}),
    ("f16", "heads", {"Hq": 2, "Hkv": 1, "row_off": 1, "Ltot": 80}),
    ("f16", "onormgate", {}),
]


@pytest.mark.parametrize("M", [1, 2, 4, 16, 70])
@pytest.mark.parametrize("enc", ["f16", "q4g32a.t64", "q8g64s.t64"])
@pytest.mark.parametrize("xmode,epi,kw", EPIS, ids=[f"{x}-{e}-{i}" for i, (x, e, _) in enumerate(EPIS)])
def test_prologue_epilogue_matrix(dev, M, enc, xmode, epi, kw, monkeypatch):
    kw = dict(kw)
    N = {"heads": (kw.get("Hq", 1) + 2 * kw.get("Hkv", 1)) * 128, "swiglu": 384, "onormgate": 256}.get(epi, 192)
    K = 256
    banner(f"matrix M={M} {enc} {xmode}/{epi} {kw}")
    c = make_case(enc=enc, xmode=xmode, epi=epi, M=M, N=N, K=K, seed=M + 5, **kw)
    kern = dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"]
    short = (M <= 2 if enc.startswith("q4") else M <= 4) and epi not in ("heads", "onormgate")
    assert kern == ("gemv_short" if short else "gemv" if M <= 4 and enc.startswith("q4") else "gemv_mfma" if M <= 16 else
                    "mfma_dma")
    got = c.run_device(dev)
    want = c.run_oracle()
    assert_close(got, want, fp16=got.dtype == np.uint16, what=f"{enc} {xmode}/{epi} M={M}")
    if short:
        # the one-row / 2-row stream kernel (q4) or the matrix-core decode (q8 / f16) on the same call (P0K_GEMV_SN=0)
        monkeypatch.setenv("P0K_GEMV_SN", "0")
        assert dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"] == ("gemv" if enc.startswith("q4") else "gemv_mfma")
        got = c.run_device(dev)
        assert_close(got, want, fp16=got.dtype == np.uint16, what=f"{enc} {xmode}/{epi} M={M} stream")
    if kern == "mfma_dma":
        # the register-staged MFMA kernel on the same call
        monkeypatch.setenv("P0K_MFMA_KERNEL", "reg")
        assert dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"] == "mfma"
        got = c.run_device(dev)
        assert_close(got, want, fp16=got.dtype == np.uint16, what=f"{enc} {xmode}/{epi} M={M} register-staged")


# ------------------------------------------------------------------------------------------------ matrix-core decode
DECODE_OFFSET_CASES = [
    # 16-byte X rows with row / column offsets: the item's X rows are copied to LDS (load-to-LDS)
    dict(enc="q4g32a.t64", epi="f16", M=5, N=320, K=384, ld_pad=8, k0=64, wk0=32, n0=8),
    dict(enc="q4g32a.t64", epi="swiglu", M=16, N=512, K=512, ld_pad=24, k0=16, wr0=64),
    # rows or k0 not a multiple of 8 halfs: the A fragments are read from X with each unit's loads
    dict(enc="q4g32a.t64", epi="f16", M=3, N=192, K=256, ld_pad=4),
    dict(enc="q4g32a.t64", epi="resadd", M=9, N=256, K=640, ld_pad=4, k0=4),
    # a slice shorter than one unit per wave (K = 128: 4 units for 8 waves)
    dict(enc="q4g32a.t64", epi="f32", M=12, N=256, K=128),
]


@pytest.mark.parametrize("path", ["mq4", "mx"])
@pytest.mark.parametrize("kw", DECODE_OFFSET_CASES, ids=lambda k: f"M{k['M']}-K{k['K']}-pad{k.get('ld_pad', 0)}-k0{k.get('k0', 0)}")
def test_matrix_core_decode_offsets(dev, kw, path, monkeypatch):
    """q4 decode with 3..16 rows: X row pitch / column offset, weight column and row offsets, output column offset;
    mq4 (k_gemv_mq4, P0K_GEMV_MX=0): both ways the kernel gets its A fragments (LDS copy of aligned X rows, per-unit
    loads otherwise) and waves left without units; mx (the stream kernel's 4x4x4 matrix-core form for 4, 8 and 16
    rows, P0K_GEMV_MX=16): the same calls. Against the oracle's CPU weight model (the one the decode kernels
    compute)."""
    monkeypatch.setenv("P0K_GEMV_MX", "0" if path == "mq4" else "16")
    banner(f"matrix-core decode {path} {kw}")
    c = make_case(seed=31, **kw)
    assert dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"] == ("gemv_mfma" if path == "mq4" else "gemv")
    got = c.run_device(dev)
    assert_close(got, c.run_oracle(weights=oracle.CPU_WEIGHTS), fp16=got.dtype == np.uint16, what=f"decode {kw}")


@pytest.mark.parametrize("M,K,slices", [(2, 8192, 1), (4, 8192, 1), (4, 8192, 0), (3, 16384, 0), (4, 12288, 0)])
def test_matrix_core_stream_long_k(dev, M, K, slices, monkeypatch):
    """q4 decode with 2..4 rows on the stream kernel's matrix-core form at long K: one slice of 8192 (its largest
    X' staging, P0K_GEMV_SLICES=1) and K split over slices that meet through the workspace (the planner's choice for
    these 4 column tiles), against the oracle's CPU weight model."""
    if slices:
        monkeypatch.setenv("P0K_GEMV_SLICES", str(slices))
    monkeypatch.setenv("P0K_GEMV_SN", "0")                        # (M = 2 would take the short-call items)
    banner(f"matrix-core stream M={M} K={K} slices={slices}")
    c = make_case(enc="q4g32a.t64", epi="swiglu", M=M, N=512, K=K, seed=41)
    assert dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"] == "gemv"
    got = c.run_device(dev)
    assert_close(got, c.run_oracle(weights=oracle.CPU_WEIGHTS), what=f"stream M={M} K={K}")


@pytest.mark.parametrize("M,N", [(0, 256), (4, 0), (0, 0)])
def test_empty_calls_write_nothing(dev, M, N):
    """src/ops/gemm.js:312-319: M = 0 or N = 0 makes zero tiles, so the call dispatches nothing and returns 2 M N K
    (0); here the call is validated and returns without a launch, leaving the output as it was."""
    c = make_case(enc="q4g32a.t64", M=4, N=256, K=256, seed=61)
    d = {k: dev.upload(v) for k, v in c.bufs.items()}
    try:
        before = dev.read(d[c.out], np.uint8)
        a = c.args(lambda n: d[n])
        a.update(M=M, N=N)
        assert dev.gemm(a) == 0
        dev.done()
        assert np.array_equal(dev.read(d[c.out], np.uint8), before)
    finally:
        for b in d.values():
            dev.free(b)


@pytest.mark.parametrize("enc,M", [("q4g32a.t64", 1), ("q4g32a.t64", 4), ("q8g64s.t64", 8), ("q4g32a.t64", 300),
                                   ("f16", 300)])
def test_weights_past_4gib_in_a_large_buffer(dev, enc, M):
    """A weight tensor stored 4.25 GiB into one large device buffer (a model shard): `w.off` is folded into the base
    the kernels address from, so their 32-bit offsets only span the tensor itself (the reference binds such a window
    from the 256-byte boundary before it, src/ops/gemm.js:289-296)."""
    c = make_case(enc=enc, epi="f16", M=M, N=256, K=512, seed=71)
    off = (4 << 30) + (256 << 20)
    big = dev.buffer(off + c.bufs["w"].nbytes)
    d = {}
    try:
        dev.upload(c.bufs["w"], dst=big, dst_off=off)
        d = {k: dev.upload(v) for k, v in c.bufs.items() if k != "w"}
        a = c.args(lambda n: big if n == "w" else d[n])
        a["w"]["off"] = off
        dev.gemm(a)
        dev.done()
        out = c.bufs[c.out]
        got = dev.read(d[c.out], out.dtype, out.size)
        assert_close(got, c.run_oracle(), fp16=got.dtype == np.uint16, what=f"{enc} M={M} at 4.25 GiB")
    finally:
        for b in d.values():
            dev.free(b)
        dev.free(big)
        dev.drain_pool()


@pytest.mark.parametrize("narrow", [True, False])
@pytest.mark.parametrize("epi,M,N,K", [("swiglu", 2, 14400, 1024), ("resadd", 3, 16000, 512), ("bias", 4, 14592, 768),
                                       ("f32", 1, 15000, 256), ("swiglu", 1, 16384, 512), ("f16", 1, 4096, 4096),
                                       ("swiglu", 4, 6144, 2048), ("swiglu", 8, 4096, 2048), ("resadd", 16, 14400, 1024),
                                       ("f16", 12, 6144, 4096), ("bias", 5, 4096, 512)])
def test_narrow_decode_items(dev, epi, M, N, K, narrow, monkeypatch):
    """q4 decode calls the planner would split: 64-column items without a K split (default; half-GPU grids, and small
    N with short K; the one-row stream up to 4 rows, k_gemv_mq4 from 5) and, with P0K_GEMV_NARROW=0, 128-column
    items in K slices meeting through the workspace; both against the oracle's CPU weight model, ragged last items
    included."""
    monkeypatch.setenv("P0K_GEMV_NARROW", "1" if narrow else "0")
    monkeypatch.setenv("P0K_GEMV_SN", "0")                        # (N 4096 at one row would take the short-call items)
    banner(f"narrow={narrow} {epi} M={M} N={N} K={K}")
    c = make_case(enc="q4g32a.t64", epi=epi, M=M, N=N, K=K, seed=91)
    t = dev.select_tile(c.args(lambda n: c.bufs[n]))
    assert t["kernel"] == ("gemv" if M <= 4 else "gemv_mfma") and t["BN"] == (64 if narrow else 128)
    got = c.run_device(dev)
    assert_close(got, c.run_oracle(weights=oracle.CPU_WEIGHTS), fp16=got.dtype == np.uint16, what=f"{epi} M={M} N={N}")


@pytest.mark.parametrize("narrow", [True, False])
@pytest.mark.parametrize("enc,epi,M,N,K,mq4", [("q8g64s.t64", "f16", 1, 14336, 4096, "1"),
                                               ("q8g64s.t64", "swiglu", 3, 14400, 1024, "1"),
                                               ("q8g64s.t64", "resadd", 16, 14400, 2048, "1"),
                                               ("f16", "bias", 2, 14336, 2048, "1"), ("f16", "swiglu", 9, 14400, 512, "1"),
                                               ("f16", "f32", 1, 16000, 512, "1"),
                                               ("q4g32a.t64", "swiglu", 8, 4096, 2048, "0"),
                                               ("q4g32a.t64", "f16", 16, 6160, 4096, "0")])
def test_narrow_matrix_core_decode(dev, enc, epi, M, N, K, mq4, narrow, monkeypatch):
    """the matrix-core decode (q8 and f16 weights; q4 with X' staged in LDS under P0K_GEMV_MQ4=0) in 64-column items
    with the 8 waves as K-eighths, against its 128-column items in K slices (P0K_GEMV_NARROW=0): both against the
    oracle's CPU weight model, ragged last items and unaligned N included."""
    monkeypatch.setenv("P0K_GEMV_NARROW", "1" if narrow else "0")
    monkeypatch.setenv("P0K_GEMV_MQ4", mq4)
    monkeypatch.setenv("P0K_GEMV_SN", "0")                  # (q8 N 14336 at one row would take the 16-row items)
    banner(f"narrow={narrow} {enc} {epi} M={M} N={N} K={K} mq4={mq4}")
    c = make_case(enc=enc, epi=epi, M=M, N=N, K=K, seed=93)
    t = dev.select_tile(c.args(lambda n: c.bufs[n]))
    assert t["kernel"] == "gemv_mfma" and t["BN"] == (64 if narrow else 128)
    got = c.run_device(dev)
    assert_close(got, c.run_oracle(weights=oracle.CPU_WEIGHTS), fp16=got.dtype == np.uint16,
                 what=f"{enc} {epi} M={M} N={N} K={K}")


# ------------------------------------------------------------------------------------------------ dequantisation
def _adversarial_q4(rows, K, seed):
    """random codes with (scale, min) words that include far-apart exponents (the decoder's exact-fp32 path)."""
    rng = np.random.default_rng(seed)
    u = rng.integers(0, 2 ** 32, size=(rows // 64) * (K // 32) * 320, dtype=np.uint64).astype(np.uint32).reshape(-1, 320)
    s = rng.integers(0x0001, 0x5800, size=u[:, 256:].shape).astype(np.uint32)        # scales up to ~128, incl. subnormal
    m = rng.integers(0x0000, 0x5C00, size=u[:, 256:].shape).astype(np.uint32) | (rng.integers(0, 2, size=s.shape).astype(np.uint32) << 15)
    u[:, 256:] = s | (m << 16)
    return u.ravel().view(np.uint8).copy()


def _adversarial_q8(rows, K, seed):
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(rows // 64) * (K // 64) * 4224, dtype=np.uint16).astype(np.uint8).reshape(-1, 4224)
    sc = rng.integers(0x0001, 0x5000, size=(b.shape[0], 64)).astype(np.uint16)
    b[:, 4096:] = sc.view(np.uint8).reshape(b.shape[0], 128)
    return b.ravel().copy()


@pytest.mark.parametrize("enc", ["q4g32a.t64", "q8g64s.t64"])
@pytest.mark.parametrize("path", ["gemv", "gemv_short", "gemv_short4", "gemv_mx2", "gemv_mx8", "gemv_mx16", "gemv_mfma",
                                  "gemv_mfma_staged", "mfma"])
def test_dequant_bit_exact(dev, enc, path, monkeypatch):
    """X = unit rows e_k: each output is ONE product 1.0 * W'[n, k], so the fp16 output is the decoded weight itself,
    which must equal the oracle's f16(f32(q*s + mn)) / f16(q*s) bit for bit — on random codes and scale words chosen
    to exercise both decoder paths. (q8 at M = 1 takes the matrix-core GEMV; P0K_GEMV_MF=0 keeps the VALU stream;
    P0K_GEMV_MX=16 the stream kernel's 4x4x4 matrix-core form for q4 with 2..16 rows; P0K_GEMV_MQ4=0 the q4
    matrix-core decode with X' staged in LDS.)"""
    if path.startswith("gemv_mx") and not enc.startswith("q4"):
        pytest.skip("the stream kernel's matrix-core form is q4 only")
    monkeypatch.setenv("P0K_GEMV_SN", "1" if path.startswith("gemv_short") else "0")
    if path == "gemv":
        monkeypatch.setenv("P0K_GEMV_MF", "0")
    if path.startswith("gemv_mx"):
        monkeypatch.setenv("P0K_GEMV_MX", "16")
    if path == "gemv_mfma_staged":
        monkeypatch.setenv("P0K_GEMV_MQ4", "0")
    rows, K = 128, 256
    wb = _adversarial_q4(rows, K, 3) if enc.startswith("q4") else _adversarial_q8(rows, K, 4)
    want = oracle.dequant(enc, wb, rows, K)                                  # [rows][K] fp16 bits
    dw = dev.upload(wb)
    try:
        M = {"gemv": 1, "gemv_short": 1, "gemv_short4": 4, "gemv_mx2": 2, "gemv_mx8": 8, "gemv_mx16": 16, "gemv_mfma": 16, "gemv_mfma_staged": 16, "mfma": K}[path]
        got = np.zeros((K, rows), np.uint16)
        for k0 in range(0, K, M):
            X = np.zeros((M, K), np.float32)
            X[np.arange(M), k0 + np.arange(M)] = 1.0
            dx = dev.upload(oracle.f16_bits(X))
            dy = dev.buffer(M * rows * 2)
            dev.gemm({"w": {"enc": enc, "buf": dw, "off": 0, "bytes": wb.nbytes, "rows": rows, "cols": K},
                      "x": {"buf": dx}, "y": {"buf": dy}, "M": M, "N": rows, "K": K})
            got[k0:k0 + M] = dev.read(dy, np.uint16, M * rows).reshape(M, rows)
            dev.free(dx)
            dev.free(dy)
        assert np.array_equal(got.T, want), f"{np.count_nonzero(got.T != want)} decoded weights differ"
    finally:
        dev.free(dw)


# ------------------------------------------------------------------------------------------------ conv3 / conv
def test_conv3_whole_clip(dev):
    c = make_conv3_case()
    T, H, W, C, N = c.dims
    got = c.run_device(dev)
    cos, _ = cos_maxerr(to_float(got), oracle.cpu_conv3(c.X, c.Wt, T, H, W, C, N))
    assert cos > 0.9995
    assert_close(got, c.run_oracle(), what="conv3")


@pytest.mark.parametrize("tile", [{"BM": 128, "BN": 128}, {"BM": 64, "BN": 64}, {"BM": 32, "BN": 128}, {"BM": 128, "BN": 64}])
def test_conv3_tiles(dev, tile):
    """test/kernels.test.js:113-122: any tile the tuning table can pick gives the same (bit-identical) result."""
    c = make_conv3_case()
    base = c.run_device(dev)
    c.spec["tile"] = tile
    assert np.array_equal(c.run_device(dev), base)


def _conv3_call(dev, c, dw, xbuf, xoff, ybuf, yoff, t0, nf, padL=0, ks=1):
    T, H, W, C, N = c.dims
    dev.gemm({"w": {"enc": c.spec["w"]["enc"], "buf": dw, "off": 0, "bytes": c.bufs["w"].nbytes, "rows": N, "cols": 27 * C},
              "x": {"buf": xbuf, "off": xoff}, "y": {"buf": ybuf, "off": yoff}, "M": nf * H * W, "N": N, "K": 27 * C,
              "conv": {"kind": "conv3", "Hi": H, "Wi": W, "Ci": C, "Ho": H, "Wo": W, "stride": T, "padT": t0,
                       "padL": padL, "ks": ks}})


@pytest.mark.parametrize("dims", [(5, 6, 6, 32, 128), (7, 5, 9, 64, 64), (4, 6, 10, 128, 128)])
def test_conv3_chunks_and_ring_bit_identical(dev, dims):
    """test/kernels.test.js:123-145: 2-frame chunks and a 3-frame ring give output bit-identical to the whole clip."""
    T, H, W, C, N = dims
    c = make_conv3_case(T, H, W, C, N)
    whole = c.run_device(dev)
    fx, fy = H * W * C * 2, H * W * N * 2
    dw, dx = dev.upload(c.bufs["w"]), dev.upload(c.bufs["x"])
    ya, ring = dev.buffer(T * fy), dev.buffer(3 * fx)
    try:
        for t0 in range(0, T, 2):
            padL = max(0, t0 - 1)
            _conv3_call(dev, c, dw, dx, padL * fx, ya, t0 * fy, t0, min(2, T - t0), padL)
        chunks = dev.read(ya, np.uint16, T * H * W * N)
        assert np.array_equal(chunks, whole), "2-frame chunks differ from the whole clip"
        yb = dev.buffer(T * fy)
        for t in range(T):
            for g in sorted({max(0, t - 1), t, min(T - 1, t + 1)}):
                dev.copy(ring, (g % 3) * fx, dx, g * fx, fx)
            _conv3_call(dev, c, dw, ring, 0, yb, t * fy, t, 1, 0, 3)
            dev.done()
        assert np.array_equal(dev.read(yb, np.uint16, T * H * W * N), whole), "3-frame ring differs from the whole clip"
        dev.free(yb)
    finally:
        for b in (dw, dx, ya, ring):
            dev.free(b)


@pytest.mark.parametrize("C", [32, 128])
def test_conv3_pixelnorm(dev, C):
    c = make_conv3_case(C=C, pn=True)
    assert dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"] == ("mfma_dma" if C % 64 == 0 else "mfma")
    assert_close(c.run_device(dev), c.run_oracle(), what=f"conv3 pn C={C}")


@pytest.mark.parametrize("enc", ["f16", "q8g64s.t64"])
@pytest.mark.parametrize("pn", [False, True])
def test_conv3_gather_every_tile(dev, enc, pn, monkeypatch):
    """The load-to-LDS conv3 gather (Ci % 64 == 0; padding taps read a zero block, PixelNorm materialised once per
    input element): every tile matches the oracle and all tiles give the same bits."""
    c = make_conv3_case(T=3, H=10, W=12, C=64, N=256, pn=pn, enc=enc)
    want = c.run_oracle()
    outs = []
    for t in MFMA_TILES:
        banner(f"conv3 gather tile {t} enc {enc} pn {pn}")
        monkeypatch.setenv("P0K_MFMA_TILE", t)
        assert dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"] == "mfma_dma"
        got = c.run_device(dev)
        assert_close(got, want, what=f"conv3 gather tile {t}")
        outs.append(got)
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])


@pytest.mark.parametrize("kw", [dict(), dict(stride=2), dict(up2=True), dict(gn=True), dict(ks=1, pad=0),
                                dict(enc="q4g32a.t64", Ci=64, N=128)], ids=str)
def test_conv2d(dev, kw):
    c = make_conv2d_case(**kw)
    assert_close(c.run_device(dev), c.run_oracle(), what=f"conv2d {kw}")


# ------------------------------------------------------------------------------------------------ rowstats, runtime
def test_rowstats(dev):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((37, 300)) * 2 + 0.5).astype(np.float32)
    for mode in ("ln", "rms"):
        want = np.zeros(80, np.float32)
        oracle.rowstats(x, 37, 296, mode, 1e-6, want, ld=300, c0=4, st_off=3)
        dx, ds = dev.upload(x), dev.buffer(80 * 4)
        dev.rowstats(dx, 37, 296, mode, 1e-6, ds, ld=300, c0=4, st_off=3)
        got = dev.read(ds, np.float32, 80)
        assert np.allclose(got, want, rtol=2e-6, atol=2e-6)
        dev.free(dx)
        dev.free(ds)


@pytest.mark.parametrize("rows,cols,ld,c0", [(64, 4096, 4096, 0), (33, 3072, 3080, 8), (5, 8192, 8192, 0),
                                            (7, 1000, 1004, 4), (3, 9000, 9000, 0), (4, 512, 517, 3)])
def test_rowstats_shapes(dev, rows, cols, ld, c0):
    """k_rowstats_reg (aligned rows of up to 8192 columns held in registers: 1..8 pieces per thread, ragged last
    piece) and k_rowstats (longer or unaligned rows), both modes, against the oracle's two-pass restatement"""
    rng = np.random.default_rng(rows + cols)
    x = (rng.standard_normal((rows, ld)) * 1.5 - 0.25).astype(np.float32)
    for mode in ("ln", "rms"):
        want = np.zeros(2 * (rows + 2), np.float32)
        oracle.rowstats(x, rows, cols, mode, 1e-6, want, ld=ld, c0=c0, st_off=2)
        dx, ds = dev.upload(x), dev.buffer(want.nbytes)
        try:
            dev.rowstats(dx, rows, cols, mode, 1e-6, ds, ld=ld, c0=c0, st_off=2)
            got = dev.read(ds, np.float32, want.size)
        finally:
            dev.free(dx)
            dev.free(ds)
        assert np.allclose(got, want, rtol=2e-6, atol=2e-6), f"{mode} rows {rows} cols {cols}"


def test_pool_reuse_is_zeroed(dev):
    b = dev.upload(np.arange(1000, dtype=np.float32))
    size = b.size
    dev.free(b)
    c = dev.buffer(size)
    assert np.all(dev.read(c, np.float32, 1000) == 0)
    s = dev.pool_stats()
    assert s["reuses"] >= 1
    dev.free(c)


def test_gemm_refuses_foreign_and_oversized_buffers(dev):
    c = make_case(enc="f16", M=4, N=64, K=64)
    d = {k: dev.upload(v) for k, v in c.bufs.items()}
    try:
        a = c.args(lambda n: d[n])
        a["y"]["size"] = d["y"].size * 4
        with pytest.raises(p0k.P0kError, match="exceeds its allocation|needs"):
            dev.gemm(a)
    finally:
        for b in d.values():
            dev.free(b)


# ------------------------------------------------------------------------------------------------ CDNA4 tile shapes
MFMA_TILES = ["128x128", "256x128", "128x256", "256x256"]
TILE_CASES = [
    dict(enc="q4g32a.t64", epi="swiglu", M=300, N=768, K=256, bias=True),
    dict(enc="q8g64s.t64", xmode="rms", epi="resadd", M=270, N=640, K=256, gate=True),
    dict(enc="q4g32a.t64", xmode="lnmod", epi="heads", M=260, N=512, K=128, Hq=2, Hkv=1, Ltot=300, row_off=7),
    dict(enc="f16", xmode="lnmod", epi="bias", M=140, N=384, K=192, res=True),
    dict(enc="q4g32a.t64", epi="onormgate", M=129, N=256, K=64),
    dict(enc="q4g32a.t64", epi="f16", M=200, N=320, K=192, ld_pad=8, k0=64, wk0=32),
    dict(enc="q8g64s.t64", epi="f32", M=333, N=192, K=128, ld_pad=16, k0=8, wk0=64),
]


@pytest.mark.parametrize("kernel", ["mfma_dma", "mfma"])
@pytest.mark.parametrize("kw", TILE_CASES, ids=lambda k: f"{k['enc']}-{k.get('xmode', 'f16')}-{k['epi']}")
def test_every_mfma_tile_matches_oracle(dev, kw, kernel, monkeypatch):
    """Each workgroup tile the library can choose (P0K_MFMA_TILE forces one) of both MFMA kernels (P0K_MFMA_KERNEL=reg
    forces the register-staged one) gives the oracle's result, and all tiles of one kernel give the same bits (the K
    order of an output element does not depend on the tile)."""
    c = make_case(seed=21, **kw)
    want = c.run_oracle()
    if kernel == "mfma":
        monkeypatch.setenv("P0K_MFMA_KERNEL", "reg")
    elif dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"] != "mfma_dma":
        pytest.skip("the call does not qualify for the load-to-LDS kernel")
    outs = []
    for t in MFMA_TILES:
        banner(f"tile {t} {kernel} {kw}")
        monkeypatch.setenv("P0K_MFMA_TILE", t)
        a = c.args(lambda n: c.bufs[n])
        assert dev.select_tile(a)["BM"] == int(t.split("x")[0]) and dev.select_tile(a)["kernel"] == kernel
        got = c.run_device(dev)
        assert_close(got, want, fp16=want.dtype == np.uint16, what=f"tile {t} {kernel}")
        outs.append(got)
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])


@pytest.mark.parametrize("kw", [dict(enc="q4g32a.t64", xmode="lnmod", epi="heads", M=4096, N=4352, K=128, Hq=32, Hkv=1),
                                dict(enc="q8g64s.t64", epi="swiglu", M=4100, N=4608, K=64, bias=True)],
                         ids=["q4-lnmod-heads", "q8-swiglu"])
def test_tail_columns_bit_identical(dev, kw, monkeypatch):
    """A grid whose last round of tiles would be mostly empty runs as two launches: whole column bands of the chosen
    tile, then the remaining columns with smaller tiles. Every tile sums K in the same order, so the result is the
    same bits as one launch (P0K_DMA_TAIL=0)."""
    c = make_case(seed=24, **kw)
    banner(f"tail columns {kw}")
    monkeypatch.setenv("P0K_DMA_TAIL", "0")
    one = c.run_device(dev)
    monkeypatch.delenv("P0K_DMA_TAIL")
    two = c.run_device(dev)
    assert np.array_equal(one, two)
    rows = [(0, 8), (kw["M"] - 8, kw["M"])]
    want = c.bufs[c.out].copy()
    for m0, m1 in rows:
        o = c.run_oracle(m0, m1)
        if kw["epi"] == "heads":
            nh = kw["Hq"] + 2 * kw["Hkv"]
            want.reshape(nh, -1, 128)[:, m0:m1] = o.reshape(nh, -1, 128)[:, m0:m1]
        else:
            want.reshape(kw["M"], -1)[m0:m1] = o.reshape(kw["M"], -1)[m0:m1]
    for m0, m1 in rows:
        if kw["epi"] == "heads":
            nh = kw["Hq"] + 2 * kw["Hkv"]
            assert_close(two.reshape(nh, -1, 128)[:, m0:m1], want.reshape(nh, -1, 128)[:, m0:m1], what="tail rows")
        else:
            assert_close(two.reshape(kw["M"], -1)[m0:m1], want.reshape(kw["M"], -1)[m0:m1], what="tail rows")


@pytest.mark.parametrize("t", MFMA_TILES)
def test_conv3_every_mfma_tile_bit_identical(dev, t, monkeypatch):
    c = make_conv3_case(T=3, H=10, W=12, C=32, N=256, pn=True)
    base = c.run_device(dev)
    monkeypatch.setenv("P0K_MFMA_TILE", t)
    got = c.run_device(dev)
    assert np.array_equal(got, base)
    assert_close(got, c.run_oracle(), what=f"conv3 tile {t}")


def test_q4_256x128_four_wave_grid(dev, monkeypatch):
    """q4 256 x 128 tiles run with 8 waves when the grid holds at most one tile per CU and with 4 waves (two
    workgroups per CU) otherwise. 4096 x 4352 gives 16 x 34 = 544 tiles, so the forced 256 x 128 tile takes the
    4-wave kernel: sampled rows match the oracle and the result is bit-identical to the 256 x 256 tile's."""
    kw = dict(enc="q4g32a.t64", epi="f16", M=4096, N=4352, K=128)
    c = make_case(seed=26, **kw)
    banner(f"q4 256x128 4-wave {kw}")
    monkeypatch.setenv("P0K_DMA_TAIL", "0")
    outs = {}
    for t in ("256x128", "256x256"):
        monkeypatch.setenv("P0K_MFMA_TILE", t)
        sel = dev.select_tile(c.args(lambda n: c.bufs[n]))
        assert sel["kernel"] == "mfma_dma" and sel["BM"] == 256 and sel["BN"] == int(t.split("x")[1])
        outs[t] = c.run_device(dev)
    assert np.array_equal(outs["256x128"], outs["256x256"])
    g = outs["256x128"].reshape(kw["M"], -1)
    for m0, m1 in [(0, 8), (2050, 2058), (4088, 4096)]:
        w = c.run_oracle(m0, m1).reshape(kw["M"], -1)
        assert_close(g[m0:m1], w[m0:m1], what=f"rows {m0}..{m1}")


# ------------------------------------------------------------------------------------------------ runtime robustness
def test_context_plans_for_the_device_cu_count(dev):
    assert dev.cus() == dev.info()["cus"] > 0


def test_alloc_and_free_refused_while_capturing(dev):
    """a buffer clear or hipFree must not land in a captured graph: alloc / free are refused during capture"""
    b = dev.buffer(256)
    dev.graph_begin()
    try:
        with pytest.raises(p0k.P0kError, match="captured into a graph"):
            dev.buffer(256)
        with pytest.raises(p0k.P0kError, match="captured into a graph"):
            lib_free = p0k.lib().p0k_free(dev.ctx, b.ptr)
            p0k._chk(lib_free)
    finally:
        g = dev.graph_end()
    dev.graph_destroy(g)
    dev.free(b)


def test_graph_survives_workspace_growth(dev):
    """A graph captured with a split-K decode call keeps the workspace it was captured with: a later, larger eager
    call grows the workspace (the old one stays allocated until the context goes), and replaying the graph still
    gives the oracle's result."""
    small = make_case(enc="q4g32a.t64", epi="swiglu", M=1, N=1024, K=4096, seed=71, wscale=0.02)
    big = make_case(enc="q4g32a.t64", epi="swiglu", M=8, N=8192, K=4096, seed=72, wscale=0.02)
    for c in (small, big):
        assert dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"].startswith("gemv")
    d = {k: dev.upload(v) for k, v in small.bufs.items()}
    db = {k: dev.upload(v) for k, v in big.bufs.items()}
    try:
        a = small.args(lambda n: d[n])
        dev.gemm(a)                                   # sizes the workspace for the small call
        dev.done()
        dev.graph_begin()
        try:
            dev.gemm(a)
        finally:
            g = dev.graph_end()
        dev.gemm(big.args(lambda n: db[n]))           # larger: grows the workspace
        dev.done()
        zero = np.zeros_like(small.bufs["y"])
        dev.upload(zero, d["y"])
        for _ in range(3):
            dev.graph_launch(g)
            dev.done()
            got = dev.read(d["y"], np.uint16, small.bufs["y"].size)
            assert_close(got, small.run_oracle(weights=oracle.CPU_WEIGHTS), what="graph replay after growth")
        dev.graph_destroy(g)
        assert_close(dev.read(db["y"], np.uint16, big.bufs["y"].size), big.run_oracle(weights=oracle.CPU_WEIGHTS),
                     what="larger eager call")
    finally:
        for b in list(d.values()) + list(db.values()):
            dev.free(b)


@pytest.mark.parametrize("kernel", ["mfma_dma", "mfma"])
def test_heads_tiles_past_n_write_nothing(dev, kernel, monkeypatch):
    """A heads call whose last column tile reaches past N (3 heads of 128 in tiles 256 wide) must not write the
    heads that do not exist: the bytes after the output's stated size stay as they were, for every tile shape."""
    c = make_case(enc="f16", epi="heads", M=70, N=384, K=256, Hq=1, Hkv=1, Ltot=70, seed=95)
    want = c.run_oracle()
    need = c.bufs["y"].nbytes
    guard = np.full(64 * 1024, 0xA5, np.uint8)
    if kernel == "mfma":
        monkeypatch.setenv("P0K_MFMA_KERNEL", "reg")
    for t in MFMA_TILES:
        monkeypatch.setenv("P0K_MFMA_TILE", t)
        banner(f"heads past N: {kernel} tile {t}")
        d = {k: dev.upload(v) for k, v in c.bufs.items() if k != "y"}
        d["y"] = dev.upload(np.concatenate([c.bufs["y"].view(np.uint8), guard]))
        try:
            a = c.args(lambda n: d[n])
            a["y"]["size"] = need
            assert dev.select_tile(a)["kernel"] == kernel
            dev.gemm(a)
            out = dev.read(d["y"], np.uint8)
        finally:
            for b in d.values():
                dev.free(b)
        assert np.array_equal(out[need:need + guard.size], guard), f"{kernel} tile {t}: wrote past the heads output"
        assert_close(out[:need].view(np.uint16), want, what=f"heads past N {kernel} tile {t}")


def test_workspace_growth_stays_bounded(dev):
    """rms X' workspaces for rising M: each grows to a power of two and the one it replaces is freed when no graph was
    captured since it was allocated (at most the first one of the series can predate a graph of an earlier test), so
    the workspaces grow by less than twice the largest need; after a graph capture the replaced one is kept (the graph
    may replay it) and the graph still replays correctly"""
    K = 512
    live0 = dev.workspace_stats()
    for M in (40, 80, 160, 320, 640, 1280):
        c = make_case(enc="q8g64s.t64", xmode="rms", epi="f16", M=M, N=128, K=K, seed=90 + M)
        assert dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"] == "mfma_dma"
        got = c.run_device(dev)
        assert_close(got, c.run_oracle(), what=f"rms M={M}")
        st = dev.workspace_stats()
        assert st["retired_buffers"] <= live0["retired_buffers"] + 1, f"M={M}: workspaces retired without a graph"
        assert st["live_bytes"] <= live0["live_bytes"] + 2 * 1280 * K * 2
    # capture a graph on the current workspace, then grow past it: the old one must be kept and the graph must replay
    c = make_case(enc="q8g64s.t64", xmode="rms", epi="f16", M=64, N=128, K=K, seed=97)
    d = {k: dev.upload(v) for k, v in c.bufs.items()}
    try:
        a = c.args(lambda n: d[n])
        dev.gemm(a)
        dev.done()
        dev.graph_begin()
        try:
            dev.gemm(a)
        finally:
            g = dev.graph_end()
        before = dev.workspace_stats()
        Mbig = (before["live_bytes"] // (2 * K) + 64 + 63) // 64 * 64       # an X' larger than every workspace held
        big = make_case(enc="q8g64s.t64", xmode="rms", epi="f16", M=Mbig, N=128, K=K, seed=98)
        print(f"[p0k-test] workspace growth past a graph: M={Mbig}", flush=True)
        big.run_device(dev)
        assert dev.workspace_stats()["retired_buffers"] == before["retired_buffers"] + 1
        dev.upload(np.zeros_like(c.bufs["y"]), d["y"])
        dev.graph_launch(g)
        dev.done()
        dev.graph_destroy(g)
        assert_close(dev.read(d["y"], np.uint16, c.bufs["y"].size), c.run_oracle(), what="graph replay after growth")
    finally:
        for b in d.values():
            dev.free(b)


SHORT_CASES = [
    dict(M=1, N=4096, K=4096, epi="f16"),
    dict(M=2, N=136, K=96, epi="f32"),
    dict(M=4, N=40, K=32, epi="f16"),          # one unit: the partials need more LDS than X' does
    dict(M=3, N=24, K=1056, epi="bias", bias=True, res=True),
    dict(M=1, N=520, K=16384, epi="resadd", gate=True, bias=True),
    dict(M=4, N=4096, K=4096, epi="resadd", gate=True, bias=True),
    dict(M=1, N=512, K=2048, epi="swiglu", bias=True),
    dict(M=2, N=272, K=3072, epi="swiglu", act="gelu"),
    dict(M=1, N=256, K=512, epi="resadd", store=True, xmode="rms"),
    dict(M=2, N=128, K=1024, epi="f16", xmode="lnmod"),
    dict(M=4, N=64, K=4096, epi="swiglu", xmode="rms", bias=True),
    dict(M=1, N=200, K=256, epi="f16", ld_pad=8, k0=64, wk0=32, n0=8),
    dict(M=2, N=96, K=160, epi="swiglu", wr0=64, ld_pad=16),
]


@pytest.mark.parametrize("kw", SHORT_CASES, ids=lambda k: f"M{k['M']}-N{k['N']}-K{k['K']}-{k.get('xmode', 'f16')}-{k['epi']}")
def test_short_decode_matches_oracle(dev, kw, monkeypatch):
    """The short-call decode (16-row items, every load in flight at once, P0K_GEMV_SN=1 forces it): 1..4 rows, K from
    one unit to its longest (16384), K not a multiple of the 1024-k round, N not a multiple of the item, every
    element-wise epilogue (bias / residual / gate / store / SwiGLU / GeGLU), the rms / lnmod prologues, X pitch and
    column offsets, weight column and row offsets, output column offset; against the oracle's CPU weight model (the
    algebraic form of the decode kernels)."""
    monkeypatch.setenv("P0K_GEMV_SN", "1")
    kw = dict(kw)
    c = make_case(enc="q4g32a.t64", seed=61 + kw["K"] % 97, wscale=0.02, **kw)
    banner(f"short decode {kw}")
    assert dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"] == "gemv_short"
    got = c.run_device(dev)
    assert_close(got, c.run_oracle(weights=oracle.CPU_WEIGHTS), fp16=got.dtype == np.uint16, what=f"short {kw}")


SHORT_CASES_Q8 = [
    dict(M=1, N=4096, K=4096, epi="f16"),
    dict(M=2, N=136, K=128, epi="f32"),
    dict(M=4, N=40, K=64, epi="f16"),           # one unit: the partials need more LDS than X' does
    dict(M=3, N=24, K=1088, epi="bias", bias=True, res=True),
    dict(M=1, N=520, K=8192, epi="resadd", gate=True, bias=True),
    dict(M=4, N=1024, K=4096, epi="resadd", gate=True, bias=True),
    dict(M=1, N=512, K=2048, epi="swiglu", bias=True),
    dict(M=2, N=272, K=3072, epi="swiglu", act="gelu"),
    dict(M=1, N=256, K=512, epi="resadd", store=True, xmode="rms"),
    dict(M=2, N=128, K=1024, epi="f16", xmode="lnmod"),
    dict(M=1, N=200, K=256, epi="f16", ld_pad=8, k0=64, wk0=64, n0=8),
    dict(M=2, N=96, K=192, epi="swiglu", wr0=64, ld_pad=16),
]


@pytest.mark.parametrize("kw", SHORT_CASES_Q8, ids=lambda k: f"M{k['M']}-N{k['N']}-K{k['K']}-{k.get('xmode', 'f16')}-{k['epi']}")
def test_short_decode_q8_matches_oracle(dev, kw, monkeypatch):
    """The short-call decode with q8 weights (64-k units, four 16-byte code loads each; P0K_GEMV_SN=1 forces it): 1..4
    rows, K from one unit to its longest (8192), K not a multiple of the 2048-k round, N not a multiple of the item,
    the element-wise epilogues, rms / lnmod, offsets; against the oracle's CPU weight model."""
    monkeypatch.setenv("P0K_GEMV_SN", "1")
    kw = dict(kw)
    c = make_case(enc="q8g64s.t64", seed=71 + kw["K"] % 89, wscale=0.02, **kw)
    banner(f"short decode q8 {kw}")
    assert dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"] == "gemv_short"
    got = c.run_device(dev)
    assert_close(got, c.run_oracle(weights=oracle.CPU_WEIGHTS), fp16=got.dtype == np.uint16, what=f"short q8 {kw}")


SHORT_CASES_F16 = [
    dict(M=1, N=4096, K=4096, epi="f16"),
    dict(M=2, N=136, K=128, epi="f32"),
    dict(M=4, N=40, K=64, epi="f16"),           # one unit: the partials need more LDS than X' does
    dict(M=3, N=24, K=1088, epi="bias", bias=True, res=True),
    dict(M=1, N=520, K=8192, epi="resadd", gate=True, bias=True),
    dict(M=4, N=1024, K=4096, epi="resadd", gate=True, bias=True),
    dict(M=1, N=512, K=2048, epi="swiglu", bias=True),
    dict(M=2, N=272, K=3072, epi="swiglu", act="gelu"),
    dict(M=1, N=256, K=512, epi="resadd", store=True, xmode="rms"),
    dict(M=2, N=128, K=1024, epi="f16", xmode="lnmod"),
    dict(M=1, N=200, K=256, epi="f16", ld_pad=8, k0=64, wk0=24, n0=8),
    dict(M=2, N=96, K=192, epi="swiglu", wr0=64, ld_pad=16),
]


@pytest.mark.parametrize("kw", SHORT_CASES_F16, ids=lambda k: f"M{k['M']}-N{k['N']}-K{k['K']}-{k.get('xmode', 'f16')}-{k['epi']}")
def test_short_decode_f16_matches_oracle(dev, kw, monkeypatch):
    """The short-call decode with f16 weights (64-k units of 128-byte row runs, P0K_GEMV_SN=1 forces it): 1..4 rows, K
    from one unit to its longest (8192), N not a multiple of the item, the element-wise epilogues, rms / lnmod, weight
    and X offsets; against the oracle."""
    monkeypatch.setenv("P0K_GEMV_SN", "1")
    kw = dict(kw)
    c = make_case(enc="f16", seed=79 + kw["K"] % 83, wscale=0.02, **kw)
    banner(f"short decode f16 {kw}")
    assert dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"] == "gemv_short"
    got = c.run_device(dev)
    assert_close(got, c.run_oracle(weights=oracle.CPU_WEIGHTS), fp16=got.dtype == np.uint16, what=f"short f16 {kw}")


def test_caller_captured_stream_keeps_its_workspace(dev):
    """A caller that captures the context's stream itself (p0k_ctx_stream + the HIP graph API) around an rms call:
    a later call that grows the X' workspace must keep the one the caller's graph uses, and the graph replays
    correctly."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    stream = p0k.lib().p0k_ctx_stream(dev.ctx)
    assert stream
    K = 512
    c = make_case(enc="q8g64s.t64", xmode="rms", epi="f16", M=64, N=128, K=K, seed=99)
    d = {k: dev.upload(v) for k, v in c.bufs.items()}
    graph, exe = C.c_void_p(), C.c_void_p()
    try:
        a = c.args(lambda n: d[n])
        dev.gemm(a)                                    # sizes the workspace outside the capture
        dev.done()
        assert hip.hipStreamBeginCapture(C.c_void_p(stream), 1) == 0          # thread-local capture mode
        try:
            dev.gemm(a)
        finally:
            assert hip.hipStreamEndCapture(C.c_void_p(stream), C.byref(graph)) == 0
        assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, C.c_size_t(0)) == 0
        before = dev.workspace_stats()
        Mbig = (before["live_bytes"] // (2 * K) + 64 + 63) // 64 * 64
        big = make_case(enc="q8g64s.t64", xmode="rms", epi="f16", M=Mbig, N=128, K=K, seed=100)
        print(f"[p0k-test] growth past a caller's capture: M={Mbig}", flush=True)
        big.run_device(dev)
        assert dev.workspace_stats()["retired_buffers"] == before["retired_buffers"] + 1
        dev.upload(np.zeros_like(c.bufs["y"]), d["y"])
        assert hip.hipGraphLaunch(exe, C.c_void_p(stream)) == 0
        dev.done()
        assert_close(dev.read(d["y"], np.uint16, c.bufs["y"].size), c.run_oracle(), what="caller's graph replay")
    finally:
        if exe:
            hip.hipGraphExecDestroy(exe)
        if graph:
            hip.hipGraphDestroy(graph)
        for b in d.values():
            dev.free(b)
