"""Parity at the benchmark sizes (BASELINE.json configs[1..4] and the attention consumer), on the GPU.

The oracle cannot redo a whole 4096-token GEMM in seconds, so each case checks what does not depend on the size:
every output row for the decode shapes (M <= 16: the whole call is cheap), and blocks of rows at the start, middle
and end of the larger calls (rows are independent: the oracle restricted to rows m0..m1 computes exactly those
outputs), with the same fp16 tolerance as the small cases (cases.assert_close). conv3 at the full clip size: sampled
image rows of the first, a middle and the last frame against the oracle, and 4-frame ring calls bit-identical to
the whole clip. Attention: sampled queries of sampled heads against a float64 numpy softmax(Q K^T / sqrt(128)) V."""
import numpy as np
import pytest

import oracle
import p0k
from cases import assert_close, make_case, make_conv3_case
from test_gemm_gpu import _conv3_call

pytestmark = pytest.mark.gpu


def banner(s):
    print(s, flush=True)


def rows_of(case, got, want, ranges):
    """compare the output rows in `ranges` (y is [M][ld], or [heads][Ltot][128] for the heads epilogue)"""
    sp = case.spec
    if sp["epi"] == "heads":
        h = sp["heads"]
        nh = h["Hq"] + 2 * h["Hkv"]
        g, w = got.reshape(nh, h["Ltot"], 128), want.reshape(nh, h["Ltot"], 128)
        for m0, m1 in ranges:
            assert_close(g[:, m0:m1], w[:, m0:m1], what=f"rows {m0}..{m1}")
        return
    ld = sp["y"].get("ld") or (sp["N"] // 2 if sp["epi"] == "swiglu" else sp["N"])
    g, w = got.reshape(sp["M"], -1), want.reshape(sp["M"], -1)
    assert g.shape[1] == ld
    for m0, m1 in ranges:
        assert_close(g[m0:m1], w[m0:m1], fp16=got.dtype == np.uint16, what=f"rows {m0}..{m1}")


def oracle_rows(case, ranges, weights):
    """the oracle's output with the rows in `ranges` computed (the other rows hold the initial output buffer)"""
    want = case.bufs[case.out].copy()
    for m0, m1 in ranges:
        o = case.run_oracle(m0, m1, weights=weights)
        if case.spec.get("epi") == "heads":
            h = case.spec["heads"]
            nh = h["Hq"] + 2 * h["Hkv"]
            want.reshape(nh, h["Ltot"], 128)[:, m0:m1] = o.reshape(nh, h["Ltot"], 128)[:, m0:m1]
        else:
            want.reshape(case.spec["M"], -1)[m0:m1] = o.reshape(case.spec["M"], -1)[m0:m1]
    return want


@pytest.mark.parametrize("M,path", [(1, "stream"), (2, "mx"), (4, "mx"), (8, "mx"), (16, "mx"), (4, "mq4"), (16, "mq4"),
                                    (16, "staged")])
def test_decode_q4_swiglu_full(dev, M, path, monkeypatch):
    """q4 N = 14336 (gate | up: 28672 weight rows), K = 4096, SwiGLU; every output row. mx: the stream
    kernel with its 4x4x4 matrix-core dot products (P0K_GEMV_MX=16); mq4: k_gemv_mq4 (P0K_GEMV_MX=0); staged: the
    matrix-core decode with X' staged in LDS before the stream (P0K_GEMV_MX=0 P0K_GEMV_MQ4=0)."""
    monkeypatch.setenv("P0K_GEMV_MX", "16" if path == "mx" else "0")
    if path == "staged":
        monkeypatch.setenv("P0K_GEMV_MQ4", "0")
    banner(f"full-size decode M={M} path={path}")
    c = make_case(enc="q4g32a.t64", epi="swiglu", M=M, N=28672, K=4096, seed=101, wscale=0.02)
    t = dev.select_tile(c.args(lambda n: c.bufs[n]))
    assert t["kernel"] == ("gemv" if path in ("stream", "mx") else "gemv_mfma")
    got = c.run_device(dev)
    assert_close(got, c.run_oracle(weights=oracle.CPU_WEIGHTS), what=f"decode M={M}")


@pytest.mark.parametrize("enc,epi,N", [("q8g64s.t64", "swiglu", 28672), ("f16", "swiglu", 28672),
                                       ("q4g32a.t64", "f16", 14336)], ids=["q8-swiglu", "f16-swiglu", "q4-plain"])
def test_decode_m1_other_weights_full(dev, enc, epi, N):
    """configs[1]'s shape at M = 1 with q8 and f16 weights (the matrix-core GEMV), and the plain q4 GEMV N = 14336,
    whose 112 column tiles split K in two and meet through the workspace; every output row."""
    banner(f"full-size decode M=1 {enc} {epi} N={N}")
    c = make_case(enc=enc, epi=epi, M=1, N=N, K=4096, seed=105, wscale=0.02)
    got = c.run_device(dev)
    assert_close(got, c.run_oracle(weights=oracle.CPU_WEIGHTS), what=f"decode M=1 {enc} {epi}")


FULL = {
    "prefill_q8_rms_resadd": dict(enc="q8g64s.t64", xmode="rms", epi="resadd", M=2048, N=4096, K=4096, wscale=0.02),
    "dit_qkv_q4_lnmod_heads": dict(enc="q4g32a.t64", xmode="lnmod", epi="heads", M=4096, N=9216, K=3072, Hq=24,
                                   Hkv=24, wscale=0.02, rope_grid_w=64),
    "dit_up_q4_geglu": dict(enc="q4g32a.t64", epi="swiglu", act="gelu", M=4096, N=24576, K=3072, wscale=0.02),
    "prefill_q8_rms_bias_f16res": dict(enc="q8g64s.t64", xmode="rms", epi="bias", res=True, M=2048, N=4096, K=4096,
                                       wscale=0.02),
}


@pytest.mark.parametrize("name", list(FULL))
def test_prefill_full(dev, name):
    """configs[2] and configs[3](a), (b) at their sizes: row blocks at the start, middle and end of M."""
    kw = FULL[name]
    banner(f"full-size {name}")
    c = make_case(seed=102, **kw)
    assert dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"] == "mfma_dma"
    got = c.run_device(dev)
    M = kw["M"]
    ranges = [(0, 8), (M // 2 - 3, M // 2 + 5), (M - 8, M)]
    rows_of(c, got, oracle_rows(c, ranges, oracle.KERNEL_WEIGHTS), ranges)


def test_conv3_full_clip(dev):
    """3x3x3 conv 128 -> 128 over 13 x 92 x 160: sampled image rows of frames 0, 6 and 12 against the
    oracle (the first and last frames repeat themselves in time: the input frame index is clamped to the clip, as in
    test/kernels.test.js:56), then 4-frame ring calls (each output frame t from a ring holding t - 1 .. t + 1) and
    linear chunks of two output frames per call (padT = t0, the chunk's input starting at frame padL = max(0, t0 - 1))
    bit-identical to the whole clip."""
    T, H, W, C, N = 13, 92, 160, 128, 128
    banner("full-size conv3")
    c = make_conv3_case(T, H, W, C, N, seed=103, wscale=0.02)
    whole = c.run_device(dev)
    ranges = [(t * H * W + y * W, t * H * W + (y + 1) * W) for t, y in ((0, 0), (6, 45), (12, 91))]
    want = oracle_rows(c, ranges, oracle.KERNEL_WEIGHTS)
    g, w = whole.reshape(T * H * W, N), want.reshape(T * H * W, N)
    for m0, m1 in ranges:
        assert_close(g[m0:m1], w[m0:m1], what=f"conv3 voxels {m0}..{m1}")
    fx, fy = H * W * C * 2, H * W * N * 2
    dw, dx = dev.upload(c.bufs["w"]), dev.upload(c.bufs["x"])
    ring, yb = dev.buffer(4 * fx), dev.buffer(T * fy)
    try:
        for t in range(T):
            for gf in sorted({max(0, t - 1), t, min(T - 1, t + 1)}):
                dev.copy(ring, (gf % 4) * fx, dx, gf * fx, fx)
            _conv3_call(dev, c, dw, ring, 0, yb, t * fy, t, 1, 0, 4)
            dev.done()
        assert np.array_equal(dev.read(yb, np.uint16, T * H * W * N), whole), "4-frame ring differs from the whole clip"
        # linear chunks: output frames t0, t0 + 1 from input frames padL .. t0 + 2, the chunk's start given by padL
        yc = dev.buffer(T * fy)
        for t0 in range(0, T, 2):
            padL = max(0, t0 - 1)
            _conv3_call(dev, c, dw, dx, padL * fx, yc, t0 * fy, t0, min(2, T - t0), padL)
        dev.done()
        chunks = dev.read(yc, np.uint16, T * H * W * N)
        dev.free(yc)
        assert np.array_equal(chunks, whole), "2-frame linear chunks differ from the whole clip"
    finally:
        for b in (dw, dx, ring, yb):
            dev.free(b)


def test_attention_full(dev):
    """the attention consumer at the bench size (24 heads, 4096 x 4096, no mask): 32 sampled queries in each of 4
    sampled heads against float64 numpy."""
    H, L, D = 24, 4096, 128
    banner("full-size attention")
    r = np.random.default_rng(104)
    f16 = lambda a: oracle.f16_bits(a.astype(np.float32))
    q, k, v = f16(0.5 * r.standard_normal(H * L * D)), f16(0.5 * r.standard_normal(H * L * D)), f16(r.standard_normal(H * L * D))
    dq, dk, dv, do = dev.upload(q), dev.upload(k), dev.upload(v), dev.buffer(L * H * D * 2)
    try:
        dev.attention({"q": {"buf": dq}, "k": {"buf": dk}, "v": {"buf": dv}, "o": {"buf": do}, "Lq": L, "Lk": L,
                       "Hq": H, "Hkv": H})
        o = oracle.h2f(dev.read(do, np.uint16, L * H * D)).reshape(L, H, D)
    finally:
        for b in (dq, dk, dv, do):
            dev.free(b)
    Q, K, V = (oracle.h2f(a).astype(np.float64).reshape(H, L, D) for a in (q, k, v))
    rows = np.concatenate([np.arange(0, 8), np.arange(2044, 2052), r.choice(L, 16, replace=False)])
    for h in (0, 7, 16, 23):
        s = Q[h, rows] @ K[h].T / np.sqrt(128.0)
        p = np.exp(s - s.max(1, keepdims=True))
        want = (p / p.sum(1, keepdims=True)) @ V[h]
        got = o[rows, h]
        err = np.abs(got - want)
        bound = 2 ** -8 * np.abs(want).max() + 2 ** -9 * np.abs(want)
        assert np.all(err <= bound), f"head {h}: max err {err.max()} (bound {bound.max()})"
