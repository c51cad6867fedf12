"""attention (src/ops/attention.js:168), head size 128 — the consumer of the `heads` epilogue's output.

CPU: the oracle (a restatement of the test suite's cpuAttn, test/kernels.test.js:30-49) against an independent numpy
formulation (masked softmax(Q K^T scale) V per head), the three mask modes, GQA and the soft cap.
GPU: the HIP kernel against the oracle on the reference's own cases (test/kernels.test.js:148-152, seeds and scales
as attnSetup at :153-157) plus ragged lengths, GQA 8:1, an offset O with ld > Hq * 128, and the soft cap.
Tolerance (fp16 output): |got - want| <= 2^-8 * max|want| + 2^-9 |want|, and the reference's cos > 0.9995; P is
rounded to fp16 before the P.V products, as in the reference kernels (pv16)."""
import numpy as np
import pytest

import oracle
import p0k

ATT = [  # test/kernels.test.js:148-152
    dict(label="no mask", Hq=2, Hkv=2, Lq=96, Lk=96, mode=0),
    dict(label="causal + valid length 80, GQA 4:2", Hq=4, Hkv=2, Lq=96, Lk=96, mode=1, nvalid=80),
    dict(label="valid length 77 of 100 keys, 64 queries", Hq=2, Hkv=2, Lq=64, Lk=100, mode=2, nvalid=77),
]
MORE = [
    dict(label="ragged 300 x 257, GQA 8:1", Hq=8, Hkv=1, Lq=300, Lk=257, mode=0),
    dict(label="causal 200, valid 150", Hq=2, Hkv=1, Lq=200, Lk=200, mode=1, nvalid=150),
    dict(label="one query", Hq=3, Hkv=3, Lq=1, Lk=130, mode=2, nvalid=129),
    dict(label="soft cap 1.0", Hq=2, Hkv=2, Lq=70, Lk=90, mode=0, cap=1.0),
]


def setup(c, seed, qs=0.5):
    """attnSetup (test/kernels.test.js:153-157): Q, K = f16(randn * 0.5), V = f16(randn)."""
    D = 128
    q = oracle.f16_bits(oracle.randn(c["Hq"] * c["Lq"] * D, seed, qs))
    k = oracle.f16_bits(oracle.randn(c["Hkv"] * c["Lk"] * D, seed + 1, qs))
    v = oracle.f16_bits(oracle.randn(c["Hkv"] * c["Lk"] * D, seed + 2))
    return q, k, v


def numpy_attention(q, k, v, c):
    D, Hq, Hkv, Lq, Lk = 128, c["Hq"], c["Hkv"], c["Lq"], c["Lk"]
    Q = oracle.h2f(q).astype(np.float64).reshape(Hq, Lq, D)
    K = oracle.h2f(k).astype(np.float64).reshape(Hkv, Lk, D)
    V = oracle.h2f(v).astype(np.float64).reshape(Hkv, Lk, D)
    nv = c.get("nvalid", Lk)
    i, j = np.arange(Lq)[:, None], np.arange(Lk)[None, :]
    vis = {0: np.ones((Lq, Lk), bool), 1: j <= np.minimum(i, nv - 1), 2: np.broadcast_to(j < nv, (Lq, Lk))}[c["mode"]]
    out = np.zeros((Lq, Hq, D))
    for h in range(Hq):
        s = Q[h] @ K[h // (Hq // Hkv)].T / np.sqrt(128.0)
        if c.get("cap"):
            s = c["cap"] * np.tanh(s / c["cap"])
        s = np.where(vis, s, -np.inf)
        p = np.exp(s - s.max(1, keepdims=True))
        out[:, h] = (p / p.sum(1, keepdims=True)) @ V[h // (Hq // Hkv)]
    return out.reshape(Lq, Hq * D)


@pytest.mark.parametrize("c", ATT + MORE, ids=lambda c: c["label"])
def test_oracle_is_masked_softmax(c):
    q, k, v = setup(c, 21)
    got = oracle.h2f(oracle.attention(q, k, v, c["Lq"], c["Lk"], c["Hq"], c["Hkv"], c["mode"], c.get("nvalid"),
                                      cap=c.get("cap", 0.0))).reshape(c["Lq"], -1)
    want = numpy_attention(q, k, v, c)
    np.testing.assert_allclose(got, want, rtol=2 ** -10, atol=2 ** -14)


def test_attention_checks():
    base = dict(Lq=4, Lk=4, Hq=2, Hkv=2)
    bufs = {n: np.zeros(4096, np.uint16) for n in "qkvo"}

    def check(**kw):
        a = {n: {"buf": bufs[n]} for n in "qkvo"}
        a.update(base)
        a.update(kw)
        return p0k.lib().p0k_attention_check(p0k.C.byref(p0k.attn_args(a, p0k.numpy_resolve)))
    assert check() == 0
    assert check(Hkv=3) == 1 and "multiple of Hkv" in p0k.lib().p0k_last_error().decode()
    assert check(mode=3) == 1
    assert check(mode=2, nvalid=9) == 1
    assert check(Lq=64) == 1 and "needs" in p0k.lib().p0k_last_error().decode()


# ------------------------------------------------------------------------------------------------ GPU
def cos_and_err(got, want):
    g, w = got.astype(np.float64).ravel(), want.astype(np.float64).ravel()
    return g @ w / (np.linalg.norm(g) * np.linalg.norm(w) + 1e-30), np.abs(g - w)


@pytest.mark.gpu
@pytest.mark.parametrize("bq", [128, 256])
@pytest.mark.parametrize("c", ATT + MORE, ids=lambda c: c["label"])
def test_attention_matches_oracle(dev, c, bq, monkeypatch):
    """Both workgroup sizes (128 / 256 queries) on every case; the library picks 256 only for large grids."""
    monkeypatch.setenv("P0K_ATTN_BQ", str(bq))
    print(f"attention bq={bq} {c}", flush=True)
    q, k, v = setup(c, 21, 1.0 if c.get("cap") else 0.5)
    Lq, Hq = c["Lq"], c["Hq"]
    ld = Hq * 128 + (8 if c["mode"] == 2 else 0)                       # a padded O row for one case
    dq, dk, dv = dev.upload(q), dev.upload(k), dev.upload(v)
    do = dev.buffer(Lq * ld * 2 + 16)
    try:
        flops = dev.attention({"q": {"buf": dq}, "k": {"buf": dk}, "v": {"buf": dv}, "o": {"buf": do, "off": 16, "ld": ld},
                               "Lq": Lq, "Lk": c["Lk"], "Hq": Hq, "Hkv": c["Hkv"], "mode": c["mode"],
                               "nvalid": c.get("nvalid", 0), "cap": c.get("cap", 0.0)})
        assert flops == 4 * Lq * c["Lk"] * 128 * Hq
        o = dev.read(do, np.uint16, (Lq * ld * 2 + 16) // 2)
        assert np.all(o[:8] == 0)
        got = o[8:8 + Lq * ld].reshape(Lq, ld)
        if ld > Hq * 128:
            assert np.all(got[:, Hq * 128:] == 0)
        got = oracle.h2f(got[:, :Hq * 128].ravel())
        want = oracle.h2f(oracle.attention(q, k, v, Lq, c["Lk"], Hq, c["Hkv"], c["mode"], c.get("nvalid"),
                                           cap=c.get("cap", 0.0)))
        cos, err = cos_and_err(got, want)
        assert cos > 0.9995
        bound = 2 ** -8 * np.abs(want).max() + 2 ** -9 * np.abs(want)
        assert np.all(err <= bound), f"max err {err.max()} (bound {bound.max()})"
    finally:
        for d in (dq, dk, dv, do):
            dev.free(d)


@pytest.mark.gpu
@pytest.mark.parametrize("pattern", ["slow ramp", "fast ramp", "late spike", "falling"])
def test_attention_moving_maximum(dev, pattern):
    """Scores whose row maximum keeps moving across the 64-key tiles: the kernel keeps the subtracted maximum until a
    row's maximum outgrows it by more than 8 in the log2 domain (P up to 2^8 meanwhile) and rescales O and l when it
    moves. Every query sees s_j = g(j) + noise: a slow ramp (about 4 log2 units per tile: the maximum moves every other
    tile), a fast ramp (16 per tile: every tile), one late spike (25 units in one tile) and a falling ramp (the maximum
    is set by the first tile and never moves); against float64 numpy with the file's fp16 tolerance."""
    Hq, Lq, Lk, D = 2, 128, 512, 128
    j = np.arange(Lk, dtype=np.float64)
    g = {"slow ramp": 0.5 * j, "fast ramp": 2.0 * j, "late spike": np.where(j == 300, 200.0, 0.0),
         "falling": 60.0 - 0.1 * j}[pattern]
    rng = np.random.default_rng(7)
    # q = (1, ..., 1) + noise, k_j = g(j) / 128 (1, ..., 1) + noise: q . k_j = g(j) + O(noise)
    Q = np.ones((Hq, Lq, D)) + 0.05 * rng.standard_normal((Hq, Lq, D))
    K = np.repeat((g / 128.0)[None, :, None], D, axis=2).repeat(Hq, axis=0) + 0.05 * rng.standard_normal((Hq, Lk, D))
    V = rng.standard_normal((Hq, Lk, D))
    q, k, v = (oracle.f16_bits(a.astype(np.float32).ravel()) for a in (Q, K, V))
    c = dict(Hq=Hq, Hkv=Hq, Lq=Lq, Lk=Lk, mode=0)
    dq, dk, dv, do = dev.upload(q), dev.upload(k), dev.upload(v), dev.buffer(Lq * Hq * D * 2)
    try:
        dev.attention({"q": {"buf": dq}, "k": {"buf": dk}, "v": {"buf": dv}, "o": {"buf": do}, "Lq": Lq, "Lk": Lk,
                       "Hq": Hq, "Hkv": Hq})
        got = oracle.h2f(dev.read(do, np.uint16, Lq * Hq * D))
    finally:
        for d in (dq, dk, dv, do):
            dev.free(d)
    want = numpy_attention(q, k, v, c).ravel()
    err = np.abs(got - want)
    bound = 2 ** -8 * np.abs(want).max() + 2 ** -9 * np.abs(want)
    assert np.all(err <= bound), f"{pattern}: max err {err.max()} (bound {bound.max()})"
