"""Pins of the oracle's gemm (or_gemm) and rowstats — no GPU.

Each case is computed a second time by an independent numpy formulation written from the reference's formulas
(src/ops/gemm.js prologues :60-95, epilogues :191-254; docs/FORMAT.md), with float64 sums, and by closed forms:
the textbook 3-D cross-correlation for conv3, norm preservation of the RoPE rotation, V passing through the heads
epilogue unchanged, and bit-identity of time-chunked / ring-buffered conv3 calls with the whole clip.
"""
import math

import numpy as np
import pytest

import oracle
from cases import (assert_close, cos_maxerr, make_case, make_conv2d_case, make_conv3_case, rope_table_2d, to_float)


def f16r(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def weights_f(case):
    s = case.spec["w"]
    if s["enc"] == "f16":
        return oracle.h2f(case.bufs["w"].view(np.uint16)).reshape(s["rows"], s["cols"]).astype(np.float64)
    return oracle.h2f(oracle.dequant(s["enc"], case.bufs["w"], s["rows"], s["cols"])).astype(np.float64)


def xprime(case):
    s, b = case.spec, case.bufs
    M, K = s["M"], s["K"]
    x = s["x"]
    ld, k0 = x["ld"], x["k0"]
    if x["mode"] == "f16":
        X = oracle.h2f(b["x"]).reshape(M, ld)[:, k0:k0 + K]
        return X.astype(np.float64)
    X = b["x"].reshape(M, ld)[:, k0:k0 + K].astype(np.float32)
    st = b["st"].reshape(-1, 2)[:M]
    if x["mode"] == "rms":
        g = b["pv"][k0:k0 + K]
        return f16r((X * st[:, 1:2]) * g).astype(np.float64)
    sc = b["pv"][k0:k0 + K]
    sh = b["pv"][s["pv"]["stride"] + k0: s["pv"]["stride"] + k0 + K]
    return f16r(((X - st[:, 0:1]) * st[:, 1:2]) * (np.float32(1) + sc) + sh).astype(np.float64)


def acc_numpy(case):
    s = case.spec
    N, K = s["N"], s["K"]
    Wd = weights_f(case)
    if s["epi"] == "swiglu":
        rows = np.empty(N, np.int64)
        rows[0::2] = s["wr0"] + np.arange(N // 2)
        rows[1::2] = s["wr1"] + np.arange(N // 2)
    else:
        rows = np.minimum(s["wr0"] + np.arange(N), s["w"]["rows"] - 1)
    Wsel = Wd[rows][:, s["wk0"]:s["wk0"] + K]
    return xprime(case) @ Wsel.T


def epi_numpy(case, acc):
    s, b = case.spec, case.bufs
    M, N = s["M"], s["N"]
    epi = s["epi"]
    y = b["y"].copy()
    if epi == "heads":
        h = s["heads"]
        out = y.reshape(-1, h["Ltot"], 128).astype(np.uint16)
        rp = b["rope"].reshape(h["Ltot"], 64, 2)
        for hd in range(N // 128):
            v = acc[:, hd * 128:(hd + 1) * 128].copy()
            sec = 0 if hd < h["Hq"] else (1 if hd < h["Hq"] + h["Hkv"] else 2)
            if sec < 2:
                inv = 1.0 / np.sqrt((v * v).sum(1, keepdims=True) / 128 + h["eps"])
                v = v * inv * b["ev"][(128 if sec else 0):(256 if sec else 128)]
                rows = h["rowOff"] + np.arange(M)
                c, sn = rp[rows, :, 0].astype(np.float64), rp[rows, :, 1].astype(np.float64)
                if h["ropeMode"] == "half":
                    lo, hi = v[:, :64].copy(), v[:, 64:].copy()
                    v[:, :64], v[:, 64:] = lo * c - hi * sn, hi * c + lo * sn
                else:
                    a0, a1 = v[:, 0::2].copy(), v[:, 1::2].copy()
                    v[:, 0::2], v[:, 1::2] = a0 * c - a1 * sn, a0 * sn + a1 * c
            out[hd, h["rowOff"]:h["rowOff"] + M] = v.astype(np.float32).astype(np.float16).view(np.uint16)
        return out.ravel()
    ld, n0 = s["y"]["ld"], s["y"]["n0"]
    if epi == "swiglu":
        g, u = acc[:, 0::2].copy(), acc[:, 1::2].copy()
        if "bv" in s:
            o, up = s["bv"]["off"], s["bv"]["up"]
            g += b["bv"][o:o + N // 2]
            u += b["bv"][o + up:o + up + N // 2]
        if s.get("act") == "gelu":
            t = np.clip(0.7978845608 * (g + 0.044715 * g ** 3), -15, 15)
            a = g * 0.5 * (1 + np.tanh(t))
        else:
            a = g / (1 + np.exp(-g))
        r = y.reshape(M, ld)
        r[:, n0:n0 + N // 2] = (a * u).astype(np.float32).astype(np.float16).view(np.uint16)
        return y
    if epi in ("f32", "resadd"):
        r = y.reshape(M, ld)
        if epi == "f32":
            r[:, n0:n0 + N] = acc
        else:
            gt = b["ev"][s["ev"]["off"]:s["ev"]["off"] + N] if "ev" in s else 1.0
            bb = b["bv"][s["bv"]["off"]:s["bv"]["off"] + N] if "bv" in s else 0.0
            prev = 0.0 if s.get("store") else r[:, n0:n0 + N].astype(np.float64)
            r[:, n0:n0 + N] = prev + gt * (acc + bb)
        return y
    r = y.reshape(M, ld)
    if epi == "f16":
        r[:, n0:n0 + N] = acc.astype(np.float32).astype(np.float16).view(np.uint16)
    elif epi == "bias":
        v = acc + b["ev"][s["ev"]["off"]:s["ev"]["off"] + N]
        if s.get("res"):
            v = v + oracle.h2f(r[:, n0:n0 + N])
        r[:, n0:n0 + N] = v.astype(np.float32).astype(np.float16).view(np.uint16)
    elif epi == "onormgate":
        Lg = s["heads"]["Ltot"]
        gt = oracle.h2f(b["gt"]).reshape(M, Lg)[:, n0:n0 + N].astype(np.float64)
        for nb in range(0, N, 128):
            v = acc[:, nb:nb + 128]
            inv = 1.0 / np.sqrt((v * v).sum(1, keepdims=True) / 128 + s["heads"]["eps"])
            o = v * inv * b["ev"][:128] / (1 + np.exp(-gt[:, nb:nb + 128]))
            r[:, n0 + nb:n0 + nb + 128] = o.astype(np.float32).astype(np.float16).view(np.uint16)
    return y


CASES = [
    dict(enc="f16", epi="f16", M=33, N=192, K=256),
    dict(enc="q4g32a.t64", epi="f16", M=5, N=128, K=256),
    dict(enc="q8g64s.t64", epi="f16", M=9, N=128, K=256),
    dict(enc="q4g32a.t64", epi="f32", M=4, N=64, K=128, ld_pad=8, k0=32, n0=8),
    dict(enc="q8g64s.t64", xmode="rms", epi="resadd", M=6, N=128, K=128, bias=True, gate=True),
    dict(enc="q4g32a.t64", xmode="lnmod", epi="resadd", M=6, N=128, K=128, store=True),
    dict(enc="f16", xmode="lnmod", epi="bias", M=7, N=64, K=64, res=True),
    dict(enc="q4g32a.t64", epi="swiglu", M=3, N=256, K=128),
    dict(enc="q8g64s.t64", epi="swiglu", M=3, N=256, K=128, act="gelu", bias=True),
    dict(enc="q4g32a.t64", epi="heads", M=5, N=384, K=128, Hq=1, Hkv=1, rope_mode="half", row_off=3, Ltot=12),
    dict(enc="f16", epi="heads", M=4, N=512, K=64, Hq=2, Hkv=1, rope_mode=None, row_off=1),
    dict(enc="q4g32a.t64", epi="onormgate", M=3, N=256, K=64, n0=0),
    dict(enc="f16", epi="f16", M=4, N=100, K=64, wr0=16),
]


@pytest.mark.parametrize("kw", CASES, ids=lambda k: f"{k['enc']}-{k.get('xmode', 'f16')}-{k['epi']}")
def test_oracle_gemm_against_numpy(kw):
    case = make_case(seed=3, **kw)
    got = case.run_oracle(weights=oracle.KERNEL_WEIGHTS)
    want = epi_numpy(case, acc_numpy(case))
    fp16 = got.dtype == np.uint16
    assert_close(got, want, fp16=fp16, what="oracle vs numpy")
    if fp16:   # same rounding points and float64 sums: almost every value is bit-identical
        assert np.mean(got == want) > 0.995


@pytest.mark.parametrize("enc", ["q4g32a.t64", "q8g64s.t64"])
def test_oracle_cpu_weight_model_is_cpuGemm(enc):
    """CPU_WEIGHTS: y = X W^T over the encoders' fp32 dequantised weights, exactly the test suite's cpuGemm
    (test/kernels.test.js:25-29, float64 sums), rounded once to fp32."""
    M, N, K = 8, 128, 256
    X = oracle.h2f(oracle.f16_bits(oracle.randn(M * K, 7)))
    W0 = oracle.randn(N * K, 11, 0.05)
    wb, deq = (oracle.pack_q4 if enc.startswith("q4") else oracle.pack_q8)(W0, N, K, want_deq=True)
    y = np.zeros(M * N, np.float32)
    oracle.gemm({"w": {"enc": enc, "buf": wb, "rows": N, "cols": K}, "x": {"buf": oracle.f16_bits(X)}, "y": {"buf": y},
                 "M": M, "N": N, "K": K, "epi": "f32"}, weights=oracle.CPU_WEIGHTS)
    assert np.array_equal(y, oracle.cpu_gemm(X, deq, M, N, K))


def test_oracle_plain_gemm_is_cpuGemm():
    """y = X W^T on fp16 data equals the test suite's cpuGemm (float64 sums) after one fp16 rounding."""
    case = make_case(enc="f16", epi="f32", M=32, N=128, K=256, seed=7)
    got = case.run_oracle()
    X = oracle.h2f(case.bufs["x"])
    Wd = oracle.h2f(case.bufs["w"].view(np.uint16))
    ref = oracle.cpu_gemm(X, Wd, 32, 128, 256)
    assert np.array_equal(got, ref)


def test_oracle_conv3_is_textbook_and_chunks_are_identical():
    c = make_conv3_case()
    T, H, W, C, N = c.dims
    whole = c.run_oracle()
    # textbook: replicate-pad time, zero-pad space, 27 taps (numpy einsum, float64)
    X = c.X.reshape(T, H, W, C).astype(np.float64)
    Xp = np.pad(X, ((1, 1), (0, 0), (0, 0), (0, 0)), mode="edge")
    Xp = np.pad(Xp, ((0, 0), (1, 1), (1, 1), (0, 0)))
    Wt = c.Wt.reshape(N, 3, 3, 3, C).astype(np.float64)
    ref = np.zeros((T, H, W, N))
    for kt in range(3):
        for ky in range(3):
            for kx in range(3):
                ref += np.einsum("thwc,nc->thwn", Xp[kt:kt + T, ky:ky + H, kx:kx + W], Wt[:, kt, ky, kx])
    assert_close(whole, ref.ravel().astype(np.float32).astype(np.float16).view(np.uint16), what="conv3 textbook")
    cpu = oracle.cpu_conv3(c.X, c.Wt, T, H, W, C, N)
    cos, _ = cos_maxerr(to_float(whole), cpu)
    assert cos > 0.9995
    # 2-frame chunks (padT = t0, input from frame padL = max(0, t0 - 1)) == whole clip, bit for bit
    fx, fy = H * W * C, H * W * N
    out = np.zeros_like(whole)
    for t0 in range(0, T, 2):
        nf, padL = min(2, T - t0), max(0, t0 - 1)
        spec = dict(c.spec)
        spec["conv"] = dict(c.spec["conv"], padT=t0, padL=padL)
        spec["M"] = nf * H * W
        xb = c.bufs["x"][padL * fx:]
        yb = np.zeros(nf * fy, np.uint16)
        h = {"x": xb.copy(), "w": c.bufs["w"], "y": yb}
        oracle.gemm({**{k: v for k, v in spec.items()}, "x": {"buf": h["x"]}, "w": dict(spec["w"], buf=h["w"]),
                     "y": {"buf": h["y"]}})
        out[t0 * fy:(t0 + nf) * fy] = yb
    assert np.array_equal(out, whole)


def test_oracle_conv2d_against_numpy():
    for kw in (dict(), dict(stride=2), dict(up2=True), dict(gn=True), dict(ks=1, pad=0)):
        c = make_conv2d_case(**kw)
        Hi, Wi, Ci, Ho, Wo, ks, stride, pad, up2 = c.geom
        N = c.spec["N"]
        X = c.X.reshape(Hi, Wi, Ci).astype(np.float32)
        if up2:
            X = X.repeat(2, 0).repeat(2, 1)
        if kw.get("gn"):
            a, b = c.bufs["pv"][:Ci], c.bufs["pv"][Ci:]
            z = X * a + b
            X = f16r(z / (np.float32(1) + np.exp(-z)))
        Xp = np.pad(X.astype(np.float64), ((pad, pad), (pad, pad), (0, 0)))
        Wt = c.Wt.reshape(N, ks, ks, Ci).astype(np.float64)
        ref = np.zeros((Ho, Wo, N))
        for ky in range(ks):
            for kx in range(ks):
                patch = Xp[ky:ky + stride * Ho:stride, kx:kx + stride * Wo:stride]
                ref += np.einsum("hwc,nc->hwn", patch, Wt[:, ky, kx])
        got = c.run_oracle()
        assert_close(got, ref.ravel().astype(np.float32).astype(np.float16).view(np.uint16), what=f"conv2d {kw}")


def test_rope_2d_table_closed_form():
    rp = rope_table_2d(4096, 64).reshape(4096, 64, 2)
    # token (y=3, x=5): pair 0 rotates by y, pair 32 by x, pair k by y * 1e4^(-k/32)
    t = 3 * 64 + 5
    assert np.allclose(rp[t, 0], [math.cos(3), math.sin(3)], atol=1e-6)
    assert np.allclose(rp[t, 32], [math.cos(5), math.sin(5)], atol=1e-6)
    assert np.allclose(rp[t, 7], [math.cos(3 * 1e4 ** (-7 / 32)), math.sin(3 * 1e4 ** (-7 / 32))], atol=1e-6)
    assert np.allclose(np.hypot(rp[..., 0], rp[..., 1]), 1.0, atol=1e-6)


def test_heads_invariants():
    """RoPE is a rotation: per pair, |v| is the same before and after; V heads pass through un-normalised."""
    case = make_case(enc="f16", epi="heads", M=6, N=384, K=64, seed=9, Hq=1, Hkv=1, rope_mode="half")
    got = oracle.h2f(case.run_oracle(weights=oracle.KERNEL_WEIGHTS)).reshape(3, -1, 128).astype(np.float64)
    acc = acc_numpy(case)
    v = got[2, :6]
    assert np.allclose(v, f16r(acc[:, 256:384]), atol=0, rtol=0)
    q = got[0, :6]
    nrm = acc[:, :128] / np.sqrt((acc[:, :128] ** 2).sum(1, keepdims=True) / 128 + 1e-6) * case.bufs["ev"][:128]
    pre = np.hypot(nrm[:, :64], nrm[:, 64:])
    post = np.hypot(q[:, :64], q[:, 64:])
    assert np.allclose(pre, post, rtol=4e-3, atol=4e-3)


def test_oracle_rowstats():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((7, 100)).astype(np.float32)
    st = np.zeros(20, np.float32)
    oracle.rowstats(x, 7, 96, "ln", 1e-6, st, ld=100, c0=4, st_off=2)
    s = st.reshape(-1, 2)[2:9]
    xx = x[:, 4:100].astype(np.float64)
    assert np.allclose(s[:, 0], xx.mean(1), atol=1e-6)
    assert np.allclose(s[:, 1], 1 / np.sqrt(xx.var(1) + 1e-6), rtol=1e-6)
    oracle.rowstats(x, 7, 96, "rms", 1e-6, st, ld=100, c0=4)
    s = st.reshape(-1, 2)[:7]
    assert np.all(s[:, 0] == 0)
    assert np.allclose(s[:, 1], 1 / np.sqrt((xx ** 2).mean(1) + 1e-6), rtol=1e-6)


def test_oracle_args_layout_is_the_header_s():
    """The oracle flattens the reference's argument object by its own code (oracle.oracle_args): its struct has the
    size and the field offsets of p0k_gemm_args as the C oracle was compiled against include/p0k.h"""
    import ctypes as C
    size, offs = oracle.args_layout()
    fields = oracle.OracleArgs._fields_
    assert size == C.sizeof(oracle.OracleArgs) and len(offs) == len(fields)
    for (name, _), off in zip(fields, offs):
        assert getattr(oracle.OracleArgs, name).offset == off, name


def test_oracle_and_product_flatten_alike():
    """The checker's flattening (oracle.oracle_args) and the product's (p0k.gemm_args) are two separate restatements of
    the reference's argument object; over the randomised parity cases, the GLU and short-call sweeps, conv / conv3 and
    heads calls, every byte of the two structs agrees"""
    import p0k
    import test_random_cases as R
    kws = R.CASES + R.GLU_CASES + R.SHORT_CASES + R.NARROW_CASES
    cases = [make_case(**kw) for kw in kws[:120]]
    cases += [make_conv3_case(T=3, H=5, W=7, C=64, N=128, pn=pn) for pn in (False, True)]
    cases += [make_conv2d_case(**kw) for kw in ({}, {"up2": True}, {"gn": True})]
    cases += [make_case(enc="q4g32a.t64", xmode="lnmod", epi="heads", M=40, N=4 * 128, K=256, Hq=2, Hkv=1,
                        rope_mode=m, row_off=3) for m in ("interleaved", "half")]
    for c in cases:
        a = c.args(lambda n: c.bufs[n])
        want = bytes(p0k.gemm_args(a, p0k.numpy_resolve))
        got = bytes(oracle.oracle_args(a))
        assert got == want, c.spec
