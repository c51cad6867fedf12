"""Randomised parity sweep of the gemm path on the GPU: a fixed list of cases drawn from a seeded generator over every
weight encoding, prologue, epilogue and the offsets of the argument objects (x.ld / x.k0, y.ld / y.n0, wk0, wr0),
with M from 1 to a few hundred rows so that every kernel (the one-row GEMV, the matrix-core decode with and without
its K split, the load-to-LDS MFMA GEMM with its tiles and tail launch, the register-staged MFMA GEMM) gets calls of
odd shapes. Each case is checked against the oracle with the weight model of the kernel that runs it (assert_close's
fp16 / fp32 tolerance). The list is generated here, not stored: the same seed gives the same cases.
"""
import numpy as np
import pytest

import p0k
from cases import assert_close, make_case

pytestmark = pytest.mark.gpu

M_CHOICES = [1, 2, 3, 5, 8, 13, 16, 17, 33, 64, 100, 129, 200, 257, 300]


def _cases(n=96, seed=20251202):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        enc = ["q4g32a.t64", "q8g64s.t64", "f16"][rng.integers(3)]
        xmode = ["f16", "f16", "rms", "lnmod"][rng.integers(4)]
        epi = ["f16", "f32", "resadd", "bias", "swiglu", "onormgate", "heads"][rng.integers(7)]
        M = int(M_CHOICES[rng.integers(len(M_CHOICES))])
        kq = 64 if enc == "q8g64s.t64" else 32
        # (half of them whole multiples of 256: the decode kernels split K into 4 or 8 parts of whole units)
        K = int(kq * rng.integers(1, 1024 // kq + 1)) if rng.integers(2) else int(256 * rng.integers(1, 5))
        kw = dict(enc=enc, xmode=xmode, epi=epi, M=M, K=K, seed=int(rng.integers(1, 1 << 20)))
        if epi == "heads":
            Hq, Hkv = int(rng.integers(1, 3)), int(rng.integers(1, 2))
            kw.update(N=(Hq + 2 * Hkv) * 128, Hq=Hq, Hkv=Hkv, rope_mode=["interleaved", "half"][rng.integers(2)],
                      row_off=int(rng.integers(0, 5)))
        elif epi == "onormgate":
            kw.update(N=128 * int(rng.integers(1, 4)))
        elif epi == "swiglu":
            kw.update(N=16 * int(rng.integers(1, 48)), act=["silu", "gelu"][rng.integers(2)], bias=bool(rng.integers(2)))
        else:
            kw.update(N=8 * int(rng.integers(1, 96)))
        if epi == "resadd":
            kw.update(gate=bool(rng.integers(2)), bias=bool(rng.integers(2)), store=bool(rng.integers(2)))
        if epi == "bias":
            kw.update(res=bool(rng.integers(2)))
        # offsets: x rows / column (multiples of 4, as the reference's vec4 rows require), output column, weight
        # column (whole groups) and first weight row (whole records)
        if rng.integers(2):
            kw.update(ld_pad=int(4 * rng.integers(0, 5)), k0=int(4 * rng.integers(0, 9)))
        if epi not in ("heads", "onormgate") and rng.integers(2):
            kw.update(n0=int(8 * rng.integers(0, 3)))
        if rng.integers(3) == 0:
            kw.update(wk0=kq * int(rng.integers(1, 3)))
        if epi not in ("swiglu",) and rng.integers(4) == 0:
            kw.update(wr0=64)
        out.append(kw)
    return out


CASES = _cases()


@pytest.mark.parametrize("kw", CASES, ids=[f"{i:02d}-{k['enc'][:2]}-{k['xmode']}-{k['epi']}-M{k['M']}-N{k['N']}-K{k['K']}"
                                           for i, k in enumerate(CASES)])
def test_random_case_matches_oracle(dev, kw):
    c = make_case(**kw)
    kern = dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"]
    print(f"[p0k-test] random case {kw} kernel={kern}", flush=True)
    got = c.run_device(dev)
    want = c.run_oracle()
    assert_close(got, want, fp16=got.dtype == np.uint16, what=f"{kw} on {kern}")


def _glu_cases(n=40, seed=20251203):
    """decode-sized SwiGLU / GeGLU calls with the gate and up row blocks at arbitrary first rows (wr0, and wr1 = wr0 +
    N / 2 with N / 2 any multiple of 8): the decode kernels give each half of a 128-column item the gate rows and the up
    rows of its ws columns, which then start anywhere inside a 64-row record"""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        enc = ["q4g32a.t64", "q4g32a.t64", "q8g64s.t64", "f16"][rng.integers(4)]
        M = int([1, 1, 2, 3, 4, 4, 5, 8, 11, 16][rng.integers(10)])
        K = int(256 * rng.integers(1, 5)) if enc != "q8g64s.t64" else int(512 * rng.integers(1, 3))
        out.append(dict(enc=enc, xmode=["f16", "f16", "rms"][rng.integers(3)], epi="swiglu", M=M, K=K,
                        N=16 * int(rng.integers(1, 40)), wr0=int([0, 1, 5, 63, 64, 100][rng.integers(6)]),
                        act=["silu", "gelu"][rng.integers(2)], bias=bool(rng.integers(2)),
                        seed=int(rng.integers(1, 1 << 20))))
    return out


GLU_CASES = _glu_cases()


@pytest.mark.parametrize("kw", GLU_CASES, ids=[f"{i:02d}-{k['enc'][:2]}-M{k['M']}-N{k['N']}-K{k['K']}-wr0{k['wr0']}"
                                               for i, k in enumerate(GLU_CASES)])
def test_random_glu_case_matches_oracle(dev, kw):
    c = make_case(**kw)
    kern = dev.select_tile(c.args(lambda n: c.bufs[n]))["kernel"]
    print(f"[p0k-test] random GLU case {kw} kernel={kern}", flush=True)
    got = c.run_device(dev)
    want = c.run_oracle()
    assert_close(got, want, fp16=got.dtype == np.uint16, what=f"{kw} on {kern}")


def _narrow_cases(n=16, seed=20251204):
    """decode calls wide enough for 64-column items without a K split (at least 14336 ws columns: the 128-column
    tiles would fill only half of the CUs), every weight encoding and 1..16 rows, with the argument offsets of the
    sweep above (x.ld / x.k0, y.n0, wk0, wr0) and ragged N"""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        enc = ["q4g32a.t64", "q8g64s.t64", "f16"][rng.integers(3)]
        M = int([1, 2, 3, 4, 5, 8, 13, 16][rng.integers(8)])
        if enc == "q4g32a.t64" and M <= 4:
            M = 5 + int(rng.integers(0, 12))       # (1..4 q4 rows: the stream kernel, covered elsewhere)
        epi = ["f16", "f32", "resadd", "bias", "swiglu"][rng.integers(5)]
        K = int(512 * rng.integers(1, 5))
        kw = dict(enc=enc, xmode=["f16", "f16", "rms"][rng.integers(3)], epi=epi, M=M, K=K,
                  N=14336 + 8 * int(rng.integers(0, 200)), seed=int(rng.integers(1, 1 << 20)))
        if epi == "swiglu":
            kw.update(act=["silu", "gelu"][rng.integers(2)], bias=bool(rng.integers(2)))
        if epi == "resadd":
            kw.update(gate=bool(rng.integers(2)), bias=bool(rng.integers(2)), store=bool(rng.integers(2)))
        if epi == "bias":
            kw.update(res=bool(rng.integers(2)))
        if rng.integers(2):
            kw.update(ld_pad=int(4 * rng.integers(0, 5)), k0=int(4 * rng.integers(0, 9)))
        if rng.integers(2):
            kw.update(n0=int(8 * rng.integers(0, 3)))
        if rng.integers(3) == 0:
            kw.update(wk0=(64 if enc == "q8g64s.t64" else 32) * int(rng.integers(1, 3)))
        if epi != "swiglu" and rng.integers(4) == 0:
            kw.update(wr0=64)
        out.append(kw)
    return out


NARROW_CASES = _narrow_cases()


@pytest.mark.parametrize("kw", NARROW_CASES, ids=[f"{i:02d}-{k['enc'][:2]}-{k['epi']}-M{k['M']}-N{k['N']}-K{k['K']}"
                                                  for i, k in enumerate(NARROW_CASES)])
def test_random_narrow_case_matches_oracle(dev, kw, monkeypatch):
    monkeypatch.setenv("P0K_GEMV_SN", "0")                  # (short q8 calls would take the 16-row items)
    c = make_case(**kw)
    t = dev.select_tile(c.args(lambda n: c.bufs[n]))
    assert t["kernel"] == "gemv_mfma" and t["BN"] == 64, t
    print(f"[p0k-test] random narrow case {kw}", flush=True)
    got = c.run_device(dev)
    want = c.run_oracle()
    assert_close(got, want, fp16=got.dtype == np.uint16, what=f"{kw} on 64-column items")


def _short_cases(n=48, seed=20251205):
    """short-call decode items (16 weight rows, every load in flight; P0K_GEMV_SN=1 forces them) over q4 / q8 / f16 with
    1..4 rows, K up to each encoding's longest (q4 16384, q8 / f16 8192 within 64 KB of X'), ragged N, every
    element-wise epilogue, the rms / lnmod prologues and the argument offsets"""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        enc = ["q4g32a.t64", "q8g64s.t64", "f16"][rng.integers(3)]
        M = int(rng.integers(1, 5))
        kq = 32 if enc == "q4g32a.t64" else 64
        kmax = 16384 if enc == "q4g32a.t64" else 8192
        per_k = {32: 2.25, 64: 2.125}[kq] if enc != "f16" else 2.0                        # X' and its unit sums
        kmax = min(kmax, int(64 * 1024 / ((M if M <= 2 else 4) * per_k)) // kq * kq)        # within 64 KB of LDS
        K = int(kq * rng.integers(1, kmax // kq + 1))
        epi = ["f16", "f32", "resadd", "bias", "swiglu"][rng.integers(5)]
        kw = dict(enc=enc, xmode=["f16", "f16", "rms", "lnmod"][rng.integers(4)], epi=epi, M=M, K=K,
                  N=(16 if epi == "swiglu" else 8) * int(rng.integers(1, 160)), seed=int(rng.integers(1, 1 << 20)))
        if epi == "swiglu":
            kw.update(act=["silu", "gelu"][rng.integers(2)], bias=bool(rng.integers(2)))
        if epi == "resadd":
            kw.update(gate=bool(rng.integers(2)), bias=bool(rng.integers(2)), store=bool(rng.integers(2)))
        if epi == "bias":
            kw.update(res=bool(rng.integers(2)))
        if rng.integers(2):
            kw.update(ld_pad=int(4 * rng.integers(0, 5)), k0=int(4 * rng.integers(0, 9)))
        if epi != "swiglu" and rng.integers(2):
            kw.update(n0=int(8 * rng.integers(0, 3)))
        if rng.integers(3) == 0:
            kw.update(wk0=(8 if enc == "f16" else kq) * int(rng.integers(1, 3)))
        if rng.integers(4) == 0:
            kw.update(wr0=int([1, 16, 64, 100][rng.integers(4)]) if enc == "f16" else 64)
        out.append(kw)
    return out


SHORT_CASES = _short_cases()


@pytest.mark.parametrize("kw", SHORT_CASES, ids=[f"{i:02d}-{k['enc'][:2]}-{k['xmode']}-{k['epi']}-M{k['M']}-N{k['N']}-K{k['K']}"
                                                 for i, k in enumerate(SHORT_CASES)])
def test_random_short_case_matches_oracle(dev, kw, monkeypatch):
    monkeypatch.setenv("P0K_GEMV_SN", "1")
    c = make_case(**kw)
    t = dev.select_tile(c.args(lambda n: c.bufs[n]))
    assert t["kernel"] == "gemv_short", t
    print(f"[p0k-test] random short case {kw}", flush=True)
    got = c.run_device(dev)
    want = c.run_oracle()
    assert_close(got, want, fp16=got.dtype == np.uint16, what=f"{kw} on 16-row items")
