"""Pins of the CPU oracle (oracle/p0k_oracle.c) — no GPU.

The reference (JavaScript) ships no binary fixtures for the gemm path; its own known answers are few
(test/convert.test.mjs:44-47, the calibrate / bench scale word src/core/tune.js:43). Each oracle function is therefore
pinned by something that does not restate its own code: an independent numpy formulation written from docs/FORMAT.md
and the WGSL formulas, closed forms, invariants, and IEEE behaviour checked against numpy's float16.
"""
import math

import numpy as np
import pytest

import oracle


# ------------------------------------------------------------------------------------------------ fp16
def test_f16_known_answers():
    # test/convert.test.mjs:47: F16 0x3c00 = 1, 0xc000 = -2
    assert oracle.f2h([1.0, -2.0]).tolist() == [0x3C00, 0xC000]
    assert oracle.h2f(np.array([0x3C00, 0xC000], np.uint16)).tolist() == [1.0, -2.0]


def test_f16_roundtrip_every_code():
    L = oracle.lib()
    codes = np.arange(65536, dtype=np.uint32)
    vals = np.array([L.or_h2f(int(c)) for c in codes], np.float32)
    ref = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(vals[finite], ref[finite])
    back = oracle.f16_bits(vals[finite])
    assert np.array_equal(back, codes[finite].astype(np.uint16))


def test_f16_rne_against_numpy():
    rng = np.random.default_rng(1)
    # random fp32 bit patterns over the whole fp16 range, plus exact ties and the edges
    x = (rng.standard_normal(200000) * np.exp2(rng.integers(-26, 17, 200000))).astype(np.float32)
    ties = (np.arange(-2000, 2000, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10)          # halfway in [-2, 2)
    sub = (np.arange(0, 4000, dtype=np.float32) * np.float32(2.0 ** -26))                    # fp16 subnormal ties
    edge = np.array([65504, 65519.99, 65520, 65536, 1e9, -65520, 2 ** -25, 2 ** -24, 3 * 2 ** -26, np.inf, -np.inf],
                    np.float32)
    for arr in (x, ties, sub, edge):
        with np.errstate(over="ignore"):
            want = arr.astype(np.float16).view(np.uint16)
        assert np.array_equal(oracle.f16_bits(arr), want)
    nan = oracle.f2h([float("nan")])[0]
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x3FF) != 0


# ------------------------------------------------------------------------------------------------ encoders
def _q4_numpy(W, rows, K):
    """FORMAT.md q4g32a.t64, written afresh in numpy float32: quantiser + record layout."""
    W = W.reshape(rows, K).astype(np.float32)
    G = K // 32
    v = W.reshape(rows, G, 32)
    mn = v.min(axis=2).astype(np.float16).astype(np.float32)
    s = ((v.max(axis=2) - mn) / np.float32(15)).astype(np.float32).astype(np.float16).astype(np.float32)
    s = np.where(s == 0, np.float32(1), s)
    q = np.clip(np.rint((v - mn[..., None]) / s[..., None]), 0, 15).astype(np.uint8)   # rint = half to even
    out = np.zeros((rows // 64, G, 1280), np.uint8)
    qq = q.reshape(rows // 64, 64, G, 16, 2)
    codes = (qq[..., 0] | (qq[..., 1] << 4)).astype(np.uint8)                           # [t, r, g, 16]
    out[:, :, :1024] = codes.transpose(0, 2, 1, 3).reshape(rows // 64, G, 1024)
    sm = (s.astype(np.float16).view(np.uint16).astype(np.uint32) |
          (mn.astype(np.float16).view(np.uint16).astype(np.uint32) << 16))
    out[:, :, 1024:] = sm.reshape(rows // 64, 64, G).transpose(0, 2, 1).astype("<u4").copy().view(np.uint8).reshape(rows // 64, G, 256)
    deq = (q.astype(np.float64) * s[..., None] + mn[..., None]).astype(np.float32).reshape(rows, K)
    return out.ravel(), deq, s, mn


def _q8_numpy(W, rows, K):
    W = W.reshape(rows, K).astype(np.float32)
    G = K // 64
    v = W.reshape(rows, G, 64)
    s = (np.abs(v).max(axis=2) / np.float32(127)).astype(np.float32).astype(np.float16).astype(np.float32)
    s = np.where(s == 0, np.float32(1), s)
    q = np.clip(np.rint(v / s[..., None]), -128, 127).astype(np.int8)
    out = np.zeros((rows // 64, G, 4224), np.uint8)
    out[:, :, :4096] = q.view(np.uint8).reshape(rows // 64, 64, G, 64).transpose(0, 2, 1, 3).reshape(rows // 64, G, 4096)
    out[:, :, 4096:] = s.astype(np.float16).reshape(rows // 64, 64, G).transpose(0, 2, 1).copy().view(np.uint8).reshape(rows // 64, G, 128)
    deq = (q.astype(np.float64) * s[..., None]).astype(np.float32).reshape(rows, K)
    return out.ravel(), deq, s


@pytest.mark.parametrize("rows,K,seed,scale", [(64, 32, 1, 0.02), (128, 256, 11, 0.05), (192, 96, 3, 1.0)])
def test_q4_bytes_match_format_md(rows, K, seed, scale):
    W = oracle.randn(rows * K, seed, scale)
    got, deq = oracle.pack_q4(W, rows, K, want_deq=True)
    want, wdeq, s, mn = _q4_numpy(W, rows, K)
    assert got.size == rows * K * 5 // 8                      # 5.0 bits per weight
    assert np.array_equal(got, want)
    assert np.array_equal(deq, wdeq.ravel())
    # quantisation error at most half a step (+ the fp32 rounding of the division)
    err = np.abs(W.reshape(rows, K // 32, 32) - deq.reshape(rows, K // 32, 32))
    assert np.all(err <= s[..., None] * 0.5 * (1 + 1e-5) + 1e-12)


@pytest.mark.parametrize("rows,K,seed,scale", [(64, 64, 2, 0.02), (128, 256, 11, 0.05), (64, 192, 5, 3.0)])
def test_q8_bytes_match_format_md(rows, K, seed, scale):
    W = oracle.randn(rows * K, seed, scale)
    got, deq = oracle.pack_q8(W, rows, K, want_deq=True)
    want, wdeq, s = _q8_numpy(W, rows, K)
    assert got.size == rows * K * 33 // 32                    # 8.25 bits per weight
    assert np.array_equal(got, want)
    assert np.array_equal(deq, wdeq.ravel())
    err = np.abs(W.reshape(rows, K // 64, 64) - deq.reshape(rows, K // 64, 64))
    assert np.all(err <= s[..., None] * 0.5 * (1 + 1e-5) + 1e-12)


def test_q4_known_group_and_bad_shapes():
    # one group holding 0, 0.1, ..., 1.5 (twice): min 0, scale f16(1.5/15) -> code i for value i*0.1
    rows, K = 64, 32
    W = np.zeros((rows, K), np.float32)
    W[5] = np.tile(np.arange(16, dtype=np.float32) * np.float32(0.1), 2)
    b = oracle.pack_q4(W, rows, K)
    rec = b.reshape(-1)
    row5 = rec[5 * 16: 5 * 16 + 16]
    assert row5.tolist() == [(2 * j % 16) | (((2 * j + 1) % 16) << 4) for j in range(16)]
    sm = int(rec[1024 + 5 * 4: 1024 + 5 * 4 + 4].view("<u4")[0])
    assert sm & 0xFFFF == int(np.float16(np.float32(1.5) / np.float32(15)).view(np.uint16))
    assert sm >> 16 == 0
    # all-equal rows: scale 0 -> 1.0 (0x3C00), codes 0, min = the value
    sm0 = int(rec[1024:1028].view("<u4")[0])
    assert sm0 == 0x3C00
    with pytest.raises(ValueError):
        oracle.pack_q4(np.zeros(32 * 32, np.float32), 32, 32)
    with pytest.raises(ValueError):
        oracle.pack_q8(np.zeros(64 * 32, np.float32), 64, 32)


def test_q4_calibrate_known_answer_records():
    # src/core/tune.js:43, bench/bench.js:19: scale word 0x2000 | (0xA800 | j) << 16 -> s = 2^-7, min = -2^-5 (1 + j/1024)
    rng = np.random.default_rng(5)
    rows, K = 128, 64
    u = rng.integers(0, 2 ** 32, size=(rows // 64) * (K // 32) * 320, dtype=np.uint64).astype(np.uint32)
    u = u.reshape(-1, 320)
    for j in range(64):
        u[:, 256 + j] = 0x2000 | ((0xA800 | j) << 16)
    w = u.ravel().view(np.uint8)
    got = oracle.h2f(oracle.dequant("q4g32a.t64", w, rows, K)).astype(np.float64)
    codes = np.zeros((rows, K), np.int64)
    words = u.reshape(rows // 64, K // 32, 320)
    for n in range(rows):
        for k in range(K):
            word = int(words[n // 64, k // 32, (n % 64) * 4 + (k % 32) // 8])
            codes[n, k] = (word >> (4 * (k % 8))) & 15
    j = np.arange(rows) % 64
    want = codes * 2.0 ** -7 - 2.0 ** -5 * (1 + j[:, None] / 1024)
    want16 = want.astype(np.float32).astype(np.float16).astype(np.float64)
    assert np.array_equal(got, want16)


def test_weight_decode_exhaustive_codes():
    """f16(f32(q*s + mn)) for all 16 codes and 256 codes over scales/mins with far-apart exponents."""
    rng = np.random.default_rng(9)
    L = oracle.lib()
    pairs = [(int(rng.integers(0, 0x7C00)), int(rng.integers(0, 0x10000)) & 0xFBFF) for _ in range(60)]
    pairs += [(0x3C00, 0x0000), (0x0001, 0x6000), (0x7BFF, 0x8001), (0x0400, 0xF800), (0x1400, 0x6BFF)]
    for sb, mb in pairs:
        if (mb & 0x7C00) == 0x7C00:
            continue
        rec = np.zeros(1280, np.uint8)
        rec[1024:1028] = np.array([sb | (mb << 16)], "<u4").view(np.uint8)
        s = np.uint16(sb).view(np.float16).astype(np.float32)
        mn = np.uint16(mb).view(np.float16).astype(np.float32)
        for q in range(16):
            rec[0] = q | (q << 4)
            want = np.float16(np.float32(q) * s + mn).view(np.uint16)
            with np.errstate(over="ignore"):
                want = (np.float32(q) * s + mn).astype(np.float16).view(np.uint16)
            assert L.or_weight_f16(1, rec.ctypes.data, 1, 0, 0) == int(want), (hex(sb), hex(mb), q)
    rec8 = np.zeros(4224, np.uint8)
    for sb in [0x3C00, 0x0001, 0x2E66, 0x7BFF, 0x0400, 0x1234]:
        rec8[4096:4098] = np.array([sb], "<u2").view(np.uint8)
        s = np.uint16(sb).view(np.float16).astype(np.float32)
        for q in range(-128, 128):
            rec8[0] = q & 255
            with np.errstate(over="ignore"):
                want = (np.float32(q) * s).astype(np.float16).view(np.uint16)
            assert L.or_weight_f16(2, rec8.ctypes.data, 1, 0, 0) == int(want)


# ------------------------------------------------------------------------------------------------ test data
def test_randn_matches_the_test_suite_generator():
    """test/kernels.test.js:12-13, re-implemented here in pure Python with JS integer semantics."""
    def js_rng(seed):
        s = (seed & 0xFFFFFFFF) or 1

        def i32(v):
            v &= 0xFFFFFFFF
            return v - (1 << 32) if v & 0x80000000 else v

        def nxt():
            nonlocal s
            s = (s ^ i32(s << 13)) & 0xFFFFFFFF
            s = (s ^ (i32(s) >> 17)) & 0xFFFFFFFF
            s = (s ^ i32(s << 5)) & 0xFFFFFFFF
            return s / 4294967296
        return nxt

    for seed, scale in [(7, 1.0), (11, 0.05), (33, 0.03)]:
        r = js_rng(seed)
        want = []
        for i in range(0, 64, 2):
            u, v = max(1e-9, r()), r()
            m = math.sqrt(-2 * math.log(u)) * scale
            want += [m * math.cos(2 * math.pi * v), m * math.sin(2 * math.pi * v)]
        got = oracle.randn(64, seed, scale)
        assert np.array_equal(got, np.array(want, np.float32))
    big = oracle.randn(200000, 123, 0.5)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 0.5) < 0.01
