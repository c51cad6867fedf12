"""Seeded GEMM cases shared by the oracle tests, the GPU parity tests, smoke() and bench.py.

A Case holds host numpy buffers (weights encoded per FORMAT.md, activations, output, vectors) and builds the
reference-style argument dict (types/index.d.ts:128-150) over any buffer objects: numpy arrays for the CPU oracle,
device Buffers for libp0k. Inputs follow BASELINE.json's recipes: weights N(0, scale) quantised with the reference
encoders, activations fp16 N(0, 1) (or U[-1, 1]), fp32 residuals holding fp16-representable values.
"""
import math

import numpy as np

import oracle


def rope_table_2d(L, grid_w, theta=10000.0):
    """2-D RoPE table RP[row][64][cos, sin] for a grid of tokens (row = y * grid_w + x): pairs 0..31 rotate by the
    row index y, pairs 32..63 by the column index x, with frequencies theta^(-k/32), k = 0..31. The reference has no
    table builder (its callers pass RP); this one is the build's own, pinned by its closed form in the tests."""
    tok = np.arange(L)
    y, x = tok // grid_w, tok % grid_w
    k = np.arange(32)
    inv = theta ** (-k / 32.0)
    ang = np.concatenate([y[:, None] * inv[None, :], x[:, None] * inv[None, :]], axis=1)   # [L, 64]
    rp = np.empty((L, 64, 2), np.float32)
    rp[..., 0] = np.cos(ang)
    rp[..., 1] = np.sin(ang)
    return rp.ravel()


def rope_table_1d(L, theta=10000.0):
    k = np.arange(64)
    inv = theta ** (-k / 64.0)
    ang = np.arange(L)[:, None] * inv[None, :]
    rp = np.empty((L, 64, 2), np.float32)
    rp[..., 0] = np.cos(ang)
    rp[..., 1] = np.sin(ang)
    return rp.ravel()


def f16_values(n, seed, scale=1.0):
    return oracle.h2f(oracle.f16_bits(oracle.randn(n, seed, scale)))


def encode_weights(enc, W, rows, K):
    if enc == "q4g32a.t64":
        return oracle.pack_q4(W, rows, K)
    if enc == "q8g64s.t64":
        return oracle.pack_q8(W, rows, K)
    return oracle.f16_bits(W).view(np.uint8).copy()


class Case:
    """One gemm call. `bufs` maps a name to a host numpy array; `spec` is the argument dict with names in place of
    buffers; args(resolve) swaps the names for buffer objects."""

    def __init__(self, spec, bufs, out="y"):
        self.spec, self.bufs, self.out = spec, bufs, out
        self.kernel = None

    def args(self, lookup):
        def sub(v):
            if isinstance(v, dict):
                return {k: (lookup(x) if k == "buf" else sub(x)) for k, x in v.items()}
            return v
        return {k: sub(v) for k, v in self.spec.items()}

    def host_copy(self):
        return {k: v.copy() for k, v in self.bufs.items()}

    def run_oracle(self, m0=0, m1=None, weights=None):
        """weights: the oracle's weight model; by default the one the HIP kernel for this call computes with (the
        decode GEMV sums over fp32 dequantised weights like the reference's cpuGemm, the MFMA GEMM over fp16 ones
        like the reference's kernel)."""
        h = self.host_copy()
        a = self.args(lambda n: h[n])
        if weights is None:
            import p0k
            # the kernel the last run_device call planned on its device (its CU count); without one, the
            # context-free plan for a 256-CU device
            kern = self.kernel or p0k.select_tile(a)["kernel"]
            weights = oracle.CPU_WEIGHTS if kern.startswith("gemv") else oracle.KERNEL_WEIGHTS
        oracle.gemm(a, m0, m1, weights)
        return h[self.out]

    def run_device(self, dev, upload=None):
        """upload every buffer, run, read the output back (bytes -> dtype of the host array)."""
        d = {k: dev.upload(v) for k, v in self.bufs.items()}
        try:
            self.kernel = dev.select_tile(self.args(lambda n: d[n]))["kernel"]
            dev.gemm(self.args(lambda n: d[n]))
            out = self.bufs[self.out]
            return dev.read(d[self.out], out.dtype, out.size)
        finally:
            for b in d.values():
                dev.free(b)


def make_case(enc="f16", xmode="f16", epi="f16", M=32, N=128, K=256, seed=1, wscale=0.05, *, act="silu", bias=False,
              gate=False, store=False, res=False, rope_mode=None, Hq=None, Hkv=None, Ltot=None, row_off=0,
              ld_pad=0, k0=0, n0=0, wk0=0, wr0=0, x_uniform=False, tile=None, eps=1e-6, acc=None, rope_grid_w=None):
    """A seeded case of any (encoding, prologue, epilogue). Shapes: ws columns N; for swiglu the weight holds
    [gate N/2 | up N/2] rows (wr0 = 0, wr1 = N/2); for heads N = (Hq + 2 Hkv) * 128, with a 1-D RoPE table, or the
    2-D table of a token grid rope_grid_w wide."""
    bufs, spec = {}, {}
    glu = epi == "swiglu"
    Kt = K + wk0
    rows = N if not glu else N
    rows_alloc = max(64, (rows + wr0 + 63) // 64 * 64) if enc != "f16" else rows + wr0
    W = oracle.randn(rows_alloc * Kt, seed * 7 + 1, wscale)
    bufs["w"] = encode_weights(enc, W, rows_alloc, Kt)
    spec["w"] = {"enc": enc, "buf": "w", "off": 0, "bytes": bufs["w"].nbytes, "rows": rows_alloc, "cols": Kt}
    if glu:
        spec["wr0"], spec["wr1"] = wr0, wr0 + N // 2
    else:
        spec["wr0"] = wr0
    spec["wk0"] = wk0
    ldx = K + k0 + ld_pad
    if xmode == "f16":
        if x_uniform:
            xv = oracle.h2f(oracle.f16_bits(oracle.rand_uniform(M * ldx, seed * 7 + 2, -1.0, 1.0)))
        else:
            xv = f16_values(M * ldx, seed * 7 + 2)
        bufs["x"] = oracle.f16_bits(xv)
    else:
        xv = f16_values(M * ldx, seed * 7 + 2)          # fp32 residual holding fp16 values
        bufs["x"] = xv.astype(np.float32)
        st = np.zeros(M * 2, np.float32)
        oracle.rowstats(bufs["x"], M, K, "rms" if xmode == "rms" else "ln", eps, st, ld=ldx, c0=k0)
        bufs["st"] = st
        spec["stats"] = {"buf": "st", "off": 0}
        if xmode == "rms":
            bufs["pv"] = (1.0 + oracle.randn(ldx, seed * 7 + 3, 0.1)).astype(np.float32)
            spec["pv"] = {"buf": "pv", "off": 0, "stride": 0}
        else:
            bufs["pv"] = oracle.randn(2 * ldx, seed * 7 + 3, 0.5).astype(np.float32)
            spec["pv"] = {"buf": "pv", "off": 0, "stride": ldx}
    spec["x"] = {"buf": "x", "ld": ldx, "k0": k0, "mode": xmode}
    spec.update({"M": M, "N": N, "K": K, "epi": epi})
    if acc:
        spec["acc"] = acc
    if tile:
        spec["tile"] = tile
    ny = N // 2 if glu else N
    ldy = ny + n0 + ld_pad
    if epi in ("f32", "resadd"):
        y = f16_values(M * ldy, seed * 7 + 4) if epi == "resadd" else np.zeros(M * ldy, np.float32)
        bufs["y"] = y.astype(np.float32)
    elif epi == "heads":
        Hq, Hkv = Hq or 1, Hkv if Hkv is not None else 1
        assert N == (Hq + 2 * Hkv) * 128
        Ltot = Ltot or (row_off + M)
        bufs["y"] = np.zeros((Hq + 2 * Hkv) * Ltot * 128, np.uint16)
        bufs["rope"] = rope_table_2d(Ltot, rope_grid_w) if rope_grid_w else rope_table_1d(Ltot)
        bufs["ev"] = (1.0 + oracle.randn(256, seed * 7 + 5, 0.1)).astype(np.float32)
        spec["ev"] = {"buf": "ev", "off": 0}
        spec["heads"] = {"Ltot": Ltot, "Hq": Hq, "Hkv": Hkv, "rowOff": row_off, "eps": eps,
                         "ropeMode": rope_mode or "interleaved", "rope": {"buf": "rope"}}
    else:
        y0 = oracle.f16_bits(f16_values(M * ldy, seed * 7 + 4)) if (epi == "bias" and res) else np.zeros(M * ldy, np.uint16)
        bufs["y"] = y0
    spec["y"] = {"buf": "y", "ld": ldy, "n0": n0} if epi != "heads" else {"buf": "y"}
    if epi == "bias":
        bufs["ev"] = oracle.randn(N + 8, seed * 7 + 6, 0.5).astype(np.float32)
        spec["ev"] = {"buf": "ev", "off": 3}
        spec["res"] = res
    if epi == "resadd":
        if gate:
            bufs["ev"] = oracle.randn(N + 4, seed * 7 + 6, 1.0).astype(np.float32)
            spec["ev"] = {"buf": "ev", "off": 4}
        if bias:
            bufs["bv"] = oracle.randn(N + 2, seed * 7 + 7, 0.5).astype(np.float32)
            spec["bv"] = {"buf": "bv", "off": 2}
        spec["store"] = store
    if glu:
        spec["act"] = act
        if bias:
            bufs["bv"] = oracle.randn(N + 16, seed * 7 + 7, 0.5).astype(np.float32)
            spec["bv"] = {"buf": "bv", "off": 1, "up": N // 2 + 5}
    if epi == "onormgate":
        Lg = N + n0
        bufs["gt"] = oracle.f16_bits(f16_values(M * Lg, seed * 7 + 8))
        spec["gt"] = {"buf": "gt"}
        bufs["ev"] = (1.0 + oracle.randn(128, seed * 7 + 5, 0.1)).astype(np.float32)
        spec["ev"] = {"buf": "ev", "off": 0}
        spec["heads"] = {"Ltot": Lg, "Hq": 0, "Hkv": 0, "eps": eps}
    return Case(spec, bufs)


def make_conv3_case(T=5, H=6, W=6, C=32, N=128, seed=31, pn=False, enc="f16", wscale=0.03):
    """The reference's 3x3x3 convolution case (test/kernels.test.js:95-105) over a THWC clip, whole-clip call."""
    K = 27 * C
    X = f16_values(T * H * W * C, seed)
    Wt = oracle.h2f(oracle.f16_bits(oracle.randn(N * K, seed + 2, wscale)))
    bufs = {"x": oracle.f16_bits(X), "w": encode_weights(enc, Wt, N, K), "y": np.zeros(T * H * W * N, np.uint16)}
    conv = {"kind": "conv3", "Hi": H, "Wi": W, "Ci": C, "Ho": H, "Wo": W, "stride": T, "padT": 0, "padL": 0, "ks": 1}
    spec = {"w": {"enc": enc, "buf": "w", "off": 0, "bytes": bufs["w"].nbytes, "rows": N, "cols": K},
            "x": {"buf": "x"}, "y": {"buf": "y"}, "M": T * H * W, "N": N, "K": K, "conv": conv}
    if pn:
        bufs["st"] = (0.5 + np.abs(oracle.randn(T * H * W, seed + 5, 1.0))).astype(np.float32)
        spec["stats"] = {"buf": "st"}
        conv["pn"] = True
    c = Case(spec, bufs)
    c.X, c.Wt, c.dims = X, Wt, (T, H, W, C, N)
    return c


def make_conv2d_case(Hi=7, Wi=9, Ci=32, N=64, ks=3, stride=1, pad=1, up2=False, gn=False, seed=51, enc="f16"):
    """2-D implicit-GEMM convolution over an HWC image (gemm.js:81-91): OHWI weights, K = ks*ks*Ci."""
    HH, WW = (2 * Hi, 2 * Wi) if up2 else (Hi, Wi)
    Ho = (HH + 2 * pad - ks) // stride + 1
    Wo = (WW + 2 * pad - ks) // stride + 1
    K = ks * ks * Ci
    X = f16_values(Hi * Wi * Ci, seed)
    Wt = oracle.h2f(oracle.f16_bits(oracle.randn(N * K, seed + 2, 0.05)))
    rows = max(64, (N + 63) // 64 * 64) if enc != "f16" else N
    Wfull = np.zeros(rows * K, np.float32)
    Wfull[: N * K] = Wt
    bufs = {"x": oracle.f16_bits(X), "w": encode_weights(enc, Wfull, rows, K), "y": np.zeros(Ho * Wo * N, np.uint16)}
    conv = {"kind": "conv", "Hi": Hi, "Wi": Wi, "Ci": Ci, "Ho": Ho, "Wo": Wo, "stride": stride, "padT": pad,
            "padL": pad, "ks": ks, "up2": up2, "gn": gn}
    spec = {"w": {"enc": enc, "buf": "w", "off": 0, "bytes": bufs["w"].nbytes, "rows": rows, "cols": K},
            "x": {"buf": "x"}, "y": {"buf": "y"}, "M": Ho * Wo, "N": N, "K": K, "conv": conv}
    if gn:
        bufs["pv"] = np.concatenate([1.0 + oracle.randn(Ci, seed + 4, 0.2), oracle.randn(Ci, seed + 5, 0.3)]).astype(np.float32)
        spec["pv"] = {"buf": "pv", "off": 0, "stride": Ci}
    c = Case(spec, bufs)
    c.X, c.Wt, c.geom = X, Wt, (Hi, Wi, Ci, Ho, Wo, ks, stride, pad, up2)
    return c


# ------------------------------------------------------------------------------------------------ comparisons
def to_float(arr):
    return oracle.h2f(arr) if arr.dtype == np.uint16 else arr.astype(np.float32)


def cos_maxerr(got, want):
    """the reference's compare() (test/kernels.test.js:16-21): cosine similarity and max abs error."""
    g, w = got.astype(np.float64), want.astype(np.float64)
    cos = float(np.dot(g, w) / math.sqrt(max(1e-30, np.dot(g, g) * np.dot(w, w))))
    return cos, float(np.max(np.abs(g - w))) if g.size else 0.0


# Tolerance of a kernel result against the oracle. The oracle rounds at the same points as the kernel (X' to fp16,
# W' to fp16, the epilogue result once) but sums in float64; the kernel sums in fp32 (MFMA / v_dot2) in another
# order, may fuse fp32 operations of the prologue, and uses hardware exp / tanh / rsqrt. For an fp16 result that
# allows one fp16 rounding step of the result plus a small absolute term scaled to the result's spread:
#     |got - want| <= 2^-9 * |want| + 2^-12 * rms(want)
# For fp32 results (f32, resadd):  |got - want| <= 2^-16 * |want| + 2^-14 * rms(want)
def assert_close(got, want, fp16=True, what=""):
    g, w = to_float(got).astype(np.float64), to_float(want).astype(np.float64)
    assert g.shape == w.shape, (g.shape, w.shape)
    fin = np.isfinite(w)
    assert np.array_equal(np.isfinite(g), fin), f"{what}: non-finite values differ"
    g, w = g[fin], w[fin]
    rms = float(np.sqrt(np.mean(w * w))) if w.size else 0.0
    if fp16:
        tol = 2.0 ** -9 * np.abs(w) + 2.0 ** -12 * rms
    else:
        tol = 2.0 ** -16 * np.abs(w) + 2.0 ** -14 * rms
    err = np.abs(g - w)
    bad = np.nonzero(err > tol)[0]
    assert bad.size == 0, (f"{what}: {bad.size} of {w.size} values outside tolerance; first at {bad[:5]}: got "
                           f"{g[bad[:5]]} want {w[bad[:5]]}; max err {err.max():.3g}, rms {rms:.3g}")
    return float(err.max()) if err.size else 0.0
