"""Known answers of the fused epilogues (src/ops/gemm.js:204-253), on the oracle (CPU) and on the GPU.

The reference ships no vectors for these epilogues, so each test builds an input whose answer is fixed by the
formula's structure rather than by retyping it, chosen so that a swapped convention fails:

* GLU (`swiglu`, types/index.d.ts:137: wr0 = first gate row, wr1 = first up row): all-zero gate rows give 0
  (act(0) = 0 for SiLU and tanh-GELU); all-zero up rows with a non-zero gate bias and a zero up bias give 0, while the
  same call with wr0 / wr1 swapped does not. Exactly 0 on the oracle and the MFMA GEMM. The matrix-core decode GEMV
  (3..16 rows) never forms the dequantised weight: it sums x against the biased codes (1024 + q) and subtracts
  1024 * sum(x) afterwards, so a zero weight leaves a cancellation residue of order 2^-24 * 1024 * sum|x|; there the
  bar is 2^-8 of the rms of the swapped call's output (measured residue: about 2^-10 of it at K = 256), 256 times
  below what a swapped convention gives.
* RoPE (`heads`): a table of (cos, sin) = (0, 1) rotates each interleaved pair (a, b) to (-b, a), and in 'half' mode
  (v_d, v_{d+64}) to (-v_{d+64}, v_d), bit for bit against the same call with the identity table (1, 0).
* Q / K norm weights: ev[0:128] scales the normalised Q heads and ev[128:256] the K heads; with 2 and 4 (powers of
  two, so the scaling is exact through the rotation and the fp16 store) Q is exactly twice and K exactly four times
  the all-ones result, and V is unchanged.
"""
import numpy as np
import pytest

import oracle
from cases import make_case


def _cpu(case):
    return case.run_oracle()


RUNNERS = ["oracle", pytest.param("gpu", marks=pytest.mark.gpu)]


@pytest.fixture
def run(request):
    if request.param == "oracle":
        return _cpu
    d = request.getfixturevalue("dev")

    def _gpu(case):
        return case.run_device(d)
    return _gpu


def _reencode(case, W):
    s = case.spec["w"]
    case.bufs["w"] = oracle.pack_q4(W.ravel(), s["rows"], s["cols"]) if s["enc"].startswith("q4") else (
        oracle.pack_q8(W.ravel(), s["rows"], s["cols"]) if s["enc"].startswith("q8") else
        oracle.f16_bits(W.ravel()).view(np.uint8).copy())
    s["bytes"] = case.bufs["w"].nbytes


@pytest.mark.parametrize("run", RUNNERS, indirect=True)
@pytest.mark.parametrize("M", [1, 4, 70])
@pytest.mark.parametrize("act", ["silu", "gelu"])
@pytest.mark.parametrize("enc", ["q4g32a.t64", "f16"])
def test_glu_zero_halves(run, M, act, enc):
    N, K = 256, 256                       # ws columns: gate rows 0..127, up rows 128..255
    c = make_case(enc=enc, epi="swiglu", act=act, M=M, N=N, K=K, seed=91)
    rows, Kt = c.spec["w"]["rows"], c.spec["w"]["cols"]
    W = oracle.randn(rows * Kt, 92, 0.05).reshape(rows, Kt)
    # zero up rows, gate bias non-zero, up bias zero; first with wr0 / wr1 swapped (gate read from the zero rows, up
    # from the others), which is not zero and sets the scale
    c2 = make_case(enc=enc, epi="swiglu", act=act, M=M, N=N, K=K, seed=91, bias=True)
    Wu = W.copy()
    Wu[N // 2: N] = 0.0
    _reencode(c2, Wu)
    sp = c2.spec["bv"]
    bv = c2.bufs["bv"]
    bv[sp["off"] + sp["up"]: sp["off"] + sp["up"] + N // 2] = 0.0
    assert np.any(bv[sp["off"]: sp["off"] + N // 2] != 0)
    c2.spec["wr0"], c2.spec["wr1"] = N // 2, 0
    swapped = oracle.h2f(run(c2)).astype(np.float64)
    rms = float(np.sqrt(np.mean(swapped ** 2)))
    assert rms > 1e-3
    exact = run.__name__ == "_cpu" or M > 16
    bar = 0.0 if exact else 2.0 ** -8 * rms

    def is_zero(out, what):
        v = np.abs(oracle.h2f(out).astype(np.float64))
        assert v.max() <= bar, f"{what}: max |y| {v.max():.3g} (bar {bar:.3g})"

    c2.spec["wr0"], c2.spec["wr1"] = 0, N // 2
    is_zero(run(c2), "zero up rows (zero up bias) must give 0 whatever the gate bias")
    Wg = W.copy()
    Wg[: N // 2] = 0.0                    # gate rows zero
    _reencode(c, Wg)
    is_zero(run(c), "zero gate rows must give 0")


def _heads_case(mode, M=70, table=(1.0, 0.0), ev=(1.0, 1.0)):
    c = make_case(enc="f16", epi="heads", M=M, N=3 * 128, K=256, Hq=1, Hkv=1, Ltot=M, rope_mode=mode, seed=93)
    rp = c.bufs["rope"].reshape(M, 64, 2)
    rp[..., 0], rp[..., 1] = table
    evb = c.bufs["ev"]
    evb[:128], evb[128:256] = ev
    return c


@pytest.mark.parametrize("run", RUNNERS, indirect=True)
@pytest.mark.parametrize("mode", ["interleaved", "half"])
def test_rope_quarter_turn(run, mode):
    M = 70
    ident = run(_heads_case(mode)).reshape(3, M, 128)
    rot = run(_heads_case(mode, table=(0.0, 1.0))).reshape(3, M, 128)
    neg = lambda a: a ^ np.uint16(0x8000)          # noqa: E731  fp16 negation
    want = ident.copy()
    for h in (0, 1):                                # Q and K rotate; V passes through
        a = ident[h]
        if mode == "interleaved":
            want[h][:, 0::2], want[h][:, 1::2] = neg(a[:, 1::2]), a[:, 0::2]
        else:
            want[h][:, :64], want[h][:, 64:] = neg(a[:, 64:]), a[:, :64]
    # +0 and -0 are the same value
    same = (rot == want) | (((rot | want) & 0x7FFF) == 0)
    assert np.all(same), f"{mode}: {np.count_nonzero(~same)} values differ from the quarter-turn"
    assert np.array_equal(rot[2], ident[2])


@pytest.mark.parametrize("run", RUNNERS, indirect=True)
def test_qk_norm_weight_sections(run):
    M = 70
    one = oracle.h2f(run(_heads_case("interleaved"))).reshape(3, M, 128)
    sc = oracle.h2f(run(_heads_case("interleaved", ev=(2.0, 4.0)))).reshape(3, M, 128)
    assert np.array_equal(sc[0], 2 * one[0]), "ev[0:128] must scale the Q heads"
    assert np.array_equal(sc[1], 4 * one[1]), "ev[128:256] must scale the K heads"
    assert np.array_equal(sc[2], one[2]), "V is written raw"
