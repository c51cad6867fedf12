"""The Node N-API addon and JavaScript shim (p0pc0rn-kernels_amd/node/index.mjs) that keep the reference's JavaScript
API: createGpu / upload / read / free (src/core/gpu.js), gemm(gpu, args) (src/ops/gemm.js:268), loadWeights
(src/weights.js:10), f2h / h2f (src/core/gpu.js:276-299), packQ4 / packQ8 / packF16 (src/convert/encode.js:56-98).

The host tests need no GPU; the gpu tests run reference-style argument objects through the shim and compare the output
with the oracle at the same tolerance as the C-ABI tests."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

import oracle
from cases import assert_close, make_case, make_conv3_case

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which("node")
DRIVER = os.path.join(ROOT, "tests", "node", "run_case.mjs")
ADDON = os.path.join(ROOT, "p0pc0rn-kernels_amd", "node", "p0k.node")
pytestmark = [pytest.mark.skipif(NODE is None, reason="node is not installed"),
              pytest.mark.skipif(not os.path.exists(ADDON), reason="p0k.node is not built")]


def node(mode, d, timeout=120):
    r = subprocess.run([NODE, DRIVER, mode, str(d)], capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, r.stderr[-3000:]


def test_host_helpers_and_errors(tmp_path):
    rng = np.random.default_rng(3)
    vals = np.concatenate([rng.standard_normal(4000).astype(np.float32) * np.float32(2.0) ** rng.integers(-30, 18, 4000),
                           np.array([0, -0.0, 65504, 65520, 65519.99, 1e-8, -2 ** -24, 2 ** -25, 3 * 2 ** -26, np.inf, -np.inf,
                                     np.nan, 6.1e-5, 6.0e-5, 1e5], np.float32)]).astype(np.float32)
    vals.tofile(str(tmp_path / "values.f32"))
    f64 = [0.1, 1 / 3, 65519.0, 2.0 ** -24 * 1.5000000001, 1.0009765625 + 2 ** -12]
    (tmp_path / "f64.json").write_text(json.dumps(f64))
    rows, K = 128, 256
    W = (rng.standard_normal(rows * K) * 0.05).astype(np.float32)
    W[:64] = 0.0                                                  # an all-zero group
    W.tofile(str(tmp_path / "W.f32"))
    (tmp_path / "pack.json").write_text(json.dumps({"rows": rows, "K": K}))
    node("host", tmp_path)

    got = np.fromfile(str(tmp_path / "f2h.u16"), np.uint16)
    np.testing.assert_array_equal(got, oracle.f2h(vals))
    h2f = np.fromfile(str(tmp_path / "h2f.f32"), np.float32)
    want = oracle.h2f(np.arange(65536, dtype=np.uint16))
    np.testing.assert_array_equal(np.isnan(h2f), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_array_equal(h2f[ok].view(np.uint32), want[ok].view(np.uint32))
    # float64 inputs round to binary32 first, then to binary16 (the reference's helper stores into a Float32Array)
    assert json.loads((tmp_path / "f2h64.json").read_text()) == [int(oracle.f2h(np.float32(v))[0]) for v in f64]

    q4, deq = oracle.pack_q4(W, rows, K, want_deq=True)
    np.testing.assert_array_equal(np.fromfile(str(tmp_path / "q4.bin"), np.uint8), q4)
    np.testing.assert_array_equal(np.fromfile(str(tmp_path / "q4deq.f32"), np.float32), deq)
    np.testing.assert_array_equal(np.fromfile(str(tmp_path / "q8.bin"), np.uint8), oracle.pack_q8(W, rows, K))
    np.testing.assert_array_equal(np.fromfile(str(tmp_path / "f16.bin"), np.uint16), oracle.f16_bits(W))

    e = json.loads((tmp_path / "errors.json").read_text())
    assert e["encoding"]["message"] == "gemm: unsupported weight encoding q5"         # src/ops/gemm.js:271
    assert e["kmul32"]["message"] == "gemm: K must be a multiple of 32"               # :283
    assert e["tile"]["message"].startswith("bad tile 48x128")                         # :31
    assert e["rms_stats"]["message"].startswith("gemm: missing binding ST")           # :313
    assert "Ci % 32" in e["conv3_ci"]["message"]
    assert not any(e[k]["gpuError"] for k in ("encoding", "kmul32", "tile", "rms_stats", "conv3_ci"))
    assert e["ok"] is None and e["plan"]["kernel"] == "gemv"                           # q4, M = 4: the stream kernel
    assert e["bytes"] == [128 // 64 * 256 // 32 * 1280, 128 // 64 * 256 // 64 * 4224, 128 * 256 * 2]


def run_shim(case, tmp_path, tune=None):
    names = sorted(case.bufs)
    for n in names:
        case.bufs[n].tofile(str(tmp_path / f"{n}.bin"))
    (tmp_path / "bufs.json").write_text(json.dumps(names))
    (tmp_path / "spec.json").write_text(json.dumps({"args": case.spec, "out": case.out, "tune": tune}, default=int))
    node("gemm", tmp_path)
    out = case.bufs[case.out]
    y = np.fromfile(str(tmp_path / f"{case.out}_gpu.bin"), out.dtype)[:out.size]
    return y, json.loads((tmp_path / "result.json").read_text())


SHIM_CASES = [
    dict(enc="q4g32a.t64", epi="swiglu", M=1, N=512, K=512),
    dict(enc="q4g32a.t64", epi="swiglu", M=70, N=512, K=256, act="gelu", bias=True),
    dict(enc="q8g64s.t64", xmode="rms", epi="resadd", M=3, N=256, K=256, bias=True, gate=True),
    dict(enc="q8g64s.t64", xmode="rms", epi="resadd", M=96, N=256, K=256, store=True),
    dict(enc="q4g32a.t64", xmode="lnmod", epi="heads", M=40, N=384, K=128, Hq=1, Hkv=1, rope_mode="half", row_off=3, Ltot=64),
    dict(enc="f16", xmode="lnmod", epi="bias", M=33, N=128, K=128, res=True),
    dict(enc="q4g32a.t64", epi="onormgate", M=20, N=128, K=128),
]


@pytest.mark.gpu
@pytest.mark.parametrize("kw", SHIM_CASES, ids=lambda k: f"{k['enc']}-{k.get('xmode', 'f16')}-{k['epi']}-M{k['M']}")
def test_shim_gemm_matches_oracle(kw, tmp_path):
    print(f"shim case {kw}", flush=True)
    case = make_case(seed=11, **kw)
    got, res = run_shim(case, tmp_path)
    want = case.run_oracle()
    assert_close(got, want, fp16=want.dtype == np.uint16, what="node shim vs oracle")
    assert res["flops"] == 2 * kw["M"] * kw["N"] * kw["K"]
    assert res["info"]["architecture"].startswith("gfx950")


@pytest.mark.gpu
def test_shim_conv3_and_tune(tmp_path):
    case = make_conv3_case(T=3, H=4, W=6, C=32, N=128, pn=True)
    got, res = run_shim(case, tmp_path, tune={"acc": "f32"})
    assert_close(got, case.run_oracle(), what="node shim conv3")
    assert res["plan"]["kernel"] == "mfma"


@pytest.mark.gpu
def test_shim_load_weights(tmp_path):
    """loadWeights on a converted-model folder (manifest format p0pc0rn-kernels.weights/1, src/convert/encode.js:134)."""
    rng = np.random.default_rng(5)
    N, K, M = 128, 256, 4
    Wq = (rng.standard_normal(N * K) * 0.05).astype(np.float32)
    q4 = oracle.pack_q4(Wq, N, K)
    vec = rng.standard_normal(96).astype(np.float32)
    shard0 = np.concatenate([np.zeros(64, np.uint8), q4])                   # tensor at a non-zero offset
    shard1 = np.concatenate([np.zeros(16, np.uint8), vec.view(np.uint8)])
    mdir = tmp_path / "model"
    mdir.mkdir()
    shard0.tofile(str(mdir / "w0.bin"))
    shard1.tofile(str(mdir / "w1.bin"))
    manifest = {"format": "p0pc0rn-kernels.weights/1",
                "shards": [{"file": "w0.bin", "bytes": int(shard0.size)}, {"file": "w1.bin", "bytes": int(shard1.size)}],
                "tensors": {"blk.fc.weight": {"enc": "q4g32a.t64", "file": "w0.bin", "offset": 64, "bytes": int(q4.size),
                                              "rows": N, "cols": K, "shape": [N, K], "layout": "rows"},
                            "blk.norm.weight": {"enc": "f32", "file": "w1.bin", "offset": 16, "bytes": 384, "rows": 1,
                                                "cols": 96, "shape": [96]}}}
    (mdir / "manifest.json").write_text(json.dumps(manifest))
    x = oracle.f16_bits(rng.standard_normal(M * K).astype(np.float32))
    x.tofile(str(tmp_path / "x.bin"))
    (tmp_path / "spec.json").write_text(json.dumps({"M": M, "N": N, "K": K, "tensor": "blk.fc.weight",
                                                    "vector": "blk.norm.weight", "vlen": 96}))
    node("weights", tmp_path)
    res = json.loads((tmp_path / "result.json").read_text())
    assert res["progress"] == shard0.size + shard1.size
    assert sorted(res["names"]) == ["blk.fc.weight", "blk.norm.weight"]
    assert "not f32" in res["bad"]["message"]
    np.testing.assert_array_equal(np.fromfile(str(tmp_path / "v_gpu.f32"), np.float32), vec)
    y = np.fromfile(str(tmp_path / "y_gpu.bin"), np.uint16)[:M * N]
    case = make_case(enc="q4g32a.t64", M=M, N=N, K=K, seed=1)
    case.bufs["w"], case.bufs["x"] = q4, x
    want = case.run_oracle()
    assert_close(y, want, fp16=True, what="loadWeights tensor gemm")


@pytest.mark.gpu
def test_shim_pixstats_groupnorm_attention(tmp_path):
    """pixstats (src/ops/video.js:317), groupnormStats (src/ops/misc.js:106) and attention (src/ops/attention.js:168)
    through the shim."""
    rng = np.random.default_rng(8)
    V, Cc, pix, GC = 500, 128, 300, 64
    x = oracle.f16_bits(rng.standard_normal(V * Cc).astype(np.float32))
    gx = oracle.f16_bits(rng.standard_normal(pix * GC).astype(np.float32))
    g, b = (1 + 0.1 * rng.standard_normal(GC)).astype(np.float32), (0.1 * rng.standard_normal(GC)).astype(np.float32)
    x.tofile(str(tmp_path / "x.bin"))
    gx.tofile(str(tmp_path / "gx.bin"))
    np.concatenate([g, b]).tofile(str(tmp_path / "gb.bin"))
    L, H = 70, 2
    aq = oracle.f16_bits(oracle.randn(H * L * 128, 3, 0.5))
    ak = oracle.f16_bits(oracle.randn(L * 128, 4, 0.5))
    av = oracle.f16_bits(oracle.randn(L * 128, 5))
    for n, a in (("aq", aq), ("ak", ak), ("av", av)):
        a.tofile(str(tmp_path / f"{n}.bin"))
    (tmp_path / "spec.json").write_text(json.dumps({"V": V, "C": Cc, "pix": pix, "GC": GC, "L": L, "H": H}))
    node("stats", tmp_path)
    res = json.loads((tmp_path / "result.json").read_text())
    assert res["attnFlops"] == 4 * L * L * 128 * H
    ao = oracle.h2f(np.fromfile(str(tmp_path / "ao_gpu.bin"), np.uint16)[:L * H * 128])
    aw = oracle.h2f(oracle.attention(aq, ak, av, L, L, H, 1, 1, L))
    assert np.abs(ao - aw).max() <= 2 ** -8 * np.abs(aw).max() + 2 ** -9 * np.abs(aw).max()
    r = np.fromfile(str(tmp_path / "r_gpu.f32"), np.float32)[:V]
    np.testing.assert_allclose(r, oracle.pixstats(x, V, Cc, 1e-8), rtol=2e-6)
    ab = np.fromfile(str(tmp_path / "ab_gpu.f32"), np.float32)[:2 * GC]
    want = oracle.gn_finalize(oracle.gn_partial(gx, pix, GC), (pix + 63) // 64, GC, g, b, 1e-6)
    np.testing.assert_allclose(ab, want, rtol=2e-6, atol=1e-7)


def _safetensors(tensors):
    """a safetensors file: 8-byte header length, JSON header (dtype, shape, data_offsets), then the data"""
    header, blobs, off = {"__metadata__": {"format": "pt"}}, [], 0
    for name, (dtype, shape, raw) in tensors.items():
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    return len(h).to_bytes(8, "little") + h + b"".join(blobs)


def test_converter_helpers(tmp_path):
    """The converter helpers of src/convert/encode.js:40-133 that loadWeights callers use, with known answers: fp8 / bf16
    / fp16 decoding (e4m3 0x38 = 1, 0x7e = 448, 0x01 = 2^-9, 0x7f NaN; e5m2 0x3c = 1, 0x7b = 57344, 0x7c = inf,
    0x01 = 2^-16; bf16 0x3f80 = 1), the matrix view and encoding rule of each tensor rank, the OITHW -> OTHWI row order
    against numpy's transpose, and encodeRows against the oracle's encoders."""
    rng = np.random.default_rng(12)
    e4 = np.arange(256, dtype=np.uint8)
    raw = {"F8_E4M3": e4, "F8_E5M2": e4, "BF16": np.array([0x3F80, 0xC000, 0x0000, 0x7F80, 0x3E80], np.uint16),
           "F16": oracle.f16_bits(np.array([1.0, -2.0, 65504.0, 2 ** -24], np.float32)),
           "F32": np.array([1.5, -0.25, 3e38], np.float32)}
    for dt, a in raw.items():
        a.tofile(str(tmp_path / f"raw_{dt}.bin"))
    N, C = 64, 32
    Wc = oracle.h2f(oracle.f16_bits((rng.standard_normal(N * C * 27) * 0.05).astype(np.float32)))
    st = _safetensors({"vae.conv3.weight": ("F32", (N, C, 3, 3, 3), Wc.astype(np.float32).tobytes()),
                       "vae.norm.bias": ("F16", (N,), oracle.f16_bits(np.ones(N, np.float32)).tobytes())})
    (tmp_path / "model.safetensors").write_bytes(st)
    W = (rng.standard_normal(64 * 256) * 0.05).astype(np.float32)
    W.tofile(str(tmp_path / "W.f32"))
    shapes = [[128, 64, 3, 3], [128, 64, 3, 3, 3], [96], [], [4, 8, 256], [3072, 3072]]
    choose = [["a", [3072, 3072], None], ["a", [3072, 3072], {"bits": 8}], ["a", [3072, 3072], {"bits": 16}],
              ["a.norm", [3072], None], ["a.keep", [3072, 3072], {"keep": "keep"}], ["a.f32", [64, 64], {"f32": "f32$"}],
              ["a", [100, 3072], None], ["a", [128, 96], None], ["a", [128, 96], {"bits": 8}]]
    (tmp_path / "spec.json").write_text(json.dumps({"raw": {dt: f"raw_{dt}.bin" for dt in raw}, "conv": "vae.conv3.weight",
                                                    "shapes": shapes, "choose": choose}))
    node("convert", tmp_path)
    res = json.loads((tmp_path / "result.json").read_text())

    f8 = np.fromfile(str(tmp_path / "f32_F8_E4M3.f32"), np.float32)
    assert (f8[0x38], f8[0x7E], f8[0x01], f8[0x08], f8[0xB8]) == (1.0, 448.0, 2.0 ** -9, 2.0 ** -6, -1.0)
    assert np.isnan(f8[0x7F]) and np.isnan(f8[0xFF]) and np.isfinite(f8[0x7E])
    f5 = np.fromfile(str(tmp_path / "f32_F8_E5M2.f32"), np.float32)
    assert (f5[0x3C], f5[0x7B], f5[0x01], f5[0xBC]) == (1.0, 57344.0, 2.0 ** -16, -1.0)
    assert f5[0x7C] == np.inf and f5[0xFC] == -np.inf and np.isnan(f5[0x7D])
    # every finite e5m2 value is the fp16 with the same top byte (e5m2 is truncated binary16)
    fin = np.isfinite(f5)
    np.testing.assert_array_equal(f5[fin], oracle.h2f((e4[fin].astype(np.uint16) << 8)))
    assert list(np.fromfile(str(tmp_path / "f32_BF16.f32"), np.float32)) == [1.0, -2.0, 0.0, np.inf, 0.25]
    assert list(np.fromfile(str(tmp_path / "f32_F16.f32"), np.float32)) == [1.0, -2.0, 65504.0, 2 ** -24]
    np.testing.assert_array_equal(np.fromfile(str(tmp_path / "f32_F32.f32"), np.float32), raw["F32"])

    assert [t["name"] for t in res["list"]] == ["vae.conv3.weight", "vae.norm.bias"]
    assert res["list"][0]["shape"] == [N, C, 3, 3, 3] and res["dataStart"] % 8 == 0
    assert res["matrix"] == {"rows": N, "cols": C * 27, "layout": "OTHWI"} and res["enc"] == "f16"
    want = Wc.reshape(N, C, 27).transpose(0, 2, 1).reshape(-1)                 # OITHW -> OTHWI
    np.testing.assert_array_equal(np.fromfile(str(tmp_path / "conv_reordered.f32"), np.float32), want)
    np.testing.assert_array_equal(np.fromfile(str(tmp_path / "conv_f16.bin"), np.uint16), oracle.f16_bits(want))
    assert res["matrices"] == [{"rows": 128, "cols": 576, "layout": "OHWI"}, {"rows": 128, "cols": 1728, "layout": "OTHWI"},
                               {"rows": 1, "cols": 96, "layout": "vector"}, {"rows": 1, "cols": 1, "layout": "vector"},
                               {"rows": 32, "cols": 256, "layout": "row-major"},
                               {"rows": 3072, "cols": 3072, "layout": "row-major"}]
    assert res["encodings"] == ["q4g32a.t64", "q8g64s.t64", "f16", "f32", "f16", "f32", "f16", "q4g32a.t64", "f16"]
    assert res["tileBytes"] == [8 * 1280, 4 * 4224, 64 * 256 * 2, 64 * 256 * 4]
    np.testing.assert_array_equal(np.fromfile(str(tmp_path / "enc_q4.bin"), np.uint8), oracle.pack_q4(W, 64, 256))
    np.testing.assert_array_equal(np.fromfile(str(tmp_path / "enc_q8.bin"), np.uint8), oracle.pack_q8(W, 64, 256))
    np.testing.assert_array_equal(np.fromfile(str(tmp_path / "enc_f32.bin"), np.float32), W)
    assert "unsupported dtype I64" in res["badDtype"]["message"] and "unknown encoding q5" in res["badEnc"]["message"]


@pytest.mark.gpu
def test_reordered_conv3_weights_run_conv3(dev, tmp_path):
    """OITHW conv3 weights as a framework stores them -> the shim's reorderConvRows + encodeRows -> the conv3 GEMM on
    the GPU, against a textbook 3-D cross-correlation with the OITHW weights (replicate-padded time, zero-padded
    space)."""
    rng = np.random.default_rng(13)
    T, H, W, C, N = 4, 6, 10, 64, 128
    Wc = oracle.h2f(oracle.f16_bits((rng.standard_normal(N * C * 27) * 0.03).astype(np.float32)))
    (tmp_path / "model.safetensors").write_bytes(_safetensors({"c3": ("F32", (N, C, 3, 3, 3), Wc.tobytes())}))
    np.zeros(64 * 256, np.float32).tofile(str(tmp_path / "W.f32"))
    (tmp_path / "spec.json").write_text(json.dumps({"raw": {}, "conv": "c3", "shapes": [], "choose": []}))
    node("convert", tmp_path)
    wb = np.fromfile(str(tmp_path / "conv_f16.bin"), np.uint8)
    c = make_conv3_case(T, H, W, C, N, seed=14)
    c.bufs["w"] = wb
    c.spec["w"]["bytes"] = wb.nbytes
    got = oracle.h2f(c.run_device(dev)).astype(np.float64).reshape(T, H, W, N)
    X = c.X.reshape(T, H, W, C).astype(np.float64)
    Xp = np.pad(np.pad(X, ((1, 1), (0, 0), (0, 0), (0, 0)), mode="edge"), ((0, 0), (1, 1), (1, 1), (0, 0)))
    Wo = Wc.reshape(N, C, 3, 3, 3).astype(np.float64)
    ref = np.zeros((T, H, W, N))
    for kt in range(3):
        for ky in range(3):
            for kx in range(3):
                ref += np.einsum("thwc,nc->thwn", Xp[kt:kt + T, ky:ky + H, kx:kx + W], Wo[:, :, kt, ky, kx])
    err = np.abs(got - ref)
    assert np.all(err <= 2 ** -9 * np.abs(ref) + 2 ** -10 * np.sqrt(np.mean(ref ** 2))), f"max err {err.max()}"


@pytest.mark.gpu
def test_calibrate_measures_gemm_and_attention(tmp_path):
    """calibrate() (src/core/tune.js:39-58) sets gpu.rate.mm from timed q4 GEMMs and gpu.rate.attn from a timed
    attention call."""
    node("calibrate", tmp_path)
    res = json.loads((tmp_path / "result.json").read_text())
    for k in ("gemmF32Gflops", "gemmF16Gflops", "attnGflops"):
        assert res["calib"][k] > 10000, res
    assert res["rate"]["attn"] == pytest.approx(0.8 * res["calib"]["attnGflops"] * 1e9, rel=0.01)
    assert res["rate"]["mm"] > 1e13
