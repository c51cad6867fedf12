"""pixstats (src/ops/video.js:301-321) and GroupNorm(32) statistics (src/ops/misc.js:50-109): the oracle pinned by
closed forms on the CPU, the HIP kernels against the oracle on the GPU. Tolerances: rstd and the affine coefficients
within 2e-6 relative of the fp64 oracle (fp32 sums of fp16 values over at most a few hundred thousand terms);
partial means / M2 within 1e-5 relative plus an absolute floor for values near zero."""
import numpy as np
import pytest

import oracle
import p0k


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def vals(x16):
    return x16.view(np.float16).astype(np.float64)


# ------------------------------------------------------------------------------------------------ oracle pins (CPU)
def test_pixstats_oracle_closed_form():
    rng = np.random.default_rng(1)
    V, C = 37, 36
    x = f16(rng.standard_normal(V * C) * 3)
    want = 1.0 / np.sqrt((vals(x).reshape(V, C) ** 2).mean(1) + 1e-8)
    np.testing.assert_allclose(oracle.pixstats(x, V, C), want, rtol=1e-6)
    z = np.zeros(4 * 8, np.uint16)                                   # all-zero voxel: 1 / sqrt(eps)
    np.testing.assert_allclose(oracle.pixstats(z, 4, 8, 1e-8), np.full(4, 1e4), rtol=1e-6)


@pytest.mark.parametrize("pix,C", [(1, 32), (64, 64), (130, 128), (300, 512), (257, 256)])
def test_groupnorm_oracle_is_whole_tensor_statistics(pix, C):
    """Merging the 64-pixel chunks (Chan) gives the statistics of the whole tensor, and a x + b is the textbook
    GroupNorm gamma (x - mean) / sqrt(var + eps) + beta (biased variance per group of C/32 channels)."""
    rng = np.random.default_rng(pix + C)
    x = f16(rng.standard_normal(pix * C) * 2 + 0.5)
    part = oracle.gn_partial(x, pix, C)
    g = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    b = (0.1 * rng.standard_normal(C)).astype(np.float32)
    ab = oracle.gn_finalize(part, (pix + 63) // 64, C, g, b, 1e-6)
    xv = vals(x).reshape(pix, 32, C // 32)
    mean = xv.mean(axis=(0, 2))
    var = xv.var(axis=(0, 2))
    a_want = g / np.sqrt(np.repeat(var, C // 32) + 1e-6)
    b_want = b - np.repeat(mean, C // 32) * a_want
    np.testing.assert_allclose(ab[:C], a_want, rtol=1e-5)
    np.testing.assert_allclose(ab[C:], b_want, rtol=1e-5, atol=1e-6 * np.abs(a_want).max())
    p = part.reshape(-1, 32, 4)
    assert np.all(p[:, :, 0].sum(0) == pix * (C // 32))               # counts
    assert np.all(p[:, :, 3] == 0)


def test_groupnorm_partial_bytes_and_checks():
    assert p0k.lib().p0k_gn_part_bytes(1) == 512 and p0k.lib().p0k_gn_part_bytes(64) == 512
    assert p0k.lib().p0k_gn_part_bytes(65) == 1024 and p0k.lib().p0k_gn_part_bytes(0) == 0


# ------------------------------------------------------------------------------------------------ HIP kernels (GPU)
@pytest.mark.gpu
@pytest.mark.parametrize("V,C,ro", [(1, 128, 0), (1000, 128, 5), (333, 36, 0), (64, 512, 3), (4097, 4, 0)])
def test_pixstats_matches_oracle(dev, V, C, ro):
    print(f"pixstats V={V} C={C}", flush=True)
    rng = np.random.default_rng(V)
    x = f16(rng.standard_normal(V * C) * 4)
    dx = dev.upload(x)
    dr = dev.buffer((V + ro) * 4)
    try:
        dev.pixstats(dx, V, C, dr, eps=0.0, ro=ro)
        got = dev.read(dr, np.float32, V + ro)
        np.testing.assert_allclose(got[ro:], oracle.pixstats(x, V, C, 1e-8), rtol=2e-6)
        assert np.all(got[:ro] == 0)
    finally:
        dev.free(dx)
        dev.free(dr)


@pytest.mark.gpu
@pytest.mark.parametrize("pix,C", [(1, 32), (100, 64), (4096, 128), (1000, 512), (777, 256)])
def test_groupnorm_matches_oracle(dev, pix, C):
    print(f"groupnorm pix={pix} C={C}", flush=True)
    rng = np.random.default_rng(pix * 7 + C)
    x = f16(rng.standard_normal(pix * C) * 1.5 - 0.25)
    g = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    b = (0.1 * rng.standard_normal(C)).astype(np.float32)
    gb = np.concatenate([np.zeros(4, np.float32), g, b])
    dx, dgb = dev.upload(x), dev.upload(gb)
    nwg = (pix + 63) // 64
    dpart = dev.buffer(p0k.lib().p0k_gn_part_bytes(pix))
    dab = dev.buffer(2 * C * 4 + 8)
    try:
        dev.groupnorm_stats(dx, pix, C, dpart, dgb, 16, 16 + 4 * C, dab, ab_off=2)
        part_want = oracle.gn_partial(x, pix, C).reshape(nwg, 32, 4)
        part = dev.read(dpart, np.float32, nwg * 128).reshape(nwg, 32, 4)
        np.testing.assert_array_equal(part[:, :, 0], part_want[:, :, 0])
        np.testing.assert_allclose(part[:, :, 1], part_want[:, :, 1], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(part[:, :, 2], part_want[:, :, 2], rtol=1e-5, atol=1e-5)
        ab = dev.read(dab, np.float32, 2 * C + 2)[2:]
        np.testing.assert_allclose(ab, oracle.gn_finalize(part_want.ravel(), nwg, C, g, b, 1e-6), rtol=2e-6, atol=1e-7)
    finally:
        for d in (dx, dgb, dpart, dab):
            dev.free(d)


@pytest.mark.gpu
def test_groupnorm_banded_partials_merge(dev):
    """gnPartial over two bands of one tensor (wgOff) then gnFinalize equals the whole-tensor statistics."""
    pix, C = 640, 128
    rng = np.random.default_rng(9)
    x = f16(rng.standard_normal(pix * C))
    g, b = np.ones(C, np.float32), np.zeros(C, np.float32)
    dgb = dev.upload(np.concatenate([g, b]))
    dx = dev.upload(x)
    dpart = dev.buffer(p0k.lib().p0k_gn_part_bytes(pix))
    dab, dab2 = dev.buffer(2 * C * 4), dev.buffer(2 * C * 4)
    try:
        n1 = dev.gn_partial(dx, 256, C, dpart)                                   # pixels [0, 256)
        n2 = dev.gn_partial(dx, pix - 256, C, dpart, wg_off=n1, x_off=256 * C * 2)
        dev.gn_finalize(dpart, n1 + n2, C, dgb, 0, 4 * C, dab)
        dev.groupnorm_stats(dx, pix, C, dpart, dgb, 0, 4 * C, dab2)
        a1, a2 = dev.read(dab, np.float32, 2 * C), dev.read(dab2, np.float32, 2 * C)
        np.testing.assert_allclose(a1, a2, rtol=1e-6, atol=1e-7)
    finally:
        for d in (dgb, dx, dpart, dab, dab2):
            dev.free(d)
