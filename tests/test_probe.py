"""The benchmark's measurement library (libp0k_probe.so): its argument checks without a GPU, and on the GPU that each
probe runs and refuses out-of-range settings. The gemm path never loads this library."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

import p0k

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "p0pc0rn-kernels_amd", "probe"))
import probe  # noqa: E402


def test_probe_library_exports():
    L = probe.lib()
    for n in probe.EXPORTS:
        assert hasattr(L, n)
    for n in ("p0k_stream_read_probe", "p0k_mfma_valu_probe", "p0k_lds_read_probe"):
        assert not hasattr(p0k.lib(), n), f"{n} is still exported by the product library"


def test_stream_read_refuses_oversized_grid_without_gpu():
    """a grid larger than the bytes need (or above 65536 workgroups) is refused before anything touches the GPU"""
    L = probe.lib()
    fake, sink = C.c_void_p(1 << 20), C.c_void_p(1 << 21)       # never dereferenced: the call is refused first
    assert L.p0kprobe_stream_read(None, fake, 1 << 20, sink, 1 << 20, 512) == p0k.E_ARG
    assert b"blocks" in L.p0kprobe_last_error()
    assert L.p0kprobe_stream_read(None, fake, 1 << 30, sink, 70000, 256) == p0k.E_ARG
    assert L.p0kprobe_stream_read(None, C.c_void_p((1 << 20) + 4), 1024, sink, 0, 512) == p0k.E_ARG   # misaligned
    assert L.p0kprobe_stream_read(None, fake, 1 << 20, sink, 0, 1024) == p0k.E_ARG                    # threads
    assert L.p0kprobe_stream_read(None, fake, 1 << 20, sink, 4, 512) == p0k.E_ARG                     # no context
    assert b"context" in L.p0kprobe_last_error()
    assert L.p0kprobe_gate(None, 10, sink) == p0k.E_ARG


@pytest.mark.gpu
def test_stream_read_probe(dev):
    """the HBM read-ceiling probe runs and refuses bad settings"""
    b, sink = dev.buffer(1 << 20), dev.buffer(16)
    try:
        probe.stream_read(dev, b, 1 << 20, sink)
        probe.stream_read(dev, b, 1 << 20, sink, blocks=9, threads=256)
        probe.gate(dev, 20, sink)
        dev.done()
        with pytest.raises(p0k.P0kError, match="threads"):
            probe.stream_read(dev, b, 1 << 20, sink, threads=1024)
        with pytest.raises(p0k.P0kError, match="blocks"):
            probe.stream_read(dev, b, 1 << 20, sink, blocks=512, threads=512)
    finally:
        dev.free(b)
        dev.free(sink)


@pytest.mark.gpu
def test_lds_read_probe(dev):
    """the LDS read probe runs, writes ordered clock pairs for every wave, and refuses out-of-range settings"""
    cus = dev.cus()
    clk = dev.buffer(32 * 16 * cus)
    try:
        for waves in (4, 8, 16):
            probe.lds_read(dev, waves, 8, clk)
            dev.done()
            t = dev.read(clk, np.uint64, 4 * waves * cus).reshape(-1, 4)
            assert np.all(t[:, 1] > t[:, 0]) and np.all(t[:, 3] >= t[:, 2]), f"waves {waves}: clocks out of order"
        with pytest.raises(p0k.P0kError, match="waves 4, 8 or 16"):
            probe.lds_read(dev, 6, 8, clk)
        small = dev.buffer(32 * 4)
        try:
            with pytest.raises(p0k.P0kError):
                probe.lds_read(dev, 4, 8, small)                 # smaller than 32 * waves * CUs bytes
        finally:
            dev.free(small)
    finally:
        dev.free(clk)


@pytest.mark.gpu
def test_mfma_valu_probe(dev):
    """the matrix-core issue probe runs and refuses out-of-range settings"""
    sink = dev.buffer(16)
    try:
        probe.mfma_valu(dev, 4, 2, 3, sink)
        probe.mfma_valu(dev, 0, 1, 3, sink, random_operands=True)
        dev.done()
        with pytest.raises(p0k.P0kError, match="waves_per_simd"):
            probe.mfma_valu(dev, 3, 2, 3, sink)
        with pytest.raises(p0k.P0kError, match="waves_per_simd"):
            probe.mfma_valu(dev, 4, 3, 3, sink)
    finally:
        dev.free(sink)
