"""ctypes binding of libp0k_probe.so, the benchmark's measurement kernels (p0k_probe.h): the HBM read ceiling, the
matrix-core issue ceiling, the LDS read ceiling and the launch gate of the timed regions. Only bench.py and the probe
tests use it; the gemm path never loads it."""
import ctypes as C
import os

import p0k

PROBE_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libp0k_probe.so")
EXPORTS = ["p0kprobe_last_error", "p0kprobe_stream_read", "p0kprobe_mfma_valu", "p0kprobe_lds_read", "p0kprobe_gate"]
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(PROBE_LIB):
            raise RuntimeError(f"{PROBE_LIB} is missing: build it with `python p0pc0rn-kernels_amd/build.py lib`")
        p0k.lib()                                   # libp0k.so first: the probe library links against it
        L = C.CDLL(PROBE_LIB)
        P, U32, U64, I = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int
        sigs = {"p0kprobe_last_error": ([], C.c_char_p),
                "p0kprobe_stream_read": ([P, P, U64, P, U32, U32], I),
                "p0kprobe_mfma_valu": ([P, I, I, I, I, P], I),
                "p0kprobe_lds_read": ([P, I, I, P], I),
                "p0kprobe_gate": ([P, U32, P], I)}
        for name, (args, res) in sigs.items():
            fn = getattr(L, name)
            fn.argtypes, fn.restype = args, res
        _lib = L
    return _lib


def _chk(code):
    if code != p0k.OK:
        raise p0k.P0kError(code, lib().p0kprobe_last_error().decode())


def stream_read(dev, buf, nbytes, sink, blocks=0, threads=512):
    """the HBM read ceiling kernel: read nbytes of buf, nothing stored"""
    _chk(lib().p0kprobe_stream_read(dev.ctx, buf.ptr, int(nbytes), sink.ptr, int(blocks), int(threads)))


def mfma_valu(dev, valu_per_mfma, waves_per_simd, iters, sink, random_operands=False):
    """the matrix-core issue ceiling kernel"""
    _chk(lib().p0kprobe_mfma_valu(dev.ctx, int(valu_per_mfma), int(waves_per_simd), int(iters),
                                  int(bool(random_operands)), sink.ptr))


def lds_read(dev, waves, iters, clk):
    """the LDS read ceiling kernel; clk: a buffer of 32 * waves * CUs bytes"""
    if clk.size < 32 * waves * dev.cus():
        raise p0k.P0kError(p0k.E_ARG, "lds_read: clk holds fewer than 32 * waves * CUs bytes")
    _chk(lib().p0kprobe_lds_read(dev.ctx, int(waves), int(iters), clk.ptr))


def gate(dev, microseconds, sink):
    """a one-wave kernel that waits `microseconds` on the GPU, so the work enqueued behind it starts back to back"""
    _chk(lib().p0kprobe_gate(dev.ctx, int(microseconds), sink.ptr))
