"""Python face of the CPU oracle (libp0k_oracle.so, built from oracle/p0k_oracle.c). TEST INFRASTRUCTURE ONLY.

Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker; the product never imports it.
Arrays are numpy; fp16 values travel as uint16 bit patterns where bit-exactness matters.
"""
import ctypes as C
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libp0k_oracle.so")
sys.path.insert(0, os.path.join(ROOT, "p0pc0rn-kernels_amd", "python"))
import p0k  # noqa: E402  (GemmArgs, the argument flattening)

ENC = p0k.ENC


def build():
    """Compile the C restatement (gcc, fp contraction off so fp32 steps round one by one)."""
    src = os.path.join(HERE, "p0k_oracle.c")
    subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-ffp-contract=off", "-fno-fast-math",
                    "-I" + os.path.join(ROOT, "include"), src, "-o", LIB, "-lm"], check=True)
    return LIB


_L = None


def lib():
    global _L
    if _L is None:
        if not os.path.exists(LIB):
            build()
        L = C.CDLL(LIB)
        P, I, F = C.c_void_p, C.c_int, C.c_float
        for name, args, res in [
            ("or_f2h", [F], C.c_uint16), ("or_h2f", [C.c_uint16], F), ("or_rhe", [F], F),
            ("or_pack_q4", [P, I, I, P, P], I), ("or_pack_q8", [P, I, I, P, P], I),
            ("or_pack_f16", [P, C.c_int64, P], None), ("or_tensor_bytes", [I, I, I], C.c_int64),
            ("or_weight_f16", [I, P, C.c_uint32, C.c_uint32, C.c_uint32], C.c_uint16),
            ("or_dequant", [I, P, I, I, P], None),
            ("or_randn", [P, C.c_int64, C.c_uint32, C.c_double], None),
            ("or_rand_uniform", [P, C.c_int64, C.c_uint32, F, F], None),
            ("or_gemm", [C.POINTER(p0k.GemmArgs), C.c_uint32, C.c_uint32], I),
            ("or_set_weight_model", [I], None),
            ("or_rowstats", [C.POINTER(p0k.RowstatsArgs)], I),
            ("or_cpu_gemm", [P, P, I, I, I, P], None),
            ("or_cpu_conv3", [P, P, I, I, I, I, I, P], None),
            ("or_pixstats", [P, C.c_uint32, C.c_uint32, C.c_float, P], None),
            ("or_attention", [P, P, P, P] + [C.c_uint32] * 7 + [C.c_float, C.c_float], None),
            ("or_gn_partial", [P, C.c_uint32, C.c_uint32, P], None),
            ("or_gn_finalize", [P, C.c_uint32, C.c_uint32, C.c_float, P, P, P], None),
        ]:
            fn = getattr(L, name)
            fn.argtypes, fn.restype = args, res
        _L = L
    return _L


def _p(a):
    return a.ctypes.data


def f2h(x):
    """fp32 array -> fp16 bit patterns (uint16), src/core/gpu.js:276-291."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(x.size, np.uint16)
    L = lib()
    for i in range(x.size):
        out[i] = L.or_f2h(float(x[i]))
    return out


def f16_bits(x):
    """fp32 -> fp16 bits in C (fast path for arrays): packF16 of src/convert/encode.js:92-95."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(x.size, np.uint16)
    lib().or_pack_f16(_p(x), x.size, _p(out))
    return out


def h2f(h):
    return np.ascontiguousarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def pack_q4(W, rows, K, want_deq=False):
    W = np.ascontiguousarray(W, dtype=np.float32)
    out = np.zeros(rows // 64 * (K // 32) * 1280, np.uint8)
    deq = np.zeros(rows * K, np.float32) if want_deq else None
    r = lib().or_pack_q4(_p(W), rows, K, _p(out), _p(deq) if want_deq else None)
    if r:
        raise ValueError("q4g32a.t64 needs rows % 64 == 0 and K % 32 == 0")
    return (out, deq) if want_deq else out


def pack_q8(W, rows, K, want_deq=False):
    W = np.ascontiguousarray(W, dtype=np.float32)
    out = np.zeros(rows // 64 * (K // 64) * 4224, np.uint8)
    deq = np.zeros(rows * K, np.float32) if want_deq else None
    r = lib().or_pack_q8(_p(W), rows, K, _p(out), _p(deq) if want_deq else None)
    if r:
        raise ValueError("q8g64s.t64 needs rows % 64 == 0 and K % 64 == 0")
    return (out, deq) if want_deq else out


def dequant(enc, w, rows, cols):
    """decode a q4/q8 tensor to the fp16 weights the kernel multiplies by (uint16 bits, [rows][cols])."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.empty(rows * cols, np.uint16)
    lib().or_dequant(ENC[enc], _p(w), rows, cols, _p(out))
    return out.reshape(rows, cols)


def randn(n, seed, scale=1.0):
    """test/kernels.test.js:13 — xorshift32 + Box-Muller, fp32."""
    out = np.empty(n, np.float32)
    lib().or_randn(_p(out), n, seed, scale)
    return out


def rand_uniform(n, seed, lo, hi):
    out = np.empty(n, np.float32)
    lib().or_rand_uniform(_p(out), n, seed, lo, hi)
    return out


KERNEL_WEIGHTS, CPU_WEIGHTS = 0, 1


def gemm(a, m0=0, m1=None, weights=KERNEL_WEIGHTS):
    """Run rows [m0, m1) of a reference-style GemmArgs dict whose buffers are numpy arrays; Y is written in place.
    weights: KERNEL_WEIGHTS (fp16-rounded, the reference kernel) or CPU_WEIGHTS (fp32, the test suite's cpuGemm)."""
    s = p0k.gemm_args(a, p0k.numpy_resolve)
    lib().or_set_weight_model(weights)
    try:
        r = lib().or_gemm(C.byref(s), m0, a["M"] if m1 is None else m1)
    finally:
        lib().or_set_weight_model(KERNEL_WEIGHTS)
    if r:
        raise ValueError("oracle: bad gemm arguments")


def rowstats(x, rows, cols, mode, eps, st, ld=0, c0=0, st_off=0):
    r = p0k.RowstatsArgs()
    r.struct_size = C.sizeof(p0k.RowstatsArgs)
    r.x_buf, r.x_off, r.x_size = x.ctypes.data, 0, x.nbytes
    r.ld, r.c0, r.rows, r.cols = ld, c0, rows, cols
    r.mode, r.eps = (1 if mode == "rms" else 0), eps
    r.st_buf, r.st_off, r.st_size = st.ctypes.data, st_off, st.nbytes
    lib().or_rowstats(C.byref(r))


def cpu_gemm(X, W, M, N, K):
    X = np.ascontiguousarray(X, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    Y = np.empty(M * N, np.float32)
    lib().or_cpu_gemm(_p(X), _p(W), M, N, K, _p(Y))
    return Y


def cpu_conv3(X, Wt, T, H, W, Cc, N):
    X = np.ascontiguousarray(X, np.float32)
    Wt = np.ascontiguousarray(Wt, np.float32)
    Y = np.empty(T * H * W * N, np.float32)
    lib().or_cpu_conv3(_p(X), _p(Wt), T, H, W, Cc, N, _p(Y))
    return Y


def pixstats(x16, V, Cc, eps=1e-8):
    """R[v] = 1 / sqrt(sum_c x^2 / C + eps) (src/ops/video.js:301-321); x16: fp16 bits [V][C]."""
    x16 = np.ascontiguousarray(x16, np.uint16)
    r = np.empty(V, np.float32)
    lib().or_pixstats(_p(x16), V, Cc, eps, _p(r))
    return r


def gn_partial(x16, pix, Cc):
    """partial rows [ceil(pix / 64)][32][(n, mean, M2, 0)] (src/ops/misc.js:50-76)."""
    x16 = np.ascontiguousarray(x16, np.uint16)
    part = np.zeros(((pix + 63) // 64) * 32 * 4, np.float32)
    lib().or_gn_partial(_p(x16), pix, Cc, _p(part))
    return part


def gn_finalize(part, nwg, Cc, gamma, beta, eps=1e-6):
    """(a[C], b[C]) with GN(x) = a x + b (src/ops/misc.js:77-91)."""
    part = np.ascontiguousarray(part, np.float32)
    gamma = np.ascontiguousarray(gamma, np.float32)
    beta = np.ascontiguousarray(beta, np.float32)
    ab = np.empty(2 * Cc, np.float32)
    lib().or_gn_finalize(_p(part), nwg, Cc, eps, _p(gamma), _p(beta), _p(ab))
    return ab


def attention(q16, k16, v16, Lq, Lk, Hq, Hkv, mode=0, nvalid=None, scale=None, cap=0.0, ldo=None):
    """cpuAttn (test/kernels.test.js:30-49), head size 128: fp16 bits in, O [Lq][ldo] fp16 bits out."""
    ldo = ldo or Hq * 128
    nvalid = Lk if nvalid is None else nvalid
    scale = 1.0 / np.sqrt(128.0) if scale is None else scale
    q16, k16, v16 = (np.ascontiguousarray(a, np.uint16) for a in (q16, k16, v16))
    o = np.zeros(Lq * ldo, np.uint16)
    lib().or_attention(_p(q16), _p(k16), _p(v16), _p(o), Lq, Lk, Hq, Hkv, ldo, mode, nvalid, scale, cap)
    return o
