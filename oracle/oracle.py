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
import p0k  # noqa: E402  (the rowstats argument struct)

# the enumerations of include/p0k.h, restated
ENC = {"q4g32a.t64": 1, "q8g64s.t64": 2, "f16": 3}
_XMODE = {"f16": 0, "lnmod": 1, "rms": 2, "conv": 3, "conv3": 4}
_EPI = {"f16": 0, "f32": 1, "resadd": 2, "swiglu": 3, "heads": 4, "bias": 5, "onormgate": 6}
_ACT = {"silu": 0, "gelu": 1}
_ACC = {"f32": 0, "f16": 1}

# p0k_gemm_args (include/p0k.h) restated for the oracle, so that the checker flattens the reference's argument object
# (types/index.d.ts GemmArgs, src/ops/gemm.js:268-327) by its own code rather than the product's; the tests hold this
# layout to the one the C oracle was compiled against (or_gemm_args_layout) and the two flattenings to each other
_CT = {"u32": C.c_uint32, "i32": C.c_int32, "u64": C.c_uint64, "ptr": C.c_void_p, "f32": C.c_float}
_ARG_FIELDS = """
struct_size:u32 w_enc:i32 w_buf:ptr w_off:u64 w_bytes:u64 w_rows:u32 w_cols:u32 w_ld:u32
x_buf:ptr x_off:u64 x_size:u64 x_ld:u32 x_k0:u32 x_mode:i32 y_buf:ptr y_off:u64 y_size:u64 y_ld:u32 y_n0:u32
M:u32 N:u32 K:u32 epi:i32 acc:i32 tile_bm:u32 tile_bn:u32 wr0:u32 wr1:u32 wk0:u32
ev_buf:ptr ev_off:u32 ev_size:u64 st_buf:ptr st_off:u32 st_size:u64 pv_buf:ptr pv_off:u32 pv_stride:u32 pv_size:u64
bv_buf:ptr bv_off:u32 bv_up:u32 bv_size:u64 gt_buf:ptr gt_size:u64 rope_buf:ptr rope_size:u64 res:i32 store:i32 act:i32
h_Ltot:u32 h_Hq:u32 h_Hkv:u32 h_rowOff:u32 h_eps:f32 h_rope_mode:i32
c_Hi:u32 c_Wi:u32 c_Ci:u32 c_Ho:u32 c_Wo:u32 c_stride:u32 c_padT:u32 c_padL:u32 c_ks:u32 c_up2:i32 c_gn:i32 c_pn:i32
"""


class OracleArgs(C.Structure):
    _fields_ = [(name, _CT[t]) for name, t in (f.split(":") for f in _ARG_FIELDS.split())]


def oracle_args(a):
    """The reference's argument object (numpy arrays as buffers) as p0k_gemm_args: views are (buffer, byte offset,
    extent from the buffer start: the given size plus the offset, else the whole buffer; gemm.js:305-307), w.bytes
    defaults to the rest of the buffer, vectors are (buffer, offset in floats or rows, buffer size), flags are 0 / 1,
    and absent fields stay 0 (the C side's defaults: ld = K / N, stride = ks = 1, eps = 1e-6)."""
    o = OracleArgs()
    o.struct_size = C.sizeof(OracleArgs)
    opt = lambda d, k, dflt=0: dflt if (d is None or d.get(k) is None) else d[k]   # noqa: E731

    w = a["w"]
    o.w_enc = ENC.get(w["enc"], 0)
    o.w_buf, o.w_off = w["buf"].ctypes.data, opt(w, "off")
    o.w_bytes = w["bytes"] if w.get("bytes") is not None else w["buf"].nbytes - o.w_off
    o.w_rows, o.w_cols, o.w_ld = w["rows"], w["cols"], opt(w, "ld")
    for key, extra in (("x", ("ld", "k0")), ("y", ("ld", "n0"))):
        v = a[key]
        off = opt(v, "off")
        setattr(o, key + "_buf", v["buf"].ctypes.data)
        setattr(o, key + "_off", off)
        setattr(o, key + "_size", v["buf"].nbytes if v.get("size") is None else v["size"] + off)
        for e in extra:
            setattr(o, key + "_" + e, opt(v, e))
    conv = a.get("conv")
    if conv:
        o.x_mode = _XMODE["conv3"] if conv.get("kind") == "conv3" else _XMODE["conv"]
        for k in ("Hi", "Wi", "Ci", "Ho", "Wo"):
            setattr(o, "c_" + k, conv[k])
        o.c_stride, o.c_ks = opt(conv, "stride", 1), opt(conv, "ks", 1)
        o.c_padT, o.c_padL = opt(conv, "padT"), opt(conv, "padL")
        o.c_up2, o.c_gn, o.c_pn = (1 if conv.get(k) else 0 for k in ("up2", "gn", "pn"))
    else:
        o.x_mode = _XMODE[a["x"].get("mode") or "f16"]
    o.M, o.N, o.K = a["M"], a["N"], a["K"]
    o.epi = _EPI.get(a.get("epi") or "f16", -1)
    o.acc = _ACC[a.get("acc") or "f32"]
    if a.get("tile"):
        o.tile_bm, o.tile_bn = a["tile"]["BM"], a["tile"]["BN"]
    o.wr0, o.wr1, o.wk0 = opt(a, "wr0"), opt(a, "wr1"), opt(a, "wk0")
    for key, pre, more in (("ev", "ev", ()), ("stats", "st", ()), ("pv", "pv", ("stride",)), ("bv", "bv", ("up",))):
        v = a.get(key)
        if not v:
            continue
        setattr(o, pre + "_buf", v["buf"].ctypes.data)
        setattr(o, pre + "_size", v["buf"].nbytes)
        setattr(o, pre + "_off", opt(v, "off"))
        for e in more:
            setattr(o, pre + "_" + e, opt(v, e))
    if a.get("gt"):
        o.gt_buf, o.gt_size = a["gt"]["buf"].ctypes.data, a["gt"]["buf"].nbytes
    o.res, o.store = (1 if a.get(k) else 0 for k in ("res", "store"))
    o.act = _ACT[a.get("act") or "silu"]
    hd = a.get("heads")
    if hd:
        o.h_Ltot, o.h_Hq, o.h_Hkv, o.h_rowOff = hd["Ltot"], hd["Hq"], hd["Hkv"], opt(hd, "rowOff")
        o.h_eps = opt(hd, "eps", 0.0)
        o.h_rope_mode = 1 if hd.get("ropeMode") == "half" else 0
        if hd.get("rope"):
            o.rope_buf, o.rope_size = hd["rope"]["buf"].ctypes.data, hd["rope"]["buf"].nbytes
    return o


def args_layout():
    """(sizeof, offsets of every field in declaration order) of p0k_gemm_args as the C oracle was compiled"""
    buf = (C.c_uint64 * 128)()
    n = lib().or_gemm_args_layout(buf, 128)
    return int(buf[0]), [int(buf[i]) for i in range(1, n)]


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
            ("or_gemm", [C.POINTER(OracleArgs), C.c_uint32, C.c_uint32], I),
            ("or_gemm_args_layout", [C.POINTER(C.c_uint64), C.c_uint32], C.c_uint32),
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
    s = oracle_args(a)
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
