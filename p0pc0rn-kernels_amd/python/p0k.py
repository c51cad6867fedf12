"""ctypes binding of libp0k.so (include/p0k.h) for the Python test and benchmark drivers.

The argument objects follow the reference's GemmArgs (types/index.d.ts:128-150): a dict with
``w: {enc, buf, off, bytes, rows, cols, ld}``, ``x: {buf, off, size, ld, k0, mode}``, ``y: {buf, off, size, ld, n0}``,
``M, N, K, epi, acc, tile, wr0, wr1, wk0, ev, stats, pv, bv, gt, res, store, act, heads, conv``. Strings are the
reference's ('q4g32a.t64', 'swiglu', 'gelu', 'half', ...). ``gemm_args(a, resolve)`` flattens such a dict into the C
struct; ``resolve(buf)`` returns ``(pointer, size_in_bytes)`` of whatever stands for a buffer (a device Buffer here, a
numpy array for the CPU oracle).
"""
import ctypes as C
import os

import numpy as np

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG, "libp0k.so")

ENC = {"q4g32a.t64": 1, "q8g64s.t64": 2, "f16": 3}
XMODE = {"f16": 0, "lnmod": 1, "rms": 2, "conv": 3, "conv3": 4}
EPI = {"f16": 0, "f32": 1, "resadd": 2, "swiglu": 3, "heads": 4, "bias": 5, "onormgate": 6}
ACT = {"silu": 0, "gelu": 1}
ACC = {"f32": 0, "f16": 1}

OK, E_ARG, E_HIP, E_NOMEM, E_UNSUPPORTED = 0, 1, 2, 3, 4


class GemmArgs(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint32),
        ("w_enc", C.c_int32),
        ("w_buf", C.c_void_p), ("w_off", C.c_uint64), ("w_bytes", C.c_uint64),
        ("w_rows", C.c_uint32), ("w_cols", C.c_uint32), ("w_ld", C.c_uint32),
        ("x_buf", C.c_void_p), ("x_off", C.c_uint64), ("x_size", C.c_uint64),
        ("x_ld", C.c_uint32), ("x_k0", C.c_uint32),
        ("x_mode", C.c_int32),
        ("y_buf", C.c_void_p), ("y_off", C.c_uint64), ("y_size", C.c_uint64),
        ("y_ld", C.c_uint32), ("y_n0", C.c_uint32),
        ("M", C.c_uint32), ("N", C.c_uint32), ("K", C.c_uint32),
        ("epi", C.c_int32), ("acc", C.c_int32),
        ("tile_bm", C.c_uint32), ("tile_bn", C.c_uint32),
        ("wr0", C.c_uint32), ("wr1", C.c_uint32), ("wk0", C.c_uint32),
        ("ev_buf", C.c_void_p), ("ev_off", C.c_uint32), ("ev_size", C.c_uint64),
        ("st_buf", C.c_void_p), ("st_off", C.c_uint32), ("st_size", C.c_uint64),
        ("pv_buf", C.c_void_p), ("pv_off", C.c_uint32), ("pv_stride", C.c_uint32), ("pv_size", C.c_uint64),
        ("bv_buf", C.c_void_p), ("bv_off", C.c_uint32), ("bv_up", C.c_uint32), ("bv_size", C.c_uint64),
        ("gt_buf", C.c_void_p), ("gt_size", C.c_uint64),
        ("rope_buf", C.c_void_p), ("rope_size", C.c_uint64),
        ("res", C.c_int32), ("store", C.c_int32), ("act", C.c_int32),
        ("h_Ltot", C.c_uint32), ("h_Hq", C.c_uint32), ("h_Hkv", C.c_uint32), ("h_rowOff", C.c_uint32),
        ("h_eps", C.c_float), ("h_rope_mode", C.c_int32),
        ("c_Hi", C.c_uint32), ("c_Wi", C.c_uint32), ("c_Ci", C.c_uint32), ("c_Ho", C.c_uint32), ("c_Wo", C.c_uint32),
        ("c_stride", C.c_uint32), ("c_padT", C.c_uint32), ("c_padL", C.c_uint32), ("c_ks", C.c_uint32),
        ("c_up2", C.c_int32), ("c_gn", C.c_int32), ("c_pn", C.c_int32),
    ]


class RowstatsArgs(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint32),
        ("x_buf", C.c_void_p), ("x_off", C.c_uint64), ("x_size", C.c_uint64),
        ("ld", C.c_uint32), ("c0", C.c_uint32), ("rows", C.c_uint32), ("cols", C.c_uint32),
        ("mode", C.c_int32), ("eps", C.c_float),
        ("st_buf", C.c_void_p), ("st_off", C.c_uint32), ("st_size", C.c_uint64),
    ]


class PixstatsArgs(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint32),
        ("x_buf", C.c_void_p), ("x_off", C.c_uint64), ("x_size", C.c_uint64),
        ("V", C.c_uint32), ("C", C.c_uint32), ("eps", C.c_float),
        ("r_buf", C.c_void_p), ("ro", C.c_uint32), ("r_size", C.c_uint64),
    ]


class GnArgs(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint32),
        ("x_buf", C.c_void_p), ("x_off", C.c_uint64), ("x_size", C.c_uint64),
        ("pix", C.c_uint32), ("C", C.c_uint32),
        ("part_buf", C.c_void_p), ("wg_off", C.c_uint32), ("nwg", C.c_uint32), ("part_size", C.c_uint64),
        ("gb_buf", C.c_void_p), ("g_off", C.c_uint64), ("b_off", C.c_uint64), ("gb_size", C.c_uint64),
        ("ab_buf", C.c_void_p), ("ab_off", C.c_uint32), ("ab_size", C.c_uint64),
        ("eps", C.c_float),
    ]


class AttnArgs(C.Structure):
    _fields_ = [
        ("struct_size", C.c_uint32),
        ("q_buf", C.c_void_p), ("q_off", C.c_uint64), ("q_size", C.c_uint64),
        ("k_buf", C.c_void_p), ("k_off", C.c_uint64), ("k_size", C.c_uint64),
        ("v_buf", C.c_void_p), ("v_off", C.c_uint64), ("v_size", C.c_uint64),
        ("o_buf", C.c_void_p), ("o_off", C.c_uint64), ("o_size", C.c_uint64), ("ldo", C.c_uint32),
        ("Lq", C.c_uint32), ("Lk", C.c_uint32), ("Hq", C.c_uint32), ("Hkv", C.c_uint32), ("mode", C.c_uint32),
        ("nvalid", C.c_uint32), ("scale", C.c_float), ("cap", C.c_float),
    ]


def attn_args(a, resolve):
    """attention(gpu, a) argument object (src/ops/attention.js:167) -> AttnArgs; resolve(buf) -> (pointer, size)."""
    s = AttnArgs()
    s.struct_size = C.sizeof(AttnArgs)
    for key in ("q", "k", "v", "o"):
        p, sz = resolve(a[key]["buf"])
        setattr(s, key + "_buf", p)
        setattr(s, key + "_off", _get(a[key], "off", 0))
        setattr(s, key + "_size", sz)
    s.ldo = _get(a["o"], "ld", 0)
    s.Lq, s.Lk, s.Hq, s.Hkv = a["Lq"], _get(a, "Lk", 0), a["Hq"], _get(a, "Hkv", 0)
    s.mode, s.nvalid = _get(a, "mode", 0), _get(a, "nvalid", 0)
    s.scale, s.cap = _get(a, "scale", 0.0), _get(a, "cap", 0.0)
    return s


class Tile(C.Structure):
    _fields_ = [("bm", C.c_uint32), ("bn", C.c_uint32), ("kernel", C.c_int32)]


class PoolStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("alive", "peak", "pooled", "high_water", "max_buf", "creates", "reuses",
                                          "evictions", "live_buffers", "pooled_buffers")]


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("arch", C.c_char * 64), ("cus", C.c_int32), ("xcds_hint", C.c_int32),
                ("hbm_bytes", C.c_uint64), ("clock_khz", C.c_int32), ("mem_clock_khz", C.c_int32),
                ("mem_bus_width", C.c_int32)]


EXPORTS = [
    "p0k_abi_version", "p0k_last_error", "p0k_ctx_create", "p0k_ctx_destroy", "p0k_device_info_get", "p0k_alloc",
    "p0k_ctx_reload_env", "p0k_ctx_cus", "p0k_gemm_noalloc", "p0k_gemm_noalloc_scratch_bytes", "p0k_ctx_stream",
    "p0k_ctx_workspace_stats", "p0k_gemm_plan",
    "p0k_free", "p0k_drain_pool", "p0k_pool_stats_get", "p0k_upload", "p0k_download", "p0k_copy", "p0k_sync",
    "p0k_gemm_check", "p0k_gemm", "p0k_gemm_flops", "p0k_select_tile", "p0k_rowstats_check", "p0k_rowstats",
    "p0k_attention_check", "p0k_attention", "p0k_attention_flops",
    "p0k_pixstats", "p0k_gn_part_bytes", "p0k_gn_partial", "p0k_gn_finalize", "p0k_groupnorm_stats",
    "p0k_event_create", "p0k_event_record", "p0k_event_elapsed_ms", "p0k_event_destroy",
    "p0k_tensor_bytes", "p0k_pack_q4", "p0k_pack_q8", "p0k_pack_f16",
    "p0k_graph_begin", "p0k_graph_end", "p0k_graph_launch", "p0k_graph_destroy",
]

_lib = None


def lib():
    """Load libp0k.so (fails loudly when it has not been built: there is no fallback path)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python p0pc0rn-kernels_amd/build.py`")
        L = C.CDLL(LIB_PATH)
        P, U64, I = C.c_void_p, C.c_uint64, C.c_int
        sigs = {
            "p0k_abi_version": ([], I), "p0k_last_error": ([], C.c_char_p),
            "p0k_ctx_create": ([I, C.POINTER(P)], I), "p0k_ctx_destroy": ([P], None),
            "p0k_ctx_reload_env": ([P], I), "p0k_ctx_cus": ([P], I),
            "p0k_gemm_noalloc": ([P, C.POINTER(GemmArgs)], I), "p0k_gemm_noalloc_scratch_bytes": ([], U64),
            "p0k_ctx_stream": ([P], P),
            "p0k_ctx_workspace_stats": ([P, C.POINTER(U64), C.POINTER(U64)], I),
            "p0k_gemm_plan": ([P, C.POINTER(GemmArgs), C.POINTER(Tile)], I),
            "p0k_device_info_get": ([P, C.POINTER(DeviceInfo)], I),
            "p0k_alloc": ([P, U64, C.POINTER(P)], I), "p0k_free": ([P, P], I), "p0k_drain_pool": ([P], I),
            "p0k_pool_stats_get": ([P, C.POINTER(PoolStats)], I),
            "p0k_upload": ([P, P, U64, P, U64], I), "p0k_download": ([P, P, U64, P, U64], I),
            "p0k_copy": ([P, P, U64, P, U64, U64], I), "p0k_sync": ([P], I),
            "p0k_gemm_check": ([C.POINTER(GemmArgs)], I), "p0k_gemm": ([P, C.POINTER(GemmArgs)], I),
            "p0k_gemm_flops": ([C.POINTER(GemmArgs)], C.c_double),
            "p0k_select_tile": ([C.POINTER(GemmArgs), C.POINTER(Tile)], I),
            "p0k_rowstats_check": ([C.POINTER(RowstatsArgs)], I), "p0k_rowstats": ([P, C.POINTER(RowstatsArgs)], I),
            "p0k_pixstats": ([P, C.POINTER(PixstatsArgs)], I), "p0k_gn_part_bytes": ([C.c_uint32], U64),
            "p0k_attention_check": ([C.POINTER(AttnArgs)], I), "p0k_attention": ([P, C.POINTER(AttnArgs)], I),
            "p0k_attention_flops": ([C.POINTER(AttnArgs)], C.c_double),
            "p0k_gn_partial": ([P, C.POINTER(GnArgs), C.POINTER(C.c_uint32)], I),
            "p0k_gn_finalize": ([P, C.POINTER(GnArgs)], I), "p0k_groupnorm_stats": ([P, C.POINTER(GnArgs)], I),
            "p0k_event_create": ([P, C.POINTER(P)], I), "p0k_event_record": ([P, P], I),
            "p0k_event_elapsed_ms": ([P, P, C.POINTER(C.c_float)], I), "p0k_event_destroy": ([P], None),
            "p0k_tensor_bytes": ([I, C.c_uint32, C.c_uint32], U64),
            "p0k_pack_q4": ([P, C.c_uint32, C.c_uint32, P, P], I), "p0k_pack_q8": ([P, C.c_uint32, C.c_uint32, P, P], I),
            "p0k_pack_f16": ([P, U64, P], I),
            "p0k_graph_begin": ([P], I), "p0k_graph_end": ([P, C.POINTER(P)], I), "p0k_graph_launch": ([P, P], I),
            "p0k_graph_destroy": ([P], None),
        }
        for name, (args, res) in sigs.items():
            fn = getattr(L, name)
            fn.argtypes, fn.restype = args, res
        _lib = L
    return _lib


class P0kError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


def _chk(code):
    if code != OK:
        raise P0kError(code, lib().p0k_last_error().decode())


# ---------------------------------------------------------------------------------------------- argument objects
def _get(d, k, default=None):
    if d is None:
        return default
    v = d.get(k, default)
    return default if v is None else v


def gemm_args(a, resolve):
    """Flatten a reference-style GemmArgs dict into GemmArgs. resolve(buf) -> (pointer, size)."""
    s = GemmArgs()
    s.struct_size = C.sizeof(GemmArgs)
    w = a["w"]
    if w["enc"] not in ENC:
        s.w_enc = 0
    else:
        s.w_enc = ENC[w["enc"]]
    wp, wsz = resolve(w["buf"])
    s.w_buf, s.w_off = wp, _get(w, "off", 0)
    s.w_bytes = _get(w, "bytes", wsz - s.w_off)
    s.w_rows, s.w_cols, s.w_ld = w["rows"], w["cols"], _get(w, "ld", 0)
    x = a["x"]
    s.x_buf, s.x_size = resolve(x["buf"])
    if x.get("size") is not None:
        s.x_size = x["size"] + _get(x, "off", 0)
    s.x_off, s.x_ld, s.x_k0 = _get(x, "off", 0), _get(x, "ld", 0), _get(x, "k0", 0)
    cv = a.get("conv")
    if cv:
        s.x_mode = XMODE["conv3" if cv.get("kind") == "conv3" else "conv"]
        s.c_Hi, s.c_Wi, s.c_Ci, s.c_Ho, s.c_Wo = cv["Hi"], cv["Wi"], cv["Ci"], cv["Ho"], cv["Wo"]
        s.c_stride, s.c_padT, s.c_padL, s.c_ks = _get(cv, "stride", 1), _get(cv, "padT", 0), _get(cv, "padL", 0), _get(cv, "ks", 1)
        s.c_up2, s.c_gn, s.c_pn = int(bool(cv.get("up2"))), int(bool(cv.get("gn"))), int(bool(cv.get("pn")))
    else:
        s.x_mode = XMODE[_get(x, "mode", "f16")]
    y = a["y"]
    s.y_buf, s.y_size = resolve(y["buf"])
    if y.get("size") is not None:
        s.y_size = y["size"] + _get(y, "off", 0)
    s.y_off, s.y_ld, s.y_n0 = _get(y, "off", 0), _get(y, "ld", 0), _get(y, "n0", 0)
    s.M, s.N, s.K = a["M"], a["N"], a["K"]
    s.epi = EPI.get(a.get("epi") or "f16", -1)
    s.acc = ACC[a.get("acc") or "f32"]
    t = a.get("tile")
    if t:
        s.tile_bm, s.tile_bn = t["BM"], t["BN"]
    s.wr0, s.wr1, s.wk0 = _get(a, "wr0", 0), _get(a, "wr1", 0), _get(a, "wk0", 0)
    for key, pfx in (("ev", "ev"), ("stats", "st"), ("pv", "pv"), ("bv", "bv")):
        v = a.get(key)
        if v:
            p, sz = resolve(v["buf"])
            setattr(s, pfx + "_buf", p)
            setattr(s, pfx + "_size", sz)
            setattr(s, pfx + "_off", _get(v, "off", 0))
            if key == "pv":
                s.pv_stride = _get(v, "stride", 0)
            if key == "bv":
                s.bv_up = _get(v, "up", 0)
    if a.get("gt"):
        s.gt_buf, s.gt_size = resolve(a["gt"]["buf"])
    s.res, s.store = int(bool(a.get("res"))), int(bool(a.get("store")))
    s.act = ACT[a.get("act") or "silu"]
    h = a.get("heads")
    if h:
        s.h_Ltot, s.h_Hq, s.h_Hkv, s.h_rowOff = h["Ltot"], h["Hq"], h["Hkv"], _get(h, "rowOff", 0)
        s.h_eps = _get(h, "eps", 0.0)
        s.h_rope_mode = 1 if h.get("ropeMode") == "half" else 0
        if h.get("rope"):
            s.rope_buf, s.rope_size = resolve(h["rope"]["buf"])
    return s


def numpy_resolve(arr):
    """resolve() for host numpy arrays (the CPU oracle's buffers)."""
    return arr.ctypes.data, arr.nbytes


# ---------------------------------------------------------------------------------------------- device runtime
class Buffer:
    """A device buffer from p0k_alloc (the reference's GPUBuffer with `_pf` = its size)."""
    __slots__ = ("ptr", "size", "dev")

    def __init__(self, ptr, size, dev):
        self.ptr, self.size, self.dev = ptr, size, dev


TUNING_SWITCHES = ("P0K_MFMA_TILE", "P0K_MFMA_KERNEL", "P0K_DMA_TAIL", "P0K_GEMV_MF", "P0K_GEMV_MQ4", "P0K_GEMV_MX", "P0K_GEMV_NARROW", "P0K_GEMV_SN", "P0K_GEMV_SLICES",
                   "P0K_ATTN_BQ")


def _tuning_env():
    return tuple(os.environ.get(k) for k in TUNING_SWITCHES)


class Device:
    """createGpu() over libp0k: one HIP device, one stream."""

    def __init__(self, device=0):
        L = lib()
        ctx = C.c_void_p()
        _chk(L.p0k_ctx_create(device, C.byref(ctx)))
        self.ctx = ctx
        self._env = _tuning_env()

    def _sync_env(self):
        """the context reads the P0K_* tuning switches once; read them again when this process has changed them"""
        env = _tuning_env()
        if env != self._env:
            _chk(lib().p0k_ctx_reload_env(self.ctx))
            self._env = env

    def close(self):
        if self.ctx:
            lib().p0k_ctx_destroy(self.ctx)
            self.ctx = None

    def cus(self):
        """the CU count the context plans tiles and splits for (the device's, not a constant)"""
        return lib().p0k_ctx_cus(self.ctx)

    def info(self):
        d = DeviceInfo()
        _chk(lib().p0k_device_info_get(self.ctx, C.byref(d)))
        return {"name": d.name.decode(), "arch": d.arch.decode(), "cus": d.cus, "hbm_bytes": d.hbm_bytes,
                "clock_khz": d.clock_khz, "mem_clock_khz": d.mem_clock_khz, "mem_bus_width": d.mem_bus_width}

    def buffer(self, nbytes):
        p = C.c_void_p()
        _chk(lib().p0k_alloc(self.ctx, int(nbytes), C.byref(p)))
        return Buffer(p.value, max(16, (int(nbytes) + 15) // 16 * 16), self)

    def upload(self, arr, dst=None, dst_off=0):
        arr = np.ascontiguousarray(arr)
        b = dst if dst is not None else self.buffer(arr.nbytes)
        _chk(lib().p0k_upload(self.ctx, b.ptr, dst_off, arr.ctypes.data, arr.nbytes))
        return b

    def read(self, buf, dtype=np.uint8, count=None, off=0):
        dtype = np.dtype(dtype)
        n = (buf.size - off) // dtype.itemsize if count is None else count
        out = np.empty(n, dtype=dtype)
        _chk(lib().p0k_download(self.ctx, buf.ptr, off, out.ctypes.data, out.nbytes))
        return out

    def copy(self, dst, dst_off, src, src_off, n):
        _chk(lib().p0k_copy(self.ctx, dst.ptr, dst_off, src.ptr, src_off, n))

    def free(self, buf):
        if buf is not None and buf.ptr:
            _chk(lib().p0k_free(self.ctx, buf.ptr))
            buf.ptr = None

    def done(self):
        _chk(lib().p0k_sync(self.ctx))

    def pool_stats(self):
        s = PoolStats()
        _chk(lib().p0k_pool_stats_get(self.ctx, C.byref(s)))
        return {n: getattr(s, n) for n, _ in PoolStats._fields_}

    def drain_pool(self):
        _chk(lib().p0k_drain_pool(self.ctx))

    @staticmethod
    def resolve(buf):
        return buf.ptr, buf.size

    def gemm(self, a):
        """gemm(gpu, args) of src/ops/gemm.js:268: validate, enqueue, return the FLOPs (2MNK)."""
        s = gemm_args(a, self.resolve)
        self._sync_env()
        _chk(lib().p0k_gemm(self.ctx, C.byref(s)))
        return 2 * a["M"] * a["N"] * a["K"]

    def gemm_noalloc(self, a):
        """the allocation-free gemm: workspaces from the device's static scratch array"""
        s = gemm_args(a, self.resolve)
        self._sync_env()
        _chk(lib().p0k_gemm_noalloc(self.ctx, C.byref(s)))
        return 2 * a["M"] * a["N"] * a["K"]

    def select_tile(self, a):
        """the kernel and tile p0k_gemm uses for these arguments on this context (its CU count and switches)"""
        s = gemm_args(a, lambda b: (b.ptr, b.size) if isinstance(b, Buffer) else numpy_resolve(b))
        self._sync_env()
        t = Tile()
        _chk(lib().p0k_gemm_plan(self.ctx, C.byref(s), C.byref(t)))
        return _tile_dict(t)

    def workspace_stats(self):
        live, retired = C.c_uint64(), C.c_uint64()
        _chk(lib().p0k_ctx_workspace_stats(self.ctx, C.byref(live), C.byref(retired)))
        return {"live_bytes": live.value, "retired_buffers": retired.value}

    def gemm_raw(self, s):
        _chk(lib().p0k_gemm(self.ctx, C.byref(s)))

    def rowstats(self, x, rows, cols, mode, eps, st, ld=0, c0=0, st_off=0, x_off=0):
        r = RowstatsArgs()
        r.struct_size = C.sizeof(RowstatsArgs)
        r.x_buf, r.x_off, r.x_size = x.ptr, x_off, x.size
        r.ld, r.c0, r.rows, r.cols = ld, c0, rows, cols
        r.mode, r.eps = (1 if mode == "rms" else 0), eps
        r.st_buf, r.st_off, r.st_size = st.ptr, st_off, st.size
        _chk(lib().p0k_rowstats(self.ctx, C.byref(r)))

    def attention_raw(self, s):
        _chk(lib().p0k_attention(self.ctx, C.byref(s)))

    def attention(self, a):
        """attention(gpu, a) of src/ops/attention.js:168 (head size 128); returns 4 Lq Lk 128 Hq."""
        s = attn_args(a, self.resolve)
        self._sync_env()
        _chk(lib().p0k_attention(self.ctx, C.byref(s)))
        return lib().p0k_attention_flops(C.byref(s))

    def pixstats(self, x, V, Cc, r, eps=0.0, ro=0, x_off=0):
        """pixstats(gpu, {x, r, V, C, eps, ro}) of src/ops/video.js:317."""
        a = PixstatsArgs()
        a.struct_size = C.sizeof(PixstatsArgs)
        a.x_buf, a.x_off, a.x_size = x.ptr, x_off, x.size
        a.V, a.C, a.eps = V, Cc, eps
        a.r_buf, a.ro, a.r_size = r.ptr, ro, r.size
        _chk(lib().p0k_pixstats(self.ctx, C.byref(a)))

    @staticmethod
    def _gn(x, pix, Cc, part, gb=None, g_off=0, b_off=0, ab=None, ab_off=0, eps=0.0, wg_off=0, nwg=0, x_off=0):
        a = GnArgs()
        a.struct_size = C.sizeof(GnArgs)
        if x is not None:
            a.x_buf, a.x_off, a.x_size = x.ptr, x_off, x.size
        a.pix, a.C = pix, Cc
        a.part_buf, a.wg_off, a.nwg, a.part_size = part.ptr, wg_off, nwg, part.size
        if gb is not None:
            a.gb_buf, a.g_off, a.b_off, a.gb_size = gb.ptr, g_off, b_off, gb.size
        if ab is not None:
            a.ab_buf, a.ab_off, a.ab_size = ab.ptr, ab_off, ab.size
        a.eps = eps
        return a

    def gn_partial(self, x, pix, Cc, part, wg_off=0, x_off=0):
        """gnPartial(gpu, {x, pix, C, part, wgOff}) of src/ops/misc.js:94; returns the number of partial rows."""
        n = C.c_uint32()
        _chk(lib().p0k_gn_partial(self.ctx, C.byref(self._gn(x, pix, Cc, part, wg_off=wg_off, x_off=x_off)), C.byref(n)))
        return n.value

    def gn_finalize(self, part, nwg, Cc, gb, g_off, b_off, ab, ab_off=0, eps=0.0):
        """gnFinalize(gpu, {part, nwg, C, gb: {buf, gOff, bOff}, ab: {buf, off}, eps}) of src/ops/misc.js:101."""
        a = self._gn(None, 0, Cc, part, gb, g_off, b_off, ab, ab_off, eps, nwg=nwg)
        _chk(lib().p0k_gn_finalize(self.ctx, C.byref(a)))

    def groupnorm_stats(self, x, pix, Cc, part, gb, g_off, b_off, ab, ab_off=0, eps=0.0):
        """groupnormStats(gpu, a) of src/ops/misc.js:106."""
        a = self._gn(x, pix, Cc, part, gb, g_off, b_off, ab, ab_off, eps)
        _chk(lib().p0k_groupnorm_stats(self.ctx, C.byref(a)))

    # -- events on the context's stream
    def event(self):
        e = C.c_void_p()
        _chk(lib().p0k_event_create(self.ctx, C.byref(e)))
        return e

    def record(self, e):
        _chk(lib().p0k_event_record(self.ctx, e))

    @staticmethod
    def elapsed_ms(a, b):
        ms = C.c_float()
        _chk(lib().p0k_event_elapsed_ms(a, b, C.byref(ms)))
        return ms.value

    @staticmethod
    def event_destroy(e):
        lib().p0k_event_destroy(e)

    # -- graphs
    def graph_begin(self):
        _chk(lib().p0k_graph_begin(self.ctx))

    def graph_end(self):
        g = C.c_void_p()
        _chk(lib().p0k_graph_end(self.ctx, C.byref(g)))
        return g

    def graph_launch(self, g):
        _chk(lib().p0k_graph_launch(self.ctx, g))

    @staticmethod
    def graph_destroy(g):
        lib().p0k_graph_destroy(g)


# ---------------------------------------------------------------------------------------------- encoders (host CPU)
def pack(enc, W, rows, K, want_deq=False):
    """FORMAT.md encoders of libp0k (src/convert/encode.js:56-95): fp32 [rows][K] -> uint8 bytes (+ fp32 deq)."""
    W = np.ascontiguousarray(W, dtype=np.float32).reshape(-1)
    if enc == "f16":
        out = np.empty(W.size, np.uint16)
        _chk(lib().p0k_pack_f16(W.ctypes.data, W.size, out.ctypes.data))
        return out.view(np.uint8)
    out = np.zeros(lib().p0k_tensor_bytes(ENC[enc], rows, K), np.uint8)
    deq = np.zeros(rows * K, np.float32) if want_deq else None
    fn = lib().p0k_pack_q4 if enc == "q4g32a.t64" else lib().p0k_pack_q8
    code = fn(W.ctypes.data, rows, K, out.ctypes.data, deq.ctypes.data if want_deq else None)
    if code:
        raise P0kError(code, f"{enc} needs rows % 64 == 0 and K % {32 if enc.startswith('q4') else 64} == 0")
    return (out, deq) if want_deq else out


def check(a):
    """Host-only validation of a GemmArgs dict (p0k_gemm_check); raises P0kError like the reference throws."""
    s = gemm_args(a, lambda b: (b.ptr, b.size) if isinstance(b, Buffer) else numpy_resolve(b))
    _chk(lib().p0k_gemm_check(C.byref(s)))


def select_tile(a):
    s = gemm_args(a, lambda b: (b.ptr, b.size) if isinstance(b, Buffer) else numpy_resolve(b))
    t = Tile()
    _chk(lib().p0k_select_tile(C.byref(s), C.byref(t)))
    return _tile_dict(t)


def _tile_dict(t):
    return {"BM": t.bm, "BN": t.bn, "kernel": {1: "gemv", 2: "gemv_mfma", 3: "mfma_dma", 4: "gemv_short"}.get(t.kernel, "mfma")}
