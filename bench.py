"""Benchmark of the MI355X `gemm` path on BASELINE.json's configurations, one GPU.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME[,NAME]] [--no-cpu]

A step is one gemm call (one pass of the hot path over one batch of synthetic input, all inputs resident in HBM).
The headline line is the q4 GEMV decode with the SwiGLU epilogue at M = 1 (weight rows 28672 =
gate 14336 | up 14336, K 4096): `value` is its HBM throughput in GB/s of algorithmic bytes. The same JSON line carries
every other config under "workloads", each with its own roofline fraction: decode M = 2, 4, 8 and 16, the plain q4 GEMV
N 14336, q8 prefill with RMSNorm + fp32 residual add (and its fp16-residual `bias` + `res` variant, and the rowstats
pass it needs, timed on its own), the DiT QKV / GeGLU GEMMs, conv3 and the attention consumer.

Timing: the timed calls are plain launches on the library's stream, enqueued behind a gate kernel (a bounded wait on
the GPU) so that the warmup calls run straight into the timed ones and the calls run back to back; HIP events on that
stream bracket them, one after every group of calls, so every workload also reports the p10 / median / p90 of its
per-call time over the groups. For the HBM-bound decode the calls rotate through enough
weight copies (> 256 MB) that no call finds its weights in the MALL. Inputs come from numpy's PCG64 generator with
fixed seeds, encoded with libp0k's own FORMAT.md encoders (BASELINE.json value recipes).

cpu_baseline: the build's JavaScript restatement of the reference's CPU path (cpuGemm, float64 sums over dequantised
fp32 weights, with the same prologue / epilogue formulas; oracle/cpu_ref.mjs) timed in Node on this host, one core,
on a bounded sample: for the headline, whole M = 1 calls repeated for about 10 s; for the other workloads one call's
weight decode plus a few rows of M, scaled linearly in M (the cost is exactly linear in M).

    python bench.py --mfma-ceiling

the matrix-core ceilings: how many VALU instructions per 32x32x16 MFMA a loop can hide (p0kprobe_mfma_valu) with
constant operands, the rate the matrix cores sustain on random operands (the clock under a full MFMA load), and the
vendor library's plain fp16 GEMM at the configs' shapes for scale.

    python bench.py --hbm-ceiling

the streaming-read ceiling of the headline's 73.4 MB over several launch shapes (p0kprobe_stream_read).

    python bench.py --lds-ceiling

the LDS read bandwidth of one CU (bytes per shader clock) and the clock the part held, with 4, 8 and 16 waves
(p0kprobe_lds_read).

    python bench.py --copy-calib

runs only a plain device-to-device copy of 1 GiB, 5 times (torch's copy kernel): the reference workload for scaling the
FETCH_SIZE / WRITE_SIZE counters of rocprofv3 into bytes (what they read for a copy of known size).
"""
import argparse
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "p0pc0rn-kernels_amd", "python"))
sys.path.insert(0, os.path.join(ROOT, "p0pc0rn-kernels_amd", "probe"))
import p0k  # noqa: E402
import probe  # noqa: E402      the measurement kernels (libp0k_probe.so): ceilings and the launch gate

HBM_PEAK = 8.0e12          # B/s, MI355X published
FP16_PEAK = 2.5e15         # FLOP/s dense fp16 MFMA, MI355X published
MALL = 256 << 20

# HBM bytes per launch from rocprofv3 counters (profiles/k_gemv*_decode_M*.md, k_stream_read_73MB_ceiling.md): FETCH_SIZE and WRITE_SIZE in
# KiB per dispatch, each times what the same counter reads per byte of a plain 1 GiB device copy (`--copy-calib`:
# FETCH_SIZE reads half the bytes, WRITE_SIZE all of them). Counters cannot be read inside the timed run: the
# headline's are measured by child rocprofv3 runs at the start of the bench (measure_traffic); for the other
# workloads, and when rocprofv3 is not available, the figures of the last profiled build are kept here.
FETCH_FACTOR, WRITE_FACTOR = 2.0, 1.0
TRAFFIC_KIB = {"decode_q4_swiglu_M1": (36003, 28), "decode_q4_swiglu_M1_long": (36003, 28),
               "decode_q4_swiglu_M4": (36123, 112), "decode_q4_swiglu_M16": (37218, 448),
               "hbm_read_ceiling_73MB": (35851, 0), "hbm_read_ceiling_10MB": (5135, 0), "prefill_rowstats_rms": (16405, 64),
               "decode_q4_plain_M1": (18020, 28), "decode_q4_plain_N4096_M1": (5192, 8), "decode_q8_plain_M1": (29663, 28), "decode_q8_plain_N4096_M1": (8526, 8),
               # MFMA workloads: every kernel of one call (prologue pass + GEMM launches)
               "prefill_q8_rms_resadd": (82670, 49152), "prefill_q8_rms_bias_f16res": (74494, 32768),
               "dit_qkv_q4_lnmod_heads": (132062, 98304), "dit_up_q4_geglu": (250812, 98304),
               "conv3_128_T13x92x160": (168504, 47840), "dit_attention_24x4096": (36917, 26433)}


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16)


# ------------------------------------------------------------------------------------------------ workloads
class Workload:
    """Device buffers + a list of argument dicts (one per rotation copy) for one config."""

    def __init__(self, name, desc, bound, flops, algo_bytes, M, args, bufs, extra=None, kind="gemm"):
        self.name, self.desc, self.bound, self.flops, self.algo_bytes = name, desc, bound, flops, algo_bytes
        self.M, self.args, self.bufs, self.extra, self.kind = M, args, bufs, extra or {}, kind


def decode_q4(dev, M, copies=None, glu=True, n_out=14336, enc="q4g32a.t64"):
    """q4 GEMV decode, out 14336 with SwiGLU (weight rows [gate 14336 | up 14336]), K 4096; glu=False:
    the plain q4 GEMV N n_out with the f16 epilogue (14336: 36.7 MB of weights; 4096: the same model's attention
    projection, 10.5 MB); enc: the same plain GEMV with q8 weights (decode of a q8-encoded model)."""
    N_out, K = n_out, 4096
    rows = 2 * N_out if glu else N_out
    r = rng(1)
    W = (r.standard_normal((rows, K), dtype=np.float32) * np.float32(0.02))
    wb = p0k.pack(enc, W, rows, K)
    del W
    copies = copies or max(4, -(-(2 * MALL) // wb.nbytes))
    bufs = [dev.upload(wb) for _ in range(copies)]
    x = dev.upload(f16(r.standard_normal(M * K)))
    y = dev.buffer(M * N_out * 2)
    bufs += [x, y]
    args = [{"w": {"enc": enc, "buf": b, "off": 0, "bytes": wb.nbytes, "rows": rows, "cols": K},
             "x": {"buf": x}, "y": {"buf": y, "ld": N_out}, "M": M, "N": rows, "K": K, "epi": "swiglu", "wr0": 0,
             "wr1": N_out} for b in bufs[:copies]]
    if not glu:
        for a in args:
            a.update(epi="f16")
            del a["wr1"]
    nbytes = wb.nbytes + M * K * 2 + M * N_out * 2
    if not glu:
        wn = "q4" if enc == "q4g32a.t64" else "q8"
        name = f"decode_{wn}_plain_M{M}" if N_out == 14336 else f"decode_{wn}_plain_N{N_out}_M{M}"
        return Workload(name, f"{wn} GEMV, M={M}, N={N_out}, K={K}, f16 epilogue", "hbm",
                        2.0 * M * rows * K, nbytes, M, args, bufs, {"weight_copies": copies, "weight_bytes": wb.nbytes})
    return Workload(f"decode_q4_swiglu_M{M}", f"q4 GEMV + SwiGLU, M={M}, out {N_out}, weight rows {rows}, K={K}",
                    "hbm", 2.0 * M * rows * K, nbytes, M, args, bufs, {"weight_copies": copies, "weight_bytes": wb.nbytes})


def prefill_q8(dev):
    """q8 GEMM M 2048 N 4096 K 4096, RMSNorm prologue (fp32 x, gamma 1+N(0,0.1), eps 1e-6 through
    rowstats) and the fp32 residual-add epilogue (R N(0,1))."""
    M, N, K = 2048, 4096, 4096
    r = rng(2)
    W = r.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    wb = p0k.pack("q8g64s.t64", W, N, K)
    del W
    xw = dev.upload(f16(r.standard_normal(M * K)).astype(np.float32))
    st = dev.buffer(M * 8)
    dev.rowstats(xw, M, K, "rms", 1e-6, st)
    gam = dev.upload((1 + 0.1 * r.standard_normal(K)).astype(np.float32))
    R = dev.upload(f16(r.standard_normal(M * N)).astype(np.float32))
    w = dev.upload(wb)
    args = [{"w": {"enc": "q8g64s.t64", "buf": w, "off": 0, "bytes": wb.nbytes, "rows": N, "cols": K},
             "x": {"buf": xw, "mode": "rms"}, "stats": {"buf": st}, "pv": {"buf": gam},
             "y": {"buf": R}, "M": M, "N": N, "K": K, "epi": "resadd"}]
    nbytes = wb.nbytes + M * K * 4 + 2 * M * N * 4 + M * 8 + K * 4
    return Workload("prefill_q8_rms_resadd", "q8 GEMM M=2048 N=4096 K=4096, RMSNorm prologue, fp32 residual add",
                    "mfma", 2.0 * M * N * K, nbytes, M, args, [xw, st, gam, R, w])


def prefill_q8_f16res(dev):
    """configs[2], the fp16-residual variant: the same q8 GEMM and RMSNorm prologue with the `bias` epilogue in place
    over an fp16 residual (`res`, zero bias): Y_f16 = f16(acc + 0 + Y_f16)."""
    M, N, K = 2048, 4096, 4096
    r = rng(2)
    W = r.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    wb = p0k.pack("q8g64s.t64", W, N, K)
    del W
    xw = dev.upload(f16(r.standard_normal(M * K)).astype(np.float32))
    st = dev.buffer(M * 8)
    dev.rowstats(xw, M, K, "rms", 1e-6, st)
    gam = dev.upload((1 + 0.1 * r.standard_normal(K)).astype(np.float32))
    R = dev.upload(f16(r.standard_normal(M * N)))
    bias = dev.buffer(N * 4)
    w = dev.upload(wb)
    args = [{"w": {"enc": "q8g64s.t64", "buf": w, "off": 0, "bytes": wb.nbytes, "rows": N, "cols": K},
             "x": {"buf": xw, "mode": "rms"}, "stats": {"buf": st}, "pv": {"buf": gam},
             "ev": {"buf": bias}, "y": {"buf": R}, "M": M, "N": N, "K": K, "epi": "bias", "res": True}]
    nbytes = wb.nbytes + M * K * 4 + 2 * M * N * 2 + M * 8 + K * 4 + N * 4
    return Workload("prefill_q8_rms_bias_f16res", "q8 GEMM M=2048 N=4096 K=4096, RMSNorm prologue, fp16 residual "
                    "(bias epilogue in place, zero bias)", "mfma", 2.0 * M * N * K, nbytes, M, args,
                    [xw, st, gam, R, bias, w])


def prefill_rowstats(dev):
    """configs[2]'s rowstats pass on its own: RMS statistics of the fp32 x (2048 x 4096, 33.5 MB read)."""
    M, K = 2048, 4096
    r = rng(2)
    x = f16(r.standard_normal(M * K)).astype(np.float32)
    copies = -(-(2 * MALL) // x.nbytes)                 # rotate copies past the MALL, as for the decode weights
    xs = [dev.upload(x) for _ in range(copies)]
    st = dev.buffer(M * 8)
    args = [{"x": xw, "rows": M, "cols": K, "mode": "rms", "eps": 1e-6, "st": st} for xw in xs]
    return Workload("prefill_rowstats_rms", "rowstats (RMS) of configs[2]'s fp32 x, 2048 x 4096", "hbm", 3.0 * M * K,
                    M * K * 4 + M * 8, M, args, xs + [st], {"x_copies": copies}, kind="rowstats")


def rope2d(L, grid_w, theta=10000.0):
    tok = np.arange(L)
    y, x = tok // grid_w, tok % grid_w
    inv = theta ** (-np.arange(32) / 32.0)
    ang = np.concatenate([y[:, None] * inv, x[:, None] * inv], axis=1)
    rp = np.empty((L, 64, 2), np.float32)
    rp[..., 0], rp[..., 1] = np.cos(ang), np.sin(ang)
    return rp.ravel()


def dit_qkv(dev):
    """configs[3](a): q4, M 4096 tokens (64x64 patches), K 3072, N 9216 = 24 Q + 24 K + 24 V heads of 128;
    LayerNorm + adaLN prologue (shift / scale N(0, 0.5)) and the QK-RMSNorm + 2-D RoPE (theta 1e4) head split."""
    M, N, K = 4096, 9216, 3072
    r = rng(3)
    W = r.standard_normal((N, K), dtype=np.float32) * np.float32(0.02)
    wb = p0k.pack("q4g32a.t64", W, N, K)
    del W
    xw = dev.upload(f16(r.standard_normal(M * K)).astype(np.float32))
    st = dev.buffer(M * 8)
    dev.rowstats(xw, M, K, "ln", 1e-6, st)
    pv = dev.upload((0.5 * r.standard_normal(2 * K)).astype(np.float32))
    ev = dev.upload((1 + 0.1 * r.standard_normal(256)).astype(np.float32))
    rp = dev.upload(rope2d(M, 64))
    w = dev.upload(wb)
    y = dev.buffer(N * M * 2)
    args = [{"w": {"enc": "q4g32a.t64", "buf": w, "off": 0, "bytes": wb.nbytes, "rows": N, "cols": K},
             "x": {"buf": xw, "mode": "lnmod"}, "stats": {"buf": st}, "pv": {"buf": pv, "stride": K},
             "ev": {"buf": ev}, "y": {"buf": y}, "M": M, "N": N, "K": K, "epi": "heads",
             "heads": {"Ltot": M, "Hq": 24, "Hkv": 24, "eps": 1e-6, "rope": {"buf": rp}}}]
    nbytes = wb.nbytes + M * K * 4 + M * N * 2 + M * 128 * 4
    return Workload("dit_qkv_q4_lnmod_heads", "q4 M=4096 N=9216 K=3072, LN+adaLN prologue, QK-norm + 2-D RoPE heads",
                    "mfma", 2.0 * M * N * K, nbytes, M, args, [xw, st, pv, ev, rp, w, y])


def dit_up(dev):
    """configs[3](b): q4 up-projection with the GeGLU epilogue, M 4096, K 3072, weight rows 24576 (gate | up)."""
    M, K, N_out = 4096, 3072, 12288
    rows = 2 * N_out
    r = rng(4)
    W = r.standard_normal((rows, K), dtype=np.float32) * np.float32(0.02)
    wb = p0k.pack("q4g32a.t64", W, rows, K)
    del W
    x = dev.upload(f16(r.standard_normal(M * K)))
    w = dev.upload(wb)
    y = dev.buffer(M * N_out * 2)
    args = [{"w": {"enc": "q4g32a.t64", "buf": w, "off": 0, "bytes": wb.nbytes, "rows": rows, "cols": K},
             "x": {"buf": x}, "y": {"buf": y, "ld": N_out}, "M": M, "N": rows, "K": K, "epi": "swiglu", "act": "gelu",
             "wr0": 0, "wr1": N_out}]
    nbytes = wb.nbytes + M * K * 2 + M * N_out * 2
    return Workload("dit_up_q4_geglu", "q4 M=4096 K=3072, weight rows 24576 (gate|up), GeGLU epilogue, out 12288",
                    "mfma", 2.0 * M * rows * K, nbytes, M, args, [x, w, y])


def conv3(dev):
    """3x3x3 conv, Ci = Co = 128, clip T 13 x 92 x 160 (THWC fp16 N(0,1)), fp16 weights N(0, 0.02)."""
    T, H, W, C, N = 13, 92, 160, 128, 128
    K, M = 27 * C, T * H * W
    r = rng(5)
    wt = dev.upload(f16(0.02 * r.standard_normal(N * K)))
    x = dev.upload(f16(r.standard_normal(M * C)))
    y = dev.buffer(M * N * 2)
    args = [{"w": {"enc": "f16", "buf": wt, "off": 0, "bytes": N * K * 2, "rows": N, "cols": K},
             "x": {"buf": x}, "y": {"buf": y}, "M": M, "N": N, "K": K,
             "conv": {"kind": "conv3", "Hi": H, "Wi": W, "Ci": C, "Ho": H, "Wo": W, "stride": T}}]
    nbytes = N * K * 2 + M * C * 2 + M * N * 2
    return Workload("conv3_128_T13x92x160", "3x3x3 conv 128->128 over a 13x92x160 clip, whole-clip call", "mfma",
                    2.0 * M * N * K, nbytes, M, args, [wt, x, y])


def dit_attn(dev):
    """the consumer of configs[3](a)'s heads output: attention over 24 heads of 128, 4096 tokens (no mask)."""
    H, L = 24, 4096
    r = rng(6)
    q = dev.upload(f16(0.5 * r.standard_normal(H * L * 128)))
    k = dev.upload(f16(0.5 * r.standard_normal(H * L * 128)))
    v = dev.upload(f16(r.standard_normal(H * L * 128)))
    o = dev.buffer(L * H * 128 * 2)
    args = [{"q": {"buf": q}, "k": {"buf": k}, "v": {"buf": v}, "o": {"buf": o}, "Lq": L, "Lk": L, "Hq": H, "Hkv": H}]
    return Workload("dit_attention_24x4096", "attention, 24 heads of 128, 4096 queries x 4096 keys, no mask", "mfma",
                    4.0 * L * L * 128 * H, 4 * H * L * 128 * 2, L, args, [q, k, v, o], kind="attn")


def hbm_ceiling(dev, blocks=0, threads=512, nbytes=None, name=None):
    """the measured HBM read ceiling for the headline: a plain streaming read (p0kprobe_stream_read, nothing computed or
    stored) of as many bytes as the q4 decode's weights (73,400,320), rotated over the same number of copies; by default
    with the decode GEMV's grid (blocks 0: 7/8 of the CUs, 512 threads)"""
    nbytes = nbytes or 28672 // 64 * (4096 // 32) * 1280
    copies = max(4, -(-(2 * MALL) // nbytes))
    bufs = [dev.buffer(nbytes) for _ in range(copies)]
    sink = dev.buffer(16)
    args = [{"buf": b, "bytes": nbytes, "sink": sink, "blocks": blocks, "threads": threads} for b in bufs]
    name = name or "hbm_read_ceiling_73MB" + (f"_{blocks}x{threads}" if blocks else "")
    return Workload(name, f"plain streaming read of the decode's weight bytes (ceiling probe, grid "
                          f"{blocks or 'GEMV'} x {threads} threads)", "hbm", 0.0,
                    nbytes, 1, args, bufs + [sink], {"weight_copies": copies}, kind="probe")


def renamed(wl, name, desc):
    wl.name, wl.desc = name, desc
    return wl


BUILDERS = {
    "decode1": lambda d: decode_q4(d, 1), "hbm_ceiling": hbm_ceiling,
    "decode1_long": lambda d: renamed(decode_q4(d, 1), "decode_q4_swiglu_M1_long",
                                      "the headline workload over a long run (at least 2000 calls, events every 64)"), "decode4": lambda d: decode_q4(d, 4), "decode16": lambda d: decode_q4(d, 16),
    "decode2": lambda d: decode_q4(d, 2), "decode8": lambda d: decode_q4(d, 8),
    "decode1_plain": lambda d: decode_q4(d, 1, glu=False),
    "decode1_proj": lambda d: decode_q4(d, 1, glu=False, n_out=4096),
    "decode1_q8": lambda d: decode_q4(d, 1, glu=False, enc="q8g64s.t64"),
    "decode1_q8_proj": lambda d: decode_q4(d, 1, glu=False, n_out=4096, enc="q8g64s.t64"),
    "hbm_ceiling_proj": lambda d: hbm_ceiling(d, 256, 256, nbytes=4096 // 64 * (4096 // 32) * 1280,
                                              name="hbm_read_ceiling_10MB"),
    "prefill": prefill_q8, "prefill_f16res": prefill_q8_f16res, "prefill_rowstats": prefill_rowstats,
    "dit_qkv": dit_qkv, "dit_up": dit_up, "conv3": conv3, "dit_attn": dit_attn,
}


# ------------------------------------------------------------------------------------------------ timing
GATE_MIN_US = 200          # the launch gate ahead of each timed region: at least this long, and longer than the host
GATE_MAX_US = 100000       # takes to enqueue the region's calls (measured per call before the region)


def time_workload(dev, wl, steps, warmup, single=False):
    """Time exactly `steps` calls of the workload (rotating over its argument sets), `warmup` untimed calls right
    before them. The calls are plain launches on the library's stream (a serving loop's calls): a gate kernel first
    holds the GPU while this thread enqueues the warmup calls, an event, the timed calls and an event, so on the GPU
    the warmup calls run straight into the timed ones and every call starts as its predecessor ends, with no host
    launch latency inside the timed region. (Replaying the same calls from a HIP graph measured 0.1-0.4 us per call
    slower on this part.) Events after every `group` timed calls (64 for memory-bound lines, 8 otherwise) give the
    per-call distribution; single: one group of all `steps` calls (the headline and its ceiling).
    Returns (ms per call from the events, wall ms per call, calls, distribution, gate facts)."""
    import ctypes as C
    L = p0k.lib()
    if wl.kind == "attn":
        structs = [p0k.attn_args(a, dev.resolve) for a in wl.args]
        run = dev.attention_raw
        for s in structs:
            p0k._chk(L.p0k_attention_check(C.byref(s)))
    elif wl.kind == "probe":
        structs = wl.args
        run = lambda a: probe.stream_read(dev, a["buf"], a["bytes"], a["sink"], a["blocks"], a["threads"])   # noqa: E731
    elif wl.kind == "rowstats":
        structs = wl.args
        run = lambda a: dev.rowstats(a["x"], a["rows"], a["cols"], a["mode"], a["eps"], a["st"])   # noqa: E731
    else:
        structs = [p0k.gemm_args(a, dev.resolve) for a in wl.args]
        run = dev.gemm_raw
        for s in structs:
            p0k._chk(L.p0k_gemm_check(C.byref(s)))
    n_arg = len(structs)
    for s in structs:
        run(s)                          # one call per argument set first: sizes the workspaces
    dev.done()
    probe_calls = max(8, 2 * n_arg)     # the host's enqueue cost per call, for the gate's length
    t = time.perf_counter()
    for i in range(probe_calls):
        run(structs[i % n_arg])
    enq_s = (time.perf_counter() - t) / probe_calls
    dev.done()
    group = steps if single else max(1, min(steps, 64 if wl.bound == "hbm" else 8))
    groups, rem = divmod(steps, group)
    gate_us = int(min(GATE_MAX_US, max(GATE_MIN_US, 2.0 * (warmup + steps) * enq_s * 1e6 + 100)))
    ev = [dev.event() for _ in range(groups + 2)]
    sink = dev.buffer(16)
    probe.gate(dev, 1, sink)            # the gate's code object is loaded at its first launch: not inside the region
    dev.done()
    t0 = time.perf_counter()
    probe.gate(dev, gate_us, sink)
    for i in range(warmup):
        run(structs[i % n_arg])
    dev.record(ev[0])
    k = warmup
    for gi in range(groups):
        for _ in range(group):
            run(structs[k % n_arg])
            k += 1
        dev.record(ev[gi + 1])
    for _ in range(rem):
        run(structs[k % n_arg])
        k += 1
    dev.record(ev[-1])
    t_enq = time.perf_counter() - t0
    dev.done()
    wall = time.perf_counter() - t0
    dev.free(sink)
    ms = dev.elapsed_ms(ev[0], ev[-1])
    per = sorted(dev.elapsed_ms(ev[i], ev[i + 1]) / group for i in range(groups))
    for e in ev:
        dev.event_destroy(e)
    assert k - warmup == steps
    gate = {"gate_us": gate_us, "host_enqueue_us": round(t_enq * 1e6, 1), "gate_covered_enqueue": t_enq * 1e6 < gate_us}
    if not gate["gate_covered_enqueue"]:
        log(f"{wl.name}: the host took {t_enq * 1e6:.0f} us to enqueue, longer than the {gate_us} us gate")
    q = lambda f: per[min(groups - 1, int(f * groups))]   # noqa: E731
    dist = None if single else {"p10": round(q(0.1), 5), "median": round(q(0.5), 5), "p90": round(q(0.9), 5),
                                "groups": groups, "calls_per_group": group, "remainder_calls": rem}
    return ms / steps, wall / steps * 1e3, steps, dist, gate


def roofline(wl, ms):
    sec = ms * 1e-3
    if wl.bound == "hbm":
        ach = wl.algo_bytes / sec / 1e9
        t = TRAFFIC_KIB.get(wl.name)
        traffic = int((FETCH_FACTOR * t[0] + WRITE_FACTOR * t[1]) * 1024) if t else None
        return {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": round(ach * 1e9 / HBM_PEAK, 4), "traffic": traffic}
    ach = wl.flops / sec / 1e12
    t = TRAFFIC_KIB.get(wl.name)
    traffic = int((FETCH_FACTOR * t[0] + WRITE_FACTOR * t[1]) * 1024) if t else None
    return {"bound": "mfma", "achieved": round(ach, 2), "peak": FP16_PEAK / 1e12, "unit": "TFLOP/s",
            "frac": round(ach * 1e12 / FP16_PEAK, 4), "traffic": traffic}


# ------------------------------------------------------------------------------------------------ live HBM traffic
def _pmc_mean(counter, args, kernel, timeout=150):
    """Mean per-dispatch value of one rocprofv3 counter for the kernels whose name contains `kernel`, from a child
    `rocprofv3 --pmc <counter> -- python3 bench.py <args>` run (its own process: this one has not touched the GPU
    yet). None when rocprofv3 is absent or the run fails."""
    import csv
    import glob
    import shutil
    import tempfile
    exe = shutil.which("rocprofv3")
    if not exe:
        return None
    d = tempfile.mkdtemp(prefix="p0k_pmc_", dir="/tmp")
    env = dict(os.environ, TMPDIR="/tmp")
    try:
        r = subprocess.run([exe, "--pmc", counter, "-d", d, "-o", "run", "--output-format", "csv", "--",
                            sys.executable, os.path.abspath(__file__)] + args, cwd="/tmp", env=env,
                           stdout=subprocess.DEVNULL, stderr=subprocess.PIPE, timeout=timeout)
        if r.returncode != 0:
            log(f"rocprofv3 --pmc {counter} failed ({r.returncode}): {r.stderr.decode(errors='replace')[-300:]}")
            return None
        vals = []
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(f) as fh:
                for row in csv.DictReader(fh):
                    if kernel in row["Kernel_Name"] and row["Counter_Name"] == counter:
                        vals.append(float(row["Counter_Value"]))
        return sum(vals) / len(vals) if vals else None
    except (OSError, subprocess.TimeoutExpired, KeyError, ValueError) as e:
        log(f"rocprofv3 --pmc {counter}: {e}")
        return None
    finally:
        shutil.rmtree(d, ignore_errors=True)


def measure_traffic():
    """The headline kernel's HBM bytes per launch, measured in this run: FETCH_SIZE and WRITE_SIZE (KiB per dispatch,
    one counter per rocprofv3 pass) of the decode call, each scaled by what the same counter reads per byte of a
    plain 1 GiB device copy (`--copy-calib`) in the same way. None (and the last profiled figures are used) when any
    pass fails."""
    big = ["--only", "decode1", "--no-cpu", "--no-traffic", "--steps", "10", "--warmup", "2"]
    fetch = _pmc_mean("FETCH_SIZE", big, "k_gemv")
    write = _pmc_mean("WRITE_SIZE", big, "k_gemv")
    cf = _pmc_mean("FETCH_SIZE", ["--copy-calib"], "copyBuffer") if fetch is not None else None
    cw = _pmc_mean("WRITE_SIZE", ["--copy-calib"], "copyBuffer") if write is not None else None
    if None in (fetch, write, cf, cw) or cf <= 0 or cw <= 0:
        return None
    ff, wf = (1 << 30) / (cf * 1024), (1 << 30) / (cw * 1024)
    return {"bytes": int(fetch * 1024 * ff + write * 1024 * wf), "fetch_kib": round(fetch, 1), "write_kib": round(write, 1),
            "fetch_factor": round(ff, 4), "write_factor": round(wf, 4)}


# ------------------------------------------------------------------------------------------------ CPU baseline
def cpu_baseline(config, rows, target_s=0.0):
    """Run the JavaScript CPU restatement in Node: one call over `rows` rows of M, repeated for about target_s seconds
    when target_s > 0; returns its JSON report or None."""
    script = os.path.join(ROOT, "oracle", "cpu_ref.mjs")
    if not os.path.exists(script):
        return None
    try:
        out = subprocess.run(["node", script, "bench", config, str(rows), str(target_s)], capture_output=True,
                             text=True, timeout=240)
    except (OSError, subprocess.TimeoutExpired) as e:
        log(f"cpu baseline {config}: {e}")
        return None
    if out.returncode != 0:
        log(f"cpu baseline {config} failed: {out.stderr[-400:]}")
        return None
    return json.loads(out.stdout.strip().splitlines()[-1])


HBM_SECONDARY_CALLS = 1000   # timed calls of each memory-bound workload other than the headline (at least)
LONG_RUN_CALLS = 2000        # timed calls of the headline's long-run line (at least)
SINGLE = ("decode1", "hbm_ceiling")   # timed as one group of exactly --steps calls (the headline and its ceiling)
CPU_HEADLINE_S = 10.0   # seconds of CPU work timed for the headline workload (whole calls, repeated)
CPU_SAMPLE = {   # workload -> (cpu_ref config, rows of M timed)
    "decode_q4_swiglu_M1": ("decode", 1), "decode_q4_swiglu_M4": ("decode", 4), "decode_q4_swiglu_M16": ("decode", 8),
    "prefill_q8_rms_resadd": ("prefill", 8), "dit_qkv_q4_lnmod_heads": ("dit_qkv", 8), "dit_up_q4_geglu": ("dit_up", 8),
    "conv3_128_T13x92x160": ("conv3", 64),
}


def copy_calib(nbytes=1 << 30, reps=5):
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "reps": reps}), flush=True)


def mfma_probe_rate(dev, sink, v, wps, iters, rnd):
    """one timed launch of p0kprobe_mfma_valu (after a short untimed one): (ms, TFLOP/s, fraction of the peak)"""
    probe.mfma_valu(dev, v, wps, 10, sink, rnd)
    dev.done()
    e0, e1 = dev.event(), dev.event()
    dev.record(e0)
    probe.mfma_valu(dev, v, wps, iters, sink, rnd)
    dev.record(e1)
    dev.done()
    ms = dev.elapsed_ms(e0, e1)
    dev.event_destroy(e0)
    dev.event_destroy(e1)
    flop = 32768.0 * 8 * iters * 4 * dev.cus() * wps
    return ms, round(flop / ms / 1e9, 1), round(flop / ms / 1e9 / (FP16_PEAK / 1e12), 4)


def lds_ceiling(dev, iters=4096):
    """`--lds-ceiling`: LDS read bandwidth of one CU with 4, 8 and 16 waves issuing conflict-free 16-byte reads
    (p0kprobe_lds_read, one workgroup per CU, all CUs). Each wave records the shader clock and the 100 MHz reference
    clock around its loop; per CU the loop runs from its first wave's start to its last wave's end, so the line gives
    bytes per shader clock of a CU and the clock the part held, averaged over the CUs of the second launch."""
    cus = dev.cus()
    clk = dev.buffer(32 * 16 * cus)
    rows = []
    for waves in (4, 8, 16):
        for _ in range(2):                                   # the first launch warms up, the second is read
            probe.lds_read(dev, waves, iters, clk)
            dev.done()
        t = dev.read(clk, np.uint64, 4 * waves * cus).reshape(cus, waves, 4).astype(np.float64)
        cyc = t[:, :, 1].max(axis=1) - t[:, :, 0].min(axis=1)
        ref = (t[:, :, 3].max(axis=1) - t[:, :, 2].min(axis=1)) / 100e6
        nbytes = waves * 64 * 16 * 16.0 * iters
        rows.append({"waves": waves, "bytes_per_clock_per_cu": round(float(np.mean(nbytes / cyc)), 1),
                     "gb_s_per_cu": round(float(np.mean(nbytes / ref)) / 1e9, 1),
                     "clock_ghz": round(float(np.mean(cyc / ref)) / 1e9, 3)})
        log(f"lds ceiling, {waves} waves: {rows[-1]}")
    dev.free(clk)
    print(json.dumps({"lds_read_ceiling": rows, "what": "16-byte conflict-free LDS reads per lane, one workgroup per "
                      "CU, all CUs (p0kprobe_lds_read)", "iters": iters}), flush=True)


def mfma_ceiling(dev):
    """`--mfma-ceiling`: FLOP rate of 8 independent 32x32x16 fp16 MFMAs per iteration with V packed-fp16 FMAs per
    MFMA, one and two waves per SIMD (p0kprobe_mfma_valu), timed with events on the library's stream; first with
    sparse constant operands (the issue rate), then with pseudo-random operands over about 50 ms per launch (the rate
    the part sustains on real data: the matrix cores' power draw sets the clock). Last, for scale, the vendor library's
    plain fp16 GEMM (torch.matmul -> hipBLASLt, no dequant, no prologue / epilogue) at the configs' shapes."""
    sink = dev.buffer(16)
    rows = []
    for rnd, iters, vs in ((False, 2000, (0, 2, 4, 6, 8, 10, 12)), (True, 40000, (0, 4, 6, 8))):
        for wps in (1, 2):
            for v in vs:
                ms, tf, fr = mfma_probe_rate(dev, sink, v, wps, iters // wps, rnd)
                rows.append({"operands": "random" if rnd else "constant", "waves_per_simd": wps, "valu_per_mfma": v,
                             "ms": round(ms, 4), "tflops": tf, "frac": fr})
                log(f"mfma probe {rows[-1]['operands']:8s} waves/SIMD {wps} VALU/MFMA {v:2d}: {tf} TFLOP/s ({fr})")
    dev.free(sink)
    # the library yardstick runs in a child process: torch's HIP runtime does not share this process's device
    lib = []
    try:
        out = subprocess.run([sys.executable, os.path.abspath(__file__), "--library-gemm"], capture_output=True, text=True,
                             timeout=300)
        sys.stderr.write(out.stderr)
        lib = json.loads(out.stdout.strip().splitlines()[-1])["library_fp16_gemm"] if out.returncode == 0 else []
    except (OSError, subprocess.TimeoutExpired, ValueError, IndexError, KeyError) as e:
        log(f"library yardstick failed: {e}")
    print(json.dumps({"mfma_valu_ceiling": rows, "library_fp16_gemm": lib}), flush=True)


def library_gemm():
    """`--library-gemm`: the vendor library's plain fp16 GEMM (torch.matmul -> hipBLASLt; no dequant, no prologue or
    epilogue) at the configs' GEMM shapes, N(0,1) x 0.02 N(0,1) operands, timed with torch events"""
    import torch
    lib = []
    for (m, n, k, what) in ((2048, 4096, 4096, "configs[2] shape"), (4096, 9216, 3072, "DiT QKV shape"),
                            (4096, 24576, 3072, "DiT up shape (weight rows)"), (4096, 4096, 4096, "4096^3"),
                            (191360, 128, 3456, "conv3 shape, X materialised (1.32 GB)")):
        g = torch.Generator(device="cuda").manual_seed(7)
        a = torch.randn(m, k, device="cuda", dtype=torch.float16, generator=g)
        b = torch.randn(n, k, device="cuda", dtype=torch.float16, generator=g) * 0.02
        for _ in range(3):
            torch.matmul(a, b.t())
        torch.cuda.synchronize()
        reps = max(5, int(2e13 // (2 * m * n * k)))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            torch.matmul(a, b.t())
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        tf = 2.0 * m * n * k / ms / 1e9
        lib.append({"what": what, "M": m, "N": n, "K": k, "ms": round(ms, 5), "tflops": round(tf, 1),
                    "frac": round(tf * 1e12 / FP16_PEAK, 4)})
        log(f"torch.matmul fp16 {m}x{n}x{k} ({what}): {ms * 1e3:.1f} us, {tf:.0f} TFLOP/s ({lib[-1]['frac']})")
    print(json.dumps({"library_fp16_gemm": lib}), flush=True)


def hbm_ceiling_sweep(dev, steps, warmup):
    """`--hbm-ceiling`: the streaming-read ceiling of the headline's 73.4 MB over several launch shapes, in the bench's
    graph timing: how much of the HBM peak one launch of that many bytes can reach on this part, whatever its grid"""
    rows = []
    for blocks, threads in ((0, 512), (256, 512), (512, 512), (512, 256), (1024, 256), (2048, 256)):
        wl = hbm_ceiling(dev, blocks, threads)
        ms, _, _, dist, _ = time_workload(dev, wl, steps, warmup)
        rows.append({"blocks": blocks or dev.cus() * 7 // 8, "threads": threads, "ms_per_call": round(ms, 5),
                     "gbps": round(wl.algo_bytes / ms / 1e6, 1), "frac": round(wl.algo_bytes / (ms * 1e-3) / HBM_PEAK, 4),
                     "median_ms": dist["median"] if dist else None})
        log(f"stream read {rows[-1]['blocks']} x {threads}: {ms * 1e3:.2f} us/call, {rows[-1]['gbps']} GB/s")
        for b in wl.bufs:
            dev.free(b)
        dev.drain_pool()
    print(json.dumps({"hbm_read_ceiling": rows}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", default="")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calib", action="store_true")
    ap.add_argument("--mfma-ceiling", action="store_true")
    ap.add_argument("--hbm-ceiling", action="store_true")
    ap.add_argument("--lds-ceiling", action="store_true")
    ap.add_argument("--library-gemm", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the live counter runs of the headline's traffic")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU (the gemm path has no multi-GPU mode here); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    if a.copy_calib:
        copy_calib()
        return
    if a.library_gemm:
        library_gemm()
        return
    names = [n for n in (a.only.split(",") if a.only else BUILDERS)]
    live_traffic = None
    if not a.no_traffic and "decode1" in names and not (a.mfma_ceiling or a.hbm_ceiling or a.lds_ceiling):
        live_traffic = measure_traffic()           # child processes, before this one touches the GPU
        log(f"headline traffic from counters in this run: {live_traffic}")
    dev = p0k.Device(0)
    if a.mfma_ceiling:
        mfma_ceiling(dev)
        dev.close()
        return
    if a.hbm_ceiling:
        hbm_ceiling_sweep(dev, a.steps, a.warmup)
        dev.close()
        return
    if a.lds_ceiling:
        lds_ceiling(dev)
        dev.close()
        return
    info = dev.info()
    log(f"device {info}")
    results = {}
    for n in names:
        wl = BUILDERS[n](dev)
        # the headline runs exactly --steps calls; the other memory-bound lines (10-20 us per call) at least
        # HBM_SECONDARY_CALLS, so that one slow group of a short burst does not decide their mean
        if wl.bound != "hbm":
            steps = max(10, a.steps // 10)
        elif n in SINGLE:
            steps = a.steps
        else:
            steps = max(a.steps, LONG_RUN_CALLS if n == "decode1_long" else HBM_SECONDARY_CALLS)
        ms, wall_ms, count, dist, gate = time_workload(dev, wl, steps,
                                                       a.warmup if wl.bound == "hbm" else max(2, a.warmup // 10),
                                                       single=n in SINGLE)
        rf = roofline(wl, ms)
        res = {"name": wl.name, "desc": wl.desc, "M": wl.M, "ms_per_call": round(ms, 5), "calls": count,
               "wall_ms_per_call": round(wall_ms, 5), "gate": gate,
               "ms_per_call_dist": dist,
               "tflops": round(wl.flops / ms / 1e9, 3), "gbps": round(wl.algo_bytes / ms / 1e6, 1),
               "algo_bytes": wl.algo_bytes, "flops": wl.flops, "roofline": rf, **wl.extra}
        log(f"{wl.name}: {ms * 1e3:.2f} us/call  {res['gbps']} GB/s  {res['tflops']} TFLOP/s  frac {rf['frac']}")
        results[n] = res
        for b in wl.bufs:
            dev.free(b)
        dev.drain_pool()
    mceil = None
    if any(r["roofline"]["bound"] == "mfma" for r in results.values()):
        # the matrix cores' sustained rate on random operands (two waves per SIMD, no other work), measured here: what
        # the part holds under a full MFMA load, against which each MFMA workload's rate is also reported
        sink = dev.buffer(16)
        ms, tf, fr = mfma_probe_rate(dev, sink, 0, 2, 20000, True)
        dev.free(sink)
        mceil = {"what": "8 independent 32x32x16 fp16 MFMAs per iteration on pseudo-random operands, two waves per "
                         "SIMD, all CUs, one launch (p0kprobe_mfma_valu)", "ms": round(ms, 3), "tflops": tf, "frac": fr}
        log(f"mfma ceiling (random operands): {tf} TFLOP/s ({fr})")
        for r in results.values():
            if r["roofline"]["bound"] == "mfma":
                r["vs_mfma_ceiling"] = round(r["tflops"] / tf, 4)
    cores = 1
    if not a.no_cpu:
        cache = {}
        for n, res in results.items():
            if res["name"] not in CPU_SAMPLE:
                continue
            cfg, rows = CPU_SAMPLE[res["name"]]
            whole = n == "decode1"                                       # the headline: time whole M=1 calls
            key = (cfg, rows, whole)
            if key not in cache:
                cache[key] = cpu_baseline(cfg, rows, CPU_HEADLINE_S if whole else 0.0)
            cb = cache[key]
            if cb:
                if whole:
                    cpu_ms = cb["ms_per_call"]
                    sample = f"{cb['calls']} whole calls of this workload in {cb['ms'] / 1e3:.1f} s"
                else:
                    cpu_ms = cb["deq_ms"] + cb["ms_per_row"] * res["M"]  # decode the weights once, then M rows
                    sample = f"{cb['rows']} row(s) of M in {cb['ms']:.0f} ms, scaled to M rows"
                res["cpu"] = {"ms_per_call": cpu_ms, "sample": sample, "node": cb.get("node"),
                              "cpu_model": cb.get("cpu"), "host_cores": cb.get("host_cores")}
                res["x_vs_cpu"] = round(cpu_ms / res["ms_per_call"], 1)
                log(f"cpu {res['name']}: {cpu_ms:.1f} ms/call ({sample}) -> x{res['x_vs_cpu']}")
    head = results.get("decode1") or next(iter(results.values()))
    cpu = head.get("cpu")
    line = {
        "metric": "q4/q8 GEMM TFLOP/s + HBM GB/s (% roofline) at M=1 and M=4096; x vs CPU ref",
        "value": head["gbps"], "unit": "GB/s", "n_gpus": 1, "steps": head["calls"], "warmup": a.warmup,
        "ms_per_step": head["ms_per_call"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4 weights (u4 codes -> fp16), fp16 activations, fp32 accumulate", "data": "synthetic (seeded PCG64)",
        "config": ({"workload": head["name"], "M": head["M"], "N": 28672, "K": 4096, "enc": "q4g32a.t64", "epi": "swiglu",
                    "weight_copies_rotated": head.get("weight_copies")} if head is results.get("decode1") else
                   {"workload": head["name"], "M": head["M"], "desc": head["desc"],
                    "weight_copies_rotated": head.get("weight_copies")}),
        "roofline": (dict(head["roofline"], traffic=live_traffic["bytes"], traffic_source="rocprofv3 FETCH_SIZE + "
                          "WRITE_SIZE of the headline kernel in this run, scaled by a 1 GiB copy's counts")
                     if live_traffic and head is results.get("decode1") else
                     dict(head["roofline"], traffic_source="counters of the last profiled build (TRAFFIC_KIB)")),
        "traffic_counters": live_traffic if head is results.get("decode1") else None,
        "cpu_baseline": ({"value": round(head["algo_bytes"] / (cpu["ms_per_call"] * 1e6), 3), "unit": "GB/s",
                          "cores": cores, "kind": "port",
                          "sample": f"{cpu['sample']}; oracle/cpu_ref.mjs on Node {cpu['node']}, one thread of "
                                    f"{cpu['host_cores']} host cores ({cpu['cpu_model']})"} if cpu else None),
        "measured_ceiling": ({"what": "plain streaming read of the headline's weight bytes, same launch shape and "
                                      "timing (p0kprobe_stream_read)", "ms_per_call": results["hbm_ceiling"]["ms_per_call"],
                              "gbps": results["hbm_ceiling"]["gbps"],
                              "headline_vs_ceiling": round(results["hbm_ceiling"]["ms_per_call"] / head["ms_per_call"], 4)}
                             if "hbm_ceiling" in results and head is results.get("decode1") else None),
        "measured_mfma_ceiling": mceil,
        "device": info["name"],
        "workloads": list(results.values()),
        "wall_ms_per_step": round(head["wall_ms_per_call"], 5),
        "timing": {"events": "HIP events on the library's stream around the timed calls (plain launches, enqueued "
                             "behind a gate kernel so they run back to back)", "gate": head["gate"],
                   "wall": "host clock from the gate's launch to the end of the synchronisation after the last call, "
                           "per call (includes the gate and the warmup calls)"},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
