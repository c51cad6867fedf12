// p0pc0rn-kernels_amd/node/index.mjs — the reference's JavaScript API for the GEMM path, on MI355X through libp0k.
//
// A caller of the reference (src/index.js) imports these names from here instead and keeps its code:
//   createGpu / Gpu (src/core/gpu.js:15, :30)      buffer, upload, read, free, done, poolStats, drainPool, freeAll, describe
//   gemm(gpu, args) (src/ops/gemm.js:268)          same argument object, same synchronous argument errors, returns 2MNK
//   rowstats(gpu, args) (src/ops/misc.js:37)       mean / rstd per row, the statistics the rms and lnmod prologues read
//   attention(gpu, args) (src/ops/attention.js:168) head size 128, the consumer of the heads epilogue
//   pixstats (src/ops/video.js:317), gnPartBytes / gnPartial / gnFinalize / groupnormStats (src/ops/misc.js:92-109)
//   defaultTune / calibrate / tuneEntry / TUNE_TABLE (src/core/tune.js:18-58)
//   loadWeights / uploadWeights (src/weights.js:10, :28)
//   f2h / h2f / toF16 / fromF16 (src/core/gpu.js:276-299), packQ4 / packQ8 / packF16 (src/convert/encode.js:56-98)
//
// Differences a caller can see: buffers are plain objects {_ptr (BigInt device address), _pf (size), label} instead of
// GPUBuffer; gemm runs on a HIP stream in call order rather than in a WebGPU batch, so the reference's watchdog-driven
// dispatch splitting does not exist; read() resolves to an ArrayBuffer copy like the reference's.
// Runs on Node 12.17+ (N-API 6). No dependencies besides the addon p0k.node beside this file.
'use strict';
import { createRequire } from 'module';
import { readFileSync } from 'fs';
import { join } from 'path';
import { fileURLToPath } from 'url';

const require = createRequire(import.meta.url);
let native = null;
function addon() {
  if (!native) {
    try {
      native = require('./p0k.node');
    } catch (e) {
      throw new GpuError('p0k.node is not built (python p0pc0rn-kernels_amd/build.py addon): ' + e.message);
    }
  }
  return native;
}

const MB = 1e6;
class GpuError extends Error {}

// errors from libp0k: argument errors (P0K_E1, P0K_E4) are plain Errors like the reference's throw new Error(...);
// HIP and allocation failures are GpuErrors like the reference's device errors.
function rethrow(e) {
  if (e && (e.code === 'P0K_E2' || e.code === 'P0K_E3')) {
    const g = new GpuError(e.message);
    g.code = e.code;
    throw g;
  }
  throw e;
}
function call(f, ...args) {
  try {
    return f(...args);
  } catch (e) {
    rethrow(e);
  }
}

/** Create the GPU context. opts: {device=0, maxDispatchSeconds} (the WebGPU options of the reference have no meaning here) */
async function createGpu(opts = {}) {
  const g = new Gpu(opts);
  g.init();
  return g;
}

class Gpu {
  constructor(opts) {
    this.opts = Object.assign({ device: 0, maxDispatchSeconds: 0.2 }, opts || {});
    this.ctx = null;
    this.bufs = new Set();
    this.lostInfo = null;
    this.f16 = true;
    this.subgroups = true;
    this.sgMin = 64;
    this.sgMax = 64;
    this.sgOK16 = true;
    // FLOP/s and bytes/s for an MI355X until calibrate() measures them (the reference sizes dispatches with these)
    this.rate = { mm: 300e12, mm32: 300e12, mm16: 300e12, attn: 100e12, mem: 4e12 };
  }

  init() {
    const A = addon();
    this.ctx = call(A.ctxCreate, this.opts.device | 0);
    const d = call(A.deviceInfo, this.ctx);
    this.info = { vendor: 'amd', architecture: d.arch, device: d.name, description: d.name + ' (' + d.cus + ' CUs)' };
    this.limits = { maxBufferSize: d.hbmBytes, maxStorageBufferBindingSize: d.hbmBytes, maxComputeWorkgroupStorageSize: 163840,
      maxComputeInvocationsPerWorkgroup: 1024, maxComputeWorkgroupSizeX: 1024 };
    this.cus = d.cus;
  }

  get lost() { return !!this.lostInfo; }
  describe() {
    return Object.assign({}, this.info, { f16: true, subgroups: true, sgMin: this.sgMin, sgMax: this.sgMax,
      maxBufferMB: Math.round(this.limits.maxBufferSize / 1048576), maxBindMB: Math.round(this.limits.maxStorageBufferBindingSize / 1048576),
      wgMem: this.limits.maxComputeWorkgroupStorageSize, wgInv: this.limits.maxComputeInvocationsPerWorkgroup });
  }

  _live() {
    if (!this.ctx) throw new GpuError('GPU context destroyed');
  }

  /** a zeroed device buffer of max(16, size rounded up to 16) bytes, reused from the pool when one of that size is free */
  buffer(size, label = '') {
    this._live();
    size = Math.max(16, Math.ceil(size / 16) * 16);
    if (size > this.limits.maxBufferSize) throw new GpuError(`buffer ${label} ${size} B exceeds maxBufferSize`);
    const ptr = call(addon().alloc, this.ctx, size);
    const b = { _ptr: ptr, _pf: size, size, label };
    this.bufs.add(b);
    return b;
  }

  /** return a buffer to the pool (or release it when the pool is full); unknown or freed buffers are ignored */
  free(b) {
    if (!b || !this.bufs.has(b)) return;
    this.bufs.delete(b);
    call(addon().free, this.ctx, b._ptr);
  }

  /** upload a TypedArray / ArrayBuffer into a NEW buffer (or into dst at dstOff) */
  upload(data, label = '', dst = null, dstOff = 0) {
    this._live();
    const u8 = data instanceof ArrayBuffer ? new Uint8Array(data) : new Uint8Array(data.buffer, data.byteOffset, data.byteLength);
    const b = dst || this.buffer(u8.byteLength, label);
    if (u8.byteLength) call(addon().upload, this.ctx, b._ptr, dstOff, u8);
    return b;
  }

  /** read back [off, off+size) of a buffer as an ArrayBuffer (after all work enqueued before it) */
  async read(buf, off = 0, size = null) {
    this._live();
    size = size == null ? buf._pf - off : size;
    return call(addon().download, this.ctx, buf._ptr, off, size);
  }

  /** device-to-device copy on the stream */
  copy(dst, dstOff, src, srcOff, size) {
    call(addon().copy, this.ctx, dst._ptr, dstOff, src._ptr, srcOff, size);
  }

  async done() {
    this._live();
    call(addon().sync, this.ctx);
  }

  drainPool() { call(addon().drainPool, this.ctx); }
  poolStats() {
    const s = call(addon().poolStats, this.ctx);
    return { aliveMB: Math.round(s.alive / 1e6), pooledMB: Math.round(s.pooled / 1e6), bufs: s.buffers, pooledN: s.pooledN,
      creates: s.creates, reuses: s.reuses, evictions: s.evictions, hwMB: Math.round(s.highWater / 1e6),
      capMB: Math.round((s.highWater + s.maxBuf) / 1e6) };
  }
  freeAll() { for (const b of Array.from(this.bufs)) this.free(b); this.drainPool(); }

  /** release every buffer and the context */
  destroy() {
    if (!this.ctx) return;
    addon().ctxDestroy(this.ctx);
    this.ctx = null;
    this.bufs.clear();
  }
}

// ------------------------------------------------------------------ the op
const ENC = { 'q4g32a.t64': 1, 'q8g64s.t64': 2, f16: 3 };
const XMODE = { f16: 0, lnmod: 1, rms: 2, conv: 3, conv3: 4 };
const EPI = { f16: 0, f32: 1, resadd: 2, swiglu: 3, heads: 4, bias: 5, onormgate: 6 };
const ACT = { silu: 0, gelu: 1 };
const ACC = { f32: 0, f16: 1 };
const DEFAULT_TILE = { BM: 64, BN: 128 };

const dflt = (v, d) => (v === undefined || v === null ? d : v);
const sizeOf = (buf) => (buf ? buf._pf || buf.size || 0 : 0);
const ptrOf = (buf) => (buf ? buf._ptr : 0n);

/** the flat libp0k descriptor (struct p0k_gemm_args) of a reference gemm argument object */
function gemmDesc(gpu, a) {
  const w = a.w, x = a.x, y = a.y, cv = a.conv || null, h = a.heads || null;
  const enc = ENC[w.enc];
  if (!enc) throw new Error('gemm: unsupported weight encoding ' + w.enc);
  const encKey = enc === 1 ? 'q4' : enc === 2 ? 'q8' : 'f16';
  const tg = gpu && gpu.tune && gpu.tune.gemm;
  const tile = a.tile || (cv && tg && tg[cv.kind === 'conv3' ? 'conv3' : 'conv']) || (tg && tg[encKey]) || null;
  const d = {
    w_enc: enc, w_buf: ptrOf(w.buf), w_off: w.off || 0, w_bytes: dflt(w.bytes, sizeOf(w.buf) - (w.off || 0)),
    w_rows: w.rows, w_cols: w.cols, w_ld: w.ld || 0,
    x_buf: ptrOf(x.buf), x_off: x.off || 0, x_size: x.size != null ? x.size + (x.off || 0) : sizeOf(x.buf),
    x_ld: x.ld || 0, x_k0: x.k0 || 0, x_mode: cv ? XMODE[cv.kind === 'conv3' ? 'conv3' : 'conv'] : XMODE[x.mode || 'f16'],
    y_buf: ptrOf(y.buf), y_off: y.off || 0, y_size: y.size != null ? y.size + (y.off || 0) : sizeOf(y.buf),
    y_ld: y.ld || 0, y_n0: y.n0 || 0,
    M: a.M, N: a.N, K: a.K,
    epi: EPI[a.epi || 'f16'], acc: ACC[a.acc || (gpu && gpu.tune && gpu.tune.acc) || 'f32'],
    tile_bm: tile ? tile.BM : 0, tile_bn: tile ? tile.BN : 0,
    wr0: a.wr0 || 0, wr1: a.wr1 || 0, wk0: a.wk0 || 0,
    res: a.res ? 1 : 0, store: a.store ? 1 : 0, act: ACT[a.act || 'silu'],
  };
  if (d.x_mode === undefined) throw new Error('gemm: unknown x mode ' + x.mode);
  if (d.epi === undefined) throw new Error('gemm: unknown epilogue ' + a.epi);
  if (d.acc === undefined) throw new Error('gemm: unknown acc ' + a.acc);
  if (d.act === undefined) throw new Error('gemm: unknown act ' + a.act);
  const vec = (v, p) => {
    if (!v) return;
    d[p + '_buf'] = ptrOf(v.buf);
    d[p + '_size'] = sizeOf(v.buf);
    d[p + '_off'] = v.off || 0;
  };
  vec(a.ev, 'ev');
  vec(a.stats, 'st');
  vec(a.pv, 'pv');
  vec(a.bv, 'bv');
  if (a.pv) d.pv_stride = a.pv.stride || 0;
  if (a.bv) d.bv_up = a.bv.up || 0;
  if (a.gt) { d.gt_buf = ptrOf(a.gt.buf); d.gt_size = sizeOf(a.gt.buf); }
  if (h) {
    d.h_Ltot = h.Ltot || 0; d.h_Hq = h.Hq || 0; d.h_Hkv = h.Hkv || 0; d.h_rowOff = h.rowOff || 0;
    d.h_eps = h.eps || 0; d.h_rope_mode = h.ropeMode === 'half' ? 1 : 0;
    if (h.rope) { d.rope_buf = ptrOf(h.rope.buf); d.rope_size = sizeOf(h.rope.buf); }
  }
  if (cv) {
    d.c_Hi = cv.Hi || 0; d.c_Wi = cv.Wi || 0; d.c_Ci = cv.Ci || 0; d.c_Ho = cv.Ho || 0; d.c_Wo = cv.Wo || 0;
    d.c_stride = dflt(cv.stride, 1); d.c_padT = cv.padT || 0; d.c_padL = cv.padL || 0; d.c_ks = dflt(cv.ks, 1);
    d.c_up2 = cv.up2 ? 1 : 0; d.c_gn = cv.gn ? 1 : 0; d.c_pn = cv.pn ? 1 : 0;
  }
  return d;
}

/** y = x · Wᵀ with the fused prologue / epilogue the arguments name; enqueued on the stream; returns 2MNK */
function gemm(gpu, a) {
  const d = gemmDesc(gpu, a);
  return call(addon().gemm, gpu.ctx, d);
}

/** the kernel and tile libp0k runs for these arguments on this gpu's device ({kernel: 'gemv'|'gemv_short'|'gemv_mfma'|
 *  'mfma_dma'|'mfma', BM, BN}); checks them like gemm does */
function gemmPlan(gpu, a) {
  return call(addon().selectTile, gemmDesc(gpu, a), gpu ? gpu.ctx : undefined);
}

/** per-row statistics of an f16 / f32 matrix: ST[(st.off+r)*2] = mean (mode 'ln') or 0 (mode 'rms'), ST[..+1] = rstd */
function rowstats(gpu, a) {
  const x = a.x, st = a.st;
  call(addon().rowstats, gpu.ctx, {
    x_buf: ptrOf(x.buf), x_off: x.off || 0, x_size: sizeOf(x.buf), ld: x.ld || a.cols, c0: x.c0 || 0,
    rows: a.rows, cols: a.cols, mode: a.mode === 'rms' ? 1 : 0, eps: a.eps,
    st_buf: ptrOf(st.buf), st_off: st.off || 0, st_size: sizeOf(st.buf),
  });
}

// ------------------------------------------------------------------ attention (src/ops/attention.js:168), head size 128
/** attention(gpu, {q, k, v: {buf, off}, o: {buf, off, ld}, Lq, Lk, Hq, Hkv, mode, nvalid, scale, cap}) -> 4 Lq Lk 128 Hq */
function attention(gpu, a) {
  const t = (x) => ({ buf: ptrOf(x.buf), off: x.off || 0, size: x.size != null ? x.size + (x.off || 0) : sizeOf(x.buf) });
  const q = t(a.q), k = t(a.k), v = t(a.v), o = t(a.o);
  return call(addon().attention, gpu.ctx, { q_buf: q.buf, q_off: q.off, q_size: q.size, k_buf: k.buf, k_off: k.off,
    k_size: k.size, v_buf: v.buf, v_off: v.off, v_size: v.size, o_buf: o.buf, o_off: o.off, o_size: o.size,
    ldo: a.o.ld || 0, Lq: a.Lq, Lk: a.Lk || 0, Hq: a.Hq, Hkv: a.Hkv || 0, mode: a.mode || 0, nvalid: a.nvalid || 0,
    scale: a.scale || 0, cap: a.cap || 0 });
}

// ------------------------------------------------------------------ conv prologue statistics (src/ops/video.js, misc.js)
/** pixstats(gpu, {x: {buf, off}, r: {buf}, V, C, eps = 1e-8, ro}): r[ro + v] = 1 / sqrt(mean_c x[v][c]^2 + eps) */
function pixstats(gpu, a) {
  call(addon().pixstats, gpu.ctx, { x_buf: ptrOf(a.x.buf), x_off: a.x.off || 0, x_size: sizeOf(a.x.buf), V: a.V, C: a.C,
    eps: a.eps || 0, r_buf: ptrOf(a.r.buf), ro: a.ro || 0, r_size: sizeOf(a.r.buf) });
}

/** bytes of the GroupNorm partial rows of pix pixels */
function gnPartBytes(pix) { return Math.ceil(pix / 64) * 512; }

function gnDesc(a) {
  const d = { pix: a.pix || 0, C: a.C, part_buf: ptrOf(a.part), part_size: sizeOf(a.part), wg_off: a.wgOff || 0,
    nwg: a.nwg || 0, eps: a.eps || 0 };
  if (a.x) Object.assign(d, { x_buf: ptrOf(a.x.buf), x_off: a.x.off || 0, x_size: a.x.size != null ? a.x.size + (a.x.off || 0) : sizeOf(a.x.buf) });
  if (a.gb) Object.assign(d, { gb_buf: ptrOf(a.gb.buf), g_off: a.gb.gOff || 0, b_off: a.gb.bOff || 0, gb_size: sizeOf(a.gb.buf) });
  if (a.ab) Object.assign(d, { ab_buf: ptrOf(a.ab.buf), ab_off: a.ab.off || 0, ab_size: sizeOf(a.ab.buf) });
  return d;
}
/** gnPartial(gpu, {x, pix, C, part, wgOff}) -> rows written (ceil(pix / 64)) */
function gnPartial(gpu, a) { return call(addon().gn, gpu.ctx, gnDesc(a), 1); }
/** gnFinalize(gpu, {part, nwg, C, gb: {buf, gOff, bOff}, ab: {buf, off}, eps = 1e-6}) */
function gnFinalize(gpu, a) { call(addon().gn, gpu.ctx, gnDesc(a), 2); }
/** groupnormStats(gpu, {x, pix, C, part, gb, ab, eps}) */
function groupnormStats(gpu, a) { call(addon().gn, gpu.ctx, gnDesc(a), 3); }

// ------------------------------------------------------------------ tune (src/core/tune.js)
/** per-device tile / accumulation choices; matched against gpu.info like the reference's table */
const TUNE_TABLE = [
  { match: { vendor: 'amd', architecture: 'gfx950' }, tune: {},
    source: 'MI355X: libp0k picks its own CDNA4 kernel and tile per call (streaming GEMV for M <= 16, load-to-LDS MFMA GEMM with 128/256 x 128/256 tiles above); the tile only matters for range checks' },
];

function tuneEntry(g, table = TUNE_TABLE) {
  const info = g.info || {};
  return table.find((e) => Object.entries(e.match || {}).every(([k, v]) => String(info[k] || '').toLowerCase().includes(String(v).toLowerCase()))) || null;
}

/** gpu.tune = {acc (default 'f16', as the reference's engines use), gemm: per-encoding tiles} */
function defaultTune(g, o = {}) {
  const t = (tuneEntry(g, o.table) || {}).tune || {};
  g.tune = { acc: o.acc || t.acc || 'f16', vaeAcc: o.vaeAcc || 'f16' };
  if (o.gemm || t.gemm) g.tune.gemm = Object.assign({}, t.gemm, o.gemm);
  return g.tune;
}

/** measure GEMM throughput (q4, M=1024 N=3072 K=3072, both accumulation modes) and attention throughput (8 heads of
 *  128, 1024 x 1024); sets gpu.rate (mm32, mm16, mm, attn) and gpu.calib, as src/core/tune.js:39-58 does */
async function calibrate(g) {
  const M = 1024, N = 3072, K = 3072, L = 1024, H = 8;
  const recs = (N / 64) * (K / 32), u = new Uint32Array(recs * 320);
  let s = 0x9e3779b9 | 0;
  const next = () => { s = (Math.imul(s, 1664525) + 1013904223) | 0; return s >>> 0; };
  for (let r = 0; r < recs; r++) {
    for (let j = 0; j < 256; j++) u[r * 320 + j] = next();
    for (let j = 0; j < 64; j++) u[r * 320 + 256 + j] = 0x2000 | ((0xa800 | (j & 0x3f)) << 16);   // scale 2^-11, min -2^-6-ish
  }
  const h16 = (n) => { const h = new Uint16Array(n); for (let i = 0; i < n; i++) h[i] = (next() & 0x83ff) | 0x3400; return h; };
  const W = g.upload(u), X = g.upload(h16(M * K)), Y = g.buffer(M * N * 2);
  const Q = g.upload(h16(H * L * 128)), O = g.buffer(L * H * 256);
  const time = async (fn, reps) => { fn(); await g.done(); const t0 = process.hrtime.bigint(); for (let i = 0; i < reps; i++) fn(); await g.done(); return Number(process.hrtime.bigint() - t0) / 1e9 / reps; };
  try {
    const mm = (acc) => time(() => gemm(g, { w: { buf: W, off: 0, bytes: W._pf, enc: 'q4g32a.t64', rows: N, cols: K }, x: { buf: X }, M, N, K, epi: 'f16', y: { buf: Y }, acc }), 20);
    const t32 = await mm('f32'), t16 = await mm('f16');
    g.rate.mm32 = 0.8 * (2 * M * N * K) / t32;
    g.rate.mm16 = 0.8 * (2 * M * N * K) / t16;
    g.rate.mm = Math.min(g.rate.mm32, g.rate.mm16);
    const ta = await time(() => attention(g, { q: { buf: Q }, k: { buf: Q }, v: { buf: Q }, o: { buf: O }, Lq: L, Lk: L, Hq: H, Hkv: H, mode: 0 }), 20);
    g.rate.attn = 0.8 * (4 * L * L * 128 * H) / ta;
    g.calib = { gemmF32Gflops: Math.round(2 * M * N * K / t32 / 1e9), gemmF16Gflops: Math.round(2 * M * N * K / t16 / 1e9),
      attnGflops: Math.round(4 * L * L * 128 * H / ta / 1e9) };
  } finally {
    [W, X, Y, Q, O].forEach((b) => g.free(b));
  }
  return g.calib;
}

// ------------------------------------------------------------------ weights (src/weights.js)
const MANIFEST_FORMAT = 'p0pc0rn-kernels.weights/1';

/** base: a folder path (or file: URL) holding manifest.json and its shards; opts: {fetch(name) -> Uint8Array | Promise, onProgress} */
async function loadWeights(gpu, base, opts = {}) {
  const dir = String(base).startsWith('file:') ? fileURLToPath(base) : String(base);
  const get = opts.fetch || ((f) => readFileSync(join(dir, f)));
  const asBytes = (v) => (v instanceof Uint8Array ? v : new Uint8Array(v));
  const manifest = JSON.parse(Buffer.from(asBytes(await get('manifest.json'))).toString('utf8'));
  if (manifest.format !== MANIFEST_FORMAT) throw new Error('not a converted model (format ' + manifest.format + ')');
  const total = manifest.shards.reduce((a, sh) => a + sh.bytes, 0), bufs = {};
  let done = 0;
  try {
    for (const sh of manifest.shards) {
      const data = asBytes(await get(sh.file));
      if (data.byteLength !== sh.bytes) throw new Error(`${sh.file}: ${data.byteLength} bytes, the manifest says ${sh.bytes}`);
      bufs[sh.file] = gpu.upload(data, sh.file);
      done += sh.bytes;
      if (opts.onProgress) opts.onProgress(done, total);
    }
  } catch (e) {
    for (const b of Object.values(bufs)) gpu.free(b);
    throw e;
  }
  return modelOf(manifest, bufs, gpu);
}

/** the same from shards already in memory ({file: Uint8Array}) */
function uploadWeights(gpu, manifest, shards) {
  if (manifest.format !== MANIFEST_FORMAT) throw new Error('not a converted model (format ' + manifest.format + ')');
  const bufs = {};
  for (const sh of manifest.shards) bufs[sh.file] = gpu.upload(shards[sh.file], sh.file);
  return modelOf(manifest, bufs, gpu);
}

function modelOf(manifest, bufs, gpu) {
  const entry = (name) => {
    const t = manifest.tensors[name];
    if (!t) throw new Error('no tensor ' + name);
    return t;
  };
  return {
    manifest,
    names: () => Object.keys(manifest.tensors),
    /** gemm's `w`: {enc, buf, off, bytes, rows, cols, shape, layout} */
    tensor(name) {
      const t = entry(name);
      return { enc: t.enc, buf: bufs[t.file], off: t.offset, bytes: t.bytes, rows: t.rows, cols: t.cols, shape: t.shape, layout: t.layout };
    },
    /** an fp32 vector as the ops take it: {buf, off} with off counted in floats */
    vector(name) {
      const t = entry(name);
      if (t.enc !== 'f32') throw new Error(name + ' is ' + t.enc + ', not f32');
      return { buf: bufs[t.file], off: t.offset / 4 };
    },
    free() { for (const b of Object.values(bufs)) gpu.free(b); },
  };
}

// ------------------------------------------------------------------ fp16 helpers (host)
const f32v = new Float32Array(1), u32v = new Uint32Array(f32v.buffer);

/** a number → binary16 bits, round to nearest even. The value is first rounded to binary32 (as a Float32Array store
 *  does), so a float64 input rounds twice, the same as the reference's helper. */
function f2h(v) {
  f32v[0] = v;
  const b = u32v[0], sign = (b >>> 16) & 0x8000, exp = (b >>> 23) & 0xff, man = b & 0x7fffff;
  if (exp === 0xff) return sign | 0x7c00 | (man ? 0x200 : 0);
  const e = exp - 127 + 15;                      // biased binary16 exponent
  if (e >= 31) return sign | 0x7c00;
  if (e <= 0) {                                  // binary16 subnormal (or zero): value = full / 2^(14 - e) in units of 2^-24
    if (e < -10) return sign;
    const full = man | 0x800000, shift = 14 - e;
    const q = full >>> shift, r = full - q * 2 ** shift, halfway = 2 ** (shift - 1);
    return sign | (q + (r > halfway || (r === halfway && (q & 1)) ? 1 : 0));
  }
  const h = sign | (e << 10) | (man >>> 13), r = man & 0x1fff;
  return h + (r > 0x1000 || (r === 0x1000 && (h & 1)) ? 1 : 0);   // a carry into the exponent (or to infinity) is correct
}

/** binary16 bits → number (exact) */
function h2f(h) {
  const neg = h & 0x8000, e = (h >>> 10) & 0x1f, m = h & 0x3ff;
  let v;
  if (e === 0) v = m * 2 ** -24;
  else if (e === 31) return m ? NaN : neg ? -Infinity : Infinity;
  else v = (1024 + m) * 2 ** (e - 25);
  return neg ? -v : v;
}

function toF16(a) { const o = new Uint16Array(a.length); for (let i = 0; i < a.length; i++) o[i] = f2h(a[i]); return o; }
function fromF16(u) { const o = new Float32Array(u.length); for (let i = 0; i < u.length; i++) o[i] = h2f(u[i]); return o; }

// ------------------------------------------------------------------ encoders (host, in libp0k)
const asF32 = (W) => (W instanceof Float32Array ? W : Float32Array.from(W));
/** W [rows][K] fp32 → q4g32a.t64 bytes; deq (optional Float32Array) receives the decoded values */
function packQ4(W, rows, K, deq = null) { return call(addon().packQ4, asF32(W), rows, K, deq); }
/** W [rows][K] fp32 → q8g64s.t64 bytes */
function packQ8(W, rows, K, deq = null) { return call(addon().packQ8, asF32(W), rows, K, deq); }
/** fp32 → fp16 bits */
function packF16(W) { return call(addon().packF16, asF32(W)); }
/** bytes of a rows × cols tensor in an encoding ('q4g32a.t64' | 'q8g64s.t64' | 'f16') */
function encodedBytes(enc, rows, cols) {
  if (!ENC[enc]) throw new Error('unknown encoding ' + enc);
  return addon().tensorBytes(ENC[enc], rows, cols);
}

// ------------------------------------------------------------------ converter helpers (src/convert/encode.js)
// What loadWeights callers use to produce the manifest tensors: raw safetensors bytes -> fp32, the matrix view of a
// tensor (convolution weights reordered so each output channel's row is the implicit GEMM's K vector, the OHWI /
// OTHWI layouts the conv / conv3 prologues read), the encoding rule, and the row encoders.
const DTYPE_BYTES = { F32: 4, F16: 2, BF16: 2, F8_E4M3: 1, F8_E5M2: 1 };
function dtypeBytes(dt) {
  if (!DTYPE_BYTES[dt]) throw new Error('unsupported dtype ' + dt + ' (F32, F16, BF16, F8_E4M3, F8_E5M2)');
  return DTYPE_BYTES[dt];
}
/** the 256 values of an 8-bit float: e4m3 (bias 7, no infinities, 0x7f / 0xff NaN) or e5m2 (bias 15, IEEE-style) */
function fp8Values(e4m3) {
  const mb = e4m3 ? 3 : 2, bias = e4m3 ? 7 : 15, out = new Float32Array(256);
  for (let b = 0; b < 256; b++) {
    const sign = b & 0x80 ? -1 : 1, e = (b & 0x7f) >> mb, m = b & ((1 << mb) - 1), emax = e4m3 ? 15 : 31;
    if (e4m3 && e === emax && m === (1 << mb) - 1) out[b] = NaN;
    else if (!e4m3 && e === emax) out[b] = m ? NaN : sign * Infinity;
    else if (e === 0) out[b] = sign * m * 2 ** (1 - bias - mb);
    else out[b] = sign * ((1 << mb) + m) * 2 ** (e - bias - mb);
  }
  return out;
}
const FP8 = {};
/** raw tensor bytes of a safetensors dtype -> Float32Array */
function toFloat32(dtype, bytes) {
  const u8 = bytes instanceof Uint8Array ? bytes : new Uint8Array(bytes), n = u8.byteLength / dtypeBytes(dtype);
  const out = new Float32Array(n);
  if (dtype === 'F32') { new Uint8Array(out.buffer).set(u8); return out; }
  if (dtype === 'F8_E4M3' || dtype === 'F8_E5M2') {
    const t = FP8[dtype] || (FP8[dtype] = fp8Values(dtype === 'F8_E4M3'));
    for (let i = 0; i < n; i++) out[i] = t[u8[i]];
    return out;
  }
  const h = new Uint16Array(n);
  new Uint8Array(h.buffer).set(u8);
  if (dtype === 'BF16') { const w = new Uint32Array(out.buffer); for (let i = 0; i < n; i++) w[i] = h[i] << 16; return out; }
  for (let i = 0; i < n; i++) out[i] = h2f(h[i]);
  return out;
}
/** {header, dataStart} of a safetensors file from its first bytes (8-byte length + JSON header) */
function safetensorsHeader(bytes) {
  const u8 = bytes instanceof Uint8Array ? bytes : new Uint8Array(bytes);
  const n = Number(new DataView(u8.buffer, u8.byteOffset, u8.byteLength).getBigUint64(0, true));
  if (n > 100e6 || 8 + n > u8.byteLength) throw new Error('safetensors: bad or truncated header');
  return { header: JSON.parse(Buffer.from(u8.subarray(8, 8 + n)).toString('utf8')), dataStart: 8 + n };
}
/** the tensors of a header in file order: [{name, dtype, shape, begin, end}] (offsets from the data start) */
function safetensorsList(header) {
  const out = [];
  for (const [name, t] of Object.entries(header)) {
    if (name === '__metadata__') continue;
    out.push({ name, dtype: t.dtype, shape: t.shape, begin: t.data_offsets[0], end: t.data_offsets[1] });
  }
  return out.sort((a, b) => a.begin - b.begin);
}
/** the matrix a tensor is stored as: 2-D as is; [O, I, kh, kw] -> OHWI rows; [O, I, kt, kh, kw] -> OTHWI rows; vectors;
 *  other ranks flatten their leading dimensions */
function matrixOf(shape) {
  const prod = (a) => a.reduce((x, y) => x * y, 1);
  if (shape.length === 4) return { rows: shape[0], cols: prod(shape.slice(1)), layout: 'OHWI' };
  if (shape.length === 5) return { rows: shape[0], cols: prod(shape.slice(1)), layout: 'OTHWI' };
  if (shape.length <= 1) return { rows: 1, cols: shape.length ? shape[0] : 1, layout: 'vector' };
  return { rows: prod(shape.slice(0, -1)), cols: shape[shape.length - 1], layout: 'row-major' };
}
/** convolution weight rows from the framework's OIHW / OITHW order (input channel outer, tap inner) to the kernels'
 *  OHWI / OTHWI order (tap outer, input channel inner); returns a new Float32Array */
function reorderConvRows(W, rows, shape) {
  const I = shape[1], taps = shape.slice(2).reduce((x, y) => x * y, 1), K = I * taps, out = new Float32Array(rows * K);
  for (let r = 0; r < rows; r++) {
    const o = r * K;
    for (let i = 0; i < I; i++) for (let t = 0; t < taps; t++) out[o + t * I + i] = W[o + i * taps + t];
  }
  return out;
}
/** the encoding a tensor gets: f32 for vectors (and names matching opts.f32), f16 for names matching opts.keep or
 *  bits 16, q4 / q8 for matrices whose rows and columns fit the record tiles (bits 4 or 8), f16 otherwise */
function chooseEncoding(name, shape, opts = {}) {
  const bits = opts.bits || 4, m = matrixOf(shape);
  if (opts.f32 && opts.f32.test(name)) return 'f32';
  if (m.layout === 'vector') return 'f32';
  if ((opts.keep && opts.keep.test(name)) || bits === 16) return 'f16';
  if (bits === 4 && m.rows % 64 === 0 && m.cols % 32 === 0) return 'q4g32a.t64';
  if ((bits === 4 || bits === 8) && m.rows % 64 === 0 && m.cols % 64 === 0) return 'q8g64s.t64';
  return 'f16';
}
/** fp32 bytes of W */
function packF32(W) { return new Uint8Array(Float32Array.from(W).buffer); }
/** bytes of one 64-row tile of K columns in an encoding */
function tileBytes(enc, K) {
  if (enc === 'q4g32a.t64') return (K / 32) * 1280;
  if (enc === 'q8g64s.t64') return (K / 64) * 4224;
  return 64 * K * (enc === 'f16' ? 2 : 4);
}
/** rows x K fp32 values in an encoding (rows a multiple of 64 for q4 / q8) -> Uint8Array */
function encodeRows(enc, W, rows, K) {
  const w = asF32(W);
  if (enc === 'q4g32a.t64') return packQ4(w, rows, K);
  if (enc === 'q8g64s.t64') return packQ8(w, rows, K);
  if (enc === 'f16') return packF16(w.subarray(0, rows * K));
  if (enc === 'f32') return packF32(w.subarray(0, rows * K));
  throw new Error('unknown encoding ' + enc);
}

export {
  MB, GpuError, createGpu, Gpu, f2h, h2f, toF16, fromF16,
  gemm, gemmPlan, gemmDesc, DEFAULT_TILE, rowstats, attention, pixstats, gnPartBytes, gnPartial, gnFinalize, groupnormStats,
  TUNE_TABLE, tuneEntry, defaultTune, calibrate,
  MANIFEST_FORMAT, loadWeights, uploadWeights,
  packQ4, packQ8, packF16, packF32, encodedBytes, tileBytes, encodeRows,
  dtypeBytes, toFloat32, safetensorsHeader, safetensorsList, matrixOf, reorderConvRows, chooseEncoding,
};
