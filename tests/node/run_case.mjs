// Driver for the Node shim tests (tests/test_node_shim.py): exercises p0pc0rn-kernels_amd/node/index.mjs the way a caller
// of the reference's JavaScript API would.
//   run_case.mjs host <dir>   no GPU: fp16 helpers, encoders, argument errors; writes results into <dir>
//   run_case.mjs gemm <dir>   GPU: spec.json (a reference gemm argument object with buffer NAMES) + <name>.bin buffers;
//                             createGpu → upload → gemm → read → <out>_gpu.bin
//   run_case.mjs weights <dir> GPU: loadWeights on a converted-model folder, then gemm with model.tensor(...)
//   run_case.mjs stats <dir>  GPU: pixstats and groupnormStats
//   run_case.mjs convert <dir> no GPU: the converter helpers (toFloat32, safetensors header, matrixOf, chooseEncoding,
//                             reorderConvRows, encodeRows, tileBytes) on inputs written by the test
//   run_case.mjs calibrate <dir> GPU: calibrate() -> gpu.rate / gpu.calib
'use strict';
import { readFileSync, writeFileSync } from 'fs';
import { join } from 'path';
import * as p0k from '../../p0pc0rn-kernels_amd/node/index.mjs';

const [mode, dir] = process.argv.slice(2);
const bin = (n) => { const b = readFileSync(join(dir, n)); return new Uint8Array(b.buffer, b.byteOffset, b.byteLength); };
const put = (n, a) => writeFileSync(join(dir, n), Buffer.from(a.buffer, a.byteOffset, a.byteLength));

function errorOf(fn) {
  try { fn(); return null; } catch (e) { return { message: e.message, gpuError: e instanceof p0k.GpuError }; }
}

async function host() {
  const v = new Float32Array(bin('values.f32').slice().buffer);
  put('f2h.u16', p0k.toF16(v));
  const h = new Uint16Array(65536); for (let i = 0; i < 65536; i++) h[i] = i;
  put('h2f.f32', p0k.fromF16(h));
  const f64 = JSON.parse(readFileSync(join(dir, 'f64.json'), 'utf8'));
  writeFileSync(join(dir, 'f2h64.json'), JSON.stringify(f64.map(p0k.f2h)));
  const w = JSON.parse(readFileSync(join(dir, 'pack.json'), 'utf8'));
  const W = new Float32Array(bin('W.f32').slice().buffer);
  put('q4.bin', p0k.packQ4(W, w.rows, w.K));
  put('q8.bin', p0k.packQ8(W, w.rows, w.K));
  put('f16.bin', p0k.packF16(W));
  const deq = new Float32Array(w.rows * w.K); p0k.packQ4(W, w.rows, w.K, deq); put('q4deq.f32', deq);
  const fake = (n) => ({ _ptr: 1n << 40n, _pf: n });   // never dereferenced: gemmPlan only checks
  const base = () => ({ w: { enc: 'q4g32a.t64', buf: fake(1 << 20), off: 0, bytes: 1 << 20, rows: 128, cols: 256 },
    x: { buf: fake(1 << 20) }, y: { buf: fake(1 << 20) }, M: 4, N: 128, K: 256 });
  const cases = {
    encoding: (a) => { a.w.enc = 'q5'; },
    kmul32: (a) => { a.K = 48; },
    tile: (a) => { a.tile = { BM: 48, BN: 128 }; },
    rms_stats: (a) => { a.x.mode = 'rms'; },
    conv3_ci: (a) => { a.conv = { kind: 'conv3', Hi: 4, Wi: 4, Ci: 48, Ho: 4, Wo: 4, stride: 2, ks: 3 }; },
  };
  const errs = {};
  for (const [k, f] of Object.entries(cases)) { const a = base(); f(a); errs[k] = errorOf(() => p0k.gemmPlan(null, a)); }
  errs.ok = errorOf(() => p0k.gemmPlan(null, base()));
  errs.plan = p0k.gemmPlan(null, base());
  errs.bytes = [p0k.encodedBytes('q4g32a.t64', 128, 256), p0k.encodedBytes('q8g64s.t64', 128, 256), p0k.encodedBytes('f16', 128, 256)];
  writeFileSync(join(dir, 'errors.json'), JSON.stringify(errs));
}

async function gemmCase() {
  const spec = JSON.parse(readFileSync(join(dir, 'spec.json'), 'utf8'));
  const names = JSON.parse(readFileSync(join(dir, 'bufs.json'), 'utf8'));
  const g = await p0k.createGpu();
  if (spec.tune) p0k.defaultTune(g, spec.tune);
  const bufs = {};
  for (const n of names) bufs[n] = g.upload(bin(n + '.bin'), n);
  const sub = (v) => {
    if (v && typeof v === 'object' && !Array.isArray(v)) {
      const o = {};
      for (const [k, x] of Object.entries(v)) o[k] = k === 'buf' ? bufs[x] : sub(x);
      return o;
    }
    return v;
  };
  const a = sub(spec.args);
  const flops = p0k.gemm(g, a);
  const out = spec.out;
  const y = await g.read(bufs[out]);
  put(out + '_gpu.bin', new Uint8Array(y));
  const st = g.poolStats();
  for (const b of Object.values(bufs)) g.free(b);
  await g.done();
  writeFileSync(join(dir, 'result.json'), JSON.stringify({ flops, plan: p0k.gemmPlan(g, a), pool: st, info: g.describe() }));
  g.destroy();
}

async function weights() {
  const spec = JSON.parse(readFileSync(join(dir, 'spec.json'), 'utf8'));
  const g = await p0k.createGpu();
  let progress = 0;
  const model = await p0k.loadWeights(g, join(dir, 'model'), { onProgress: (d) => { progress = d; } });
  const x = g.upload(bin('x.bin')), y = g.buffer(spec.M * spec.N * 2);
  p0k.gemm(g, { w: model.tensor(spec.tensor), x: { buf: x }, y: { buf: y }, M: spec.M, N: spec.N, K: spec.K, epi: 'f16' });
  put('y_gpu.bin', new Uint8Array(await g.read(y)));
  const vec = model.vector(spec.vector);
  const v = new Float32Array(await g.read(vec.buf, vec.off * 4, spec.vlen * 4));
  put('v_gpu.f32', v);
  const bad = errorOf(() => model.vector(spec.tensor));
  writeFileSync(join(dir, 'result.json'), JSON.stringify({ progress, names: model.names(), bad }));
  model.free(); g.free(x); g.free(y); await g.done(); g.destroy();
}

async function stats() {
  const spec = JSON.parse(readFileSync(join(dir, 'spec.json'), 'utf8'));
  const g = await p0k.createGpu();
  const x = g.upload(bin('x.bin')), r = g.buffer(spec.V * 4);
  p0k.pixstats(g, { x: { buf: x }, r: { buf: r }, V: spec.V, C: spec.C });
  put('r_gpu.f32', new Float32Array(await g.read(r)));
  const gx = g.upload(bin('gx.bin')), gb = g.upload(bin('gb.bin'));
  const part = g.buffer(p0k.gnPartBytes(spec.pix)), ab = g.buffer(spec.GC * 8);
  p0k.groupnormStats(g, { x: { buf: gx }, pix: spec.pix, C: spec.GC, part, gb: { buf: gb, gOff: 0, bOff: spec.GC * 4 }, ab: { buf: ab } });
  put('ab_gpu.f32', new Float32Array(await g.read(ab)));
  const aq = g.upload(bin('aq.bin')), ak = g.upload(bin('ak.bin')), av = g.upload(bin('av.bin')), ao = g.buffer(spec.L * spec.H * 256);
  const fl = p0k.attention(g, { q: { buf: aq }, k: { buf: ak }, v: { buf: av }, o: { buf: ao }, Lq: spec.L, Hq: spec.H, Hkv: 1, mode: 1, nvalid: spec.L });
  put('ao_gpu.bin', new Uint8Array(await g.read(ao)));
  writeFileSync(join(dir, 'result.json'), JSON.stringify({ attnFlops: fl }));
  [x, r, gx, gb, part, ab, aq, ak, av, ao].forEach((b) => g.free(b));
  await g.done(); g.destroy();
}

async function convert() {
  const spec = JSON.parse(readFileSync(join(dir, 'spec.json'), 'utf8'));
  const res = {};
  for (const [dt, file] of Object.entries(spec.raw)) put('f32_' + dt + '.f32', p0k.toFloat32(dt, bin(file)));
  const st = bin('model.safetensors');
  const { header, dataStart } = p0k.safetensorsHeader(st);
  res.list = p0k.safetensorsList(header);
  res.dataStart = dataStart;
  const conv = res.list.find((t) => t.name === spec.conv);
  const Wc = p0k.toFloat32(conv.dtype, st.subarray(dataStart + conv.begin, dataStart + conv.end));
  const m = p0k.matrixOf(conv.shape);
  res.matrix = m;
  res.enc = p0k.chooseEncoding(conv.name, conv.shape, { bits: 16 });
  const Wr = p0k.reorderConvRows(Wc, m.rows, conv.shape);
  put('conv_reordered.f32', Wr);
  put('conv_f16.bin', p0k.encodeRows(res.enc, Wr, m.rows, m.cols));
  res.matrices = spec.shapes.map((sh) => p0k.matrixOf(sh));
  res.encodings = spec.choose.map(([n, sh, o]) => p0k.chooseEncoding(n, sh, o ? { bits: o.bits, keep: o.keep && new RegExp(o.keep), f32: o.f32 && new RegExp(o.f32) } : {}));
  res.tileBytes = ['q4g32a.t64', 'q8g64s.t64', 'f16', 'f32'].map((e) => p0k.tileBytes(e, 256));
  const W = new Float32Array(bin('W.f32').slice().buffer);
  put('enc_q4.bin', p0k.encodeRows('q4g32a.t64', W, 64, 256));
  put('enc_q8.bin', p0k.encodeRows('q8g64s.t64', W, 64, 256));
  put('enc_f32.bin', p0k.encodeRows('f32', W, 64, 256));
  res.badDtype = errorOf(() => p0k.toFloat32('I64', new Uint8Array(8)));
  res.badEnc = errorOf(() => p0k.encodeRows('q5', W, 64, 256));
  writeFileSync(join(dir, 'result.json'), JSON.stringify(res));
}

async function calibrate() {
  const g = await p0k.createGpu();
  const calib = await p0k.calibrate(g);
  writeFileSync(join(dir, 'result.json'), JSON.stringify({ calib, rate: g.rate }));
  await g.done(); g.destroy();
}

const run = { host, gemm: gemmCase, weights, stats, convert, calibrate }[mode];
run().catch((e) => { console.error(e && e.stack || e); process.exit(1); });
