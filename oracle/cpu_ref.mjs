// cpu_ref.mjs — JavaScript restatement of the reference's CPU path for the `gemm` op. TEST INFRASTRUCTURE ONLY: the
// timed CPU baseline of bench.py and a second CPU implementation the tests compare with the C oracle.
//
// It restates, in plain ES2019 (Node 12 runs it): the FORMAT.md weight decoders (the dequantised weights the test
// suite's encoders hand to cpuGemm, src/convert/encode.js:68,85), the reference's CPU GEMM (test/kernels.test.js:29:
// a triple loop accumulating in float64) and conv3 loop (:52-65), and the prologue / epilogue formulas of
// src/ops/gemm.js (:60-95, :191-254), rounding to fp16 where the reference kernel does.
//
//   node cpu_ref.mjs check <dir>            spec.json + *.bin in <dir> -> writes <dir>/y_js.bin
//   node cpu_ref.mjs bench <config> <rows>  times the CPU path on a row sample of a BASELINE config -> one JSON line
import fs from 'fs';
import os from 'os';
import path from 'path';

// ------------------------------------------------------------------ fp16 (src/core/gpu.js:276-297)
const F = Math.fround;
const _f = new Float32Array(1), _u = new Uint32Array(_f.buffer);
export function f2h(v) {
  _f[0] = v; const x = _u[0];
  const sign = (x >>> 16) & 0x8000, ex = (x >>> 23) & 0xff; let man = x & 0x7fffff;
  if (ex === 0xff) return sign | 0x7c00 | (man ? 0x200 : 0);
  const e = ex - 112;
  if (e >= 31) return sign | 0x7c00;
  if (e <= 0) {
    if (e < -10) return sign;
    man |= 0x800000; const sh = 14 - e, keep = man >>> sh, rem = man & ((1 << sh) - 1), half = 1 << (sh - 1);
    return sign | (keep + ((rem > half || (rem === half && (keep & 1))) ? 1 : 0));
  }
  const base = sign | (e << 10) | (man >>> 13), rem = man & 0x1fff;
  return base + ((rem > 0x1000 || (rem === 0x1000 && (base & 1))) ? 1 : 0);
}
const H2F = new Float32Array(65536);
for (let h = 0; h < 65536; h++) {
  const s = (h & 0x8000) ? -1 : 1, e = (h >>> 10) & 0x1f, m = h & 0x3ff;
  H2F[h] = e === 0 ? s * m * 5.960464477539063e-8 : e === 31 ? (m ? NaN : s * Infinity) : s * (1 + m / 1024) * Math.pow(2, e - 15);
}
export const h2f = (h) => H2F[h];
const rf16 = (v) => H2F[f2h(v)];

// ------------------------------------------------------------------ weights (docs/FORMAT.md)
const ENC = { 1: 'q4', 2: 'q8', 3: 'f16' };
/** the dequantised weights W(r, kc), kc in [k0, k0 + K), into out[o ..]: the fp32 values the test suite's encoders
 *  hand to cpuGemm (src/convert/encode.js:68,85: F(q*s + mn), F(q*s)); fp16 weights as stored */
function weightRow(enc, w, dv, wG, r, k0, K, out, o) {
  if (enc === 'q4') {
    for (let k = 0; k < K; k += 32) {
      const kc = k0 + k, rec = ((r >>> 6) * wG + (kc >>> 5)) * 1280, rr = r & 63;
      const sm = dv.getUint32(rec + 1024 + rr * 4, true), s = H2F[sm & 0xffff], mn = H2F[sm >>> 16];
      for (let j = 0; j < 16; j++) {
        const b = w[rec + rr * 16 + j];
        out[o + k + 2 * j] = F(F((b & 15) * s) + mn);
        out[o + k + 2 * j + 1] = F(F((b >>> 4) * s) + mn);
      }
    }
  } else if (enc === 'q8') {
    for (let k = 0; k < K; k += 32) {
      const kc = k0 + k, rec = ((r >>> 6) * wG + (kc >>> 6)) * 4224, rr = r & 63, hf = (kc >>> 5) & 1;
      const s = H2F[dv.getUint16(rec + 4096 + rr * 2, true)];
      for (let i = 0; i < 32; i++) out[o + k + i] = F(((w[rec + rr * 64 + hf * 32 + i] << 24) >> 24) * s);
    }
  } else {
    for (let k = 0; k < K; k++) out[o + k] = H2F[dv.getUint16((r * wG + k0 + k) * 2, true)];
  }
}

// ------------------------------------------------------------------ one gemm call, rows [m0, m1) (src/ops/gemm.js)
/** a: the argument object (numbers); b: {name: Uint8Array}; the output buffer b[a.y.buf] is written in place */
export function gemmRows(a, b, m0, m1, pre) {
  const enc = ENC[a.w_enc], M = a.M, N = a.N, K = a.K, epi = a.epi;
  const ldx = a.x_ld || K, ldy = a.y_ld || N, kx0 = a.x_k0 || 0;
  const w = b.w, wdv = new DataView(w.buffer, w.byteOffset, w.byteLength);
  const wG = enc === 'q4' ? a.w_cols / 32 : enc === 'q8' ? a.w_cols / 64 : (a.w_ld || a.w_cols);
  const view = (n, T) => (b[n] ? new T(b[n].buffer, b[n].byteOffset, b[n].byteLength / T.BYTES_PER_ELEMENT) : null);
  const X16 = view('x', Uint16Array), X32 = view('x', Float32Array), ST = view('st', Float32Array), PV = view('pv', Float32Array);
  const EV = view('ev', Float32Array), BV = view('bv', Float32Array), RP = view('rope', Float32Array), GT = view('gt', Uint16Array);
  const Y16 = view('y', Uint16Array), Y32 = view('y', Float32Array);
  const glu = epi === 3, rowOf = (n) => glu ? ((n & 1) ? a.wr1 : a.wr0) + (n >>> 1) : Math.min(a.wr0 + n, a.w_rows - 1);
  // dequantised weights of the call, once (the test suite decodes before cpuGemm)
  let Wd = pre;
  if (!Wd) { Wd = new Float32Array(N * K); for (let n = 0; n < N; n++) weightRow(enc, w, wdv, wG, rowOf(n), a.wk0 || 0, K, Wd, n * K); }
  const xr = new Float32Array(K), acc = new Float64Array(N);
  const silu = (z) => z / (1 + Math.exp(-z));
  for (let m = m0; m < m1; m++) {
    // prologue
    if (a.x_mode === 0) for (let k = 0; k < K; k++) xr[k] = H2F[X16[m * ldx + kx0 + k]];
    else if (a.x_mode === 2) { const r = ST[(a.st_off + m) * 2 + 1]; for (let k = 0; k < K; k++) xr[k] = rf16(F(F(X32[m * ldx + kx0 + k] * r) * PV[a.pv_off + kx0 + k])); }
    else if (a.x_mode === 1) {
      const mu = ST[(a.st_off + m) * 2], r = ST[(a.st_off + m) * 2 + 1];
      for (let k = 0; k < K; k++) xr[k] = rf16(F(F(F(F(X32[m * ldx + kx0 + k] - mu) * r) * F(1 + PV[a.pv_off + kx0 + k])) + PV[a.pv_off + a.pv_stride + kx0 + k]));
    } else if (a.x_mode === 4) {
      const Ci = a.c_Ci, HW = a.c_Ho * a.c_Wo, ot = Math.floor(m / HW), rem = m % HW, oy = Math.floor(rem / a.c_Wo), ox = rem % a.c_Wo;
      const T = a.c_stride || 1, ks = a.c_ks || 1;
      for (let k = 0; k < K; k++) {
        const tap = Math.floor(k / Ci), c = k % Ci, kt = Math.floor(tap / 9), ky = Math.floor(tap / 3) % 3, kx = tap % 3;
        const itg = Math.min(T - 1, Math.max(0, ot + a.c_padT + kt - 1)), it = ks > 1 ? itg % ks : itg - a.c_padL;
        const iy = oy + ky - 1, ix = ox + kx - 1;
        if (iy < 0 || ix < 0 || iy >= a.c_Hi || ix >= a.c_Wi) { xr[k] = 0; continue; }
        const vox = (it * a.c_Hi + iy) * a.c_Wi + ix;
        let v = H2F[X16[vox * Ci + c]];
        if (a.c_pn) v = rf16(silu(F(v * ST[vox])));
        xr[k] = v;
      }
    } else throw new Error('cpu_ref: x mode ' + a.x_mode + ' not restated here');
    // the test suite's cpuGemm row: float64 sums
    for (let n = 0; n < N; n++) { let s = 0; const o = n * K; for (let k = 0; k < K; k++) s += xr[k] * Wd[o + k]; acc[n] = s; }
    // epilogue
    const yr = m * ldy + (a.y_n0 || 0);
    if (epi === 0) for (let n = 0; n < N; n++) Y16[yr + n] = f2h(acc[n]);
    else if (epi === 1) for (let n = 0; n < N; n++) Y32[yr + n] = acc[n];
    else if (epi === 2) for (let n = 0; n < N; n++) {
      const g = EV ? EV[a.ev_off + n] : 1, bb = BV ? BV[a.bv_off + n] : 0;
      Y32[yr + n] = (a.store ? 0 : Y32[yr + n]) + g * (acc[n] + bb);
    } else if (epi === 5) for (let n = 0; n < N; n++) Y16[yr + n] = f2h(acc[n] + EV[a.ev_off + n] + (a.res ? H2F[Y16[yr + n]] : 0));
    else if (epi === 3) for (let o = 0; o < N / 2; o++) {
      let g = acc[2 * o], u = acc[2 * o + 1];
      if (BV) { g += BV[a.bv_off + o]; u += BV[a.bv_off + a.bv_up + o]; }
      const act = a.act === 1 ? g * 0.5 * (1 + Math.tanh(Math.max(-15, Math.min(15, 0.7978845608 * (g + 0.044715 * g * g * g))))) : silu(g);
      Y16[yr + o] = f2h(act * u);
    } else if (epi === 4) {
      const row = a.h_rowOff + m, eps = a.h_eps || 1e-6, v = new Float64Array(128);
      for (let hd = 0; hd < N / 128; hd++) {
        for (let d = 0; d < 128; d++) v[d] = acc[hd * 128 + d];
        const sec = hd < a.h_Hq ? 0 : hd < a.h_Hq + a.h_Hkv ? 1 : 2;
        if (sec < 2) {
          let ss = 0; for (let d = 0; d < 128; d++) ss += v[d] * v[d];
          const inv = 1 / Math.sqrt(ss / 128 + eps), nw = a.ev_off + (sec ? 128 : 0), rp = row * 128;
          for (let d = 0; d < 128; d++) v[d] *= inv * EV[nw + d];
          if (a.h_rope_mode === 1) for (let d = 0; d < 64; d++) {
            const c = RP[rp + 2 * d], s = RP[rp + 2 * d + 1], lo = v[d], hi = v[d + 64];
            v[d] = lo * c - hi * s; v[d + 64] = hi * c + lo * s;
          } else for (let p = 0; p < 64; p++) {
            const c = RP[rp + 2 * p], s = RP[rp + 2 * p + 1], x0 = v[2 * p], x1 = v[2 * p + 1];
            v[2 * p] = x0 * c - x1 * s; v[2 * p + 1] = x0 * s + x1 * c;
          }
        }
        const ob = (hd * a.h_Ltot + row) * 128;
        for (let d = 0; d < 128; d++) Y16[ob + d] = f2h(v[d]);
      }
    } else if (epi === 6) {
      const eps = a.h_eps || 1e-6;
      for (let nb = 0; nb < N; nb += 128) {
        let ss = 0; for (let d = 0; d < 128; d++) ss += acc[nb + d] * acc[nb + d];
        const inv = 1 / Math.sqrt(ss / 128 + eps);
        for (let d = 0; d < 128; d++) Y16[yr + nb + d] = f2h(acc[nb + d] * inv * EV[a.ev_off + d] / (1 + Math.exp(-H2F[GT[m * a.h_Ltot + (a.y_n0 || 0) + nb + d]])));
      }
    }
  }
  return Wd;
}

// ------------------------------------------------------------------ synthetic inputs for the timed sample
function xorshift(seed) { let s = seed >>> 0 || 1; return () => { s ^= s << 13; s >>>= 0; s ^= s >>> 17; s ^= s << 5; s >>>= 0; return s; }; }
function randnF16(n, seed) {
  const r = xorshift(seed), o = new Uint16Array(n);
  for (let i = 0; i < n; i += 2) {
    const u = Math.max(1e-9, r() / 4294967296), v = r() / 4294967296, m = Math.sqrt(-2 * Math.log(u));
    o[i] = f2h(m * Math.cos(2 * Math.PI * v)); if (i + 1 < n) o[i + 1] = f2h(m * Math.sin(2 * Math.PI * v));
  }
  return o;
}
/** q4 / q8 records with random codes and scale words of N(0, 0.02) weights (the decode work does not depend on them) */
function records(enc, rows, K, seed) {
  const r = xorshift(seed);
  if (enc === 'q4') {
    const u = new Uint32Array((rows / 64) * (K / 32) * 320);
    for (let i = 0; i < u.length; i++) u[i] = r();
    for (let t = 0; t < u.length / 320; t++) for (let j = 0; j < 64; j++) u[t * 320 + 256 + j] = f2h(0.0055 + (r() & 255) * 1e-6) | (f2h(-0.045 - (r() & 255) * 1e-5) << 16);
    return new Uint8Array(u.buffer);
  }
  const b = new Uint8Array((rows / 64) * (K / 64) * 4224);
  for (let i = 0; i < b.length; i += 4) { const v = r(); b[i] = v; b[i + 1] = v >>> 8; b[i + 2] = v >>> 16; b[i + 3] = v >>> 24; }
  const dv = new DataView(b.buffer);
  for (let t = 0; t < b.length / 4224; t++) for (let j = 0; j < 64; j++) dv.setUint16(t * 4224 + 4096 + 2 * j, f2h(0.0004 + (r() & 255) * 1e-7), true);
  return b;
}
const bytesOf = (a) => new Uint8Array(a.buffer, a.byteOffset, a.byteLength);

const CONFIGS = {   // BASELINE.json configs, as (args, buffers) for the given number of rows
  decode: (M) => { const K = 4096, rows = 28672;
    return [{ w_enc: 1, w_rows: rows, w_cols: K, wr0: 0, wr1: rows / 2, x_mode: 0, M, N: rows, K, epi: 3, act: 0 },
      { w: records('q4', rows, K, 1), x: bytesOf(randnF16(M * K, 2)), y: new Uint8Array(M * rows) }]; },
  prefill: (M) => { const K = 4096, N = 4096, x = new Float32Array(M * K), st = new Float32Array(M * 2), g = new Float32Array(K);
    const xh = randnF16(M * K, 3); for (let i = 0; i < x.length; i++) x[i] = H2F[xh[i]];
    for (let m = 0; m < M; m++) { let q = 0; for (let k = 0; k < K; k++) q += x[m * K + k] * x[m * K + k]; st[2 * m + 1] = 1 / Math.sqrt(q / K + 1e-6); }
    for (let k = 0; k < K; k++) g[k] = 1 + 0.1 * H2F[randnF16(1, 100 + k)[0]];
    const R = new Float32Array(M * N); const rh = randnF16(M * N, 4); for (let i = 0; i < R.length; i++) R[i] = H2F[rh[i]];
    return [{ w_enc: 2, w_rows: N, w_cols: K, wr0: 0, x_mode: 2, st_off: 0, pv_off: 0, M, N, K, epi: 2 },
      { w: records('q8', N, K, 5), x: bytesOf(x), st: bytesOf(st), pv: bytesOf(g), y: bytesOf(R) }]; },
  dit_qkv: (M) => { const K = 3072, N = 9216, x = new Float32Array(M * K), st = new Float32Array(M * 2), pv = new Float32Array(2 * K);
    const xh = randnF16(M * K, 6); for (let i = 0; i < x.length; i++) x[i] = H2F[xh[i]];
    for (let m = 0; m < M; m++) { let s = 0, q = 0; for (let k = 0; k < K; k++) s += x[m * K + k]; const mu = s / K; for (let k = 0; k < K; k++) q += (x[m * K + k] - mu) ** 2; st[2 * m] = mu; st[2 * m + 1] = 1 / Math.sqrt(q / K + 1e-6); }
    const ph = randnF16(2 * K, 7); for (let i = 0; i < pv.length; i++) pv[i] = 0.5 * H2F[ph[i]];
    const ev = new Float32Array(256).fill(1), rp = new Float32Array(M * 128);
    for (let t = 0; t < M; t++) for (let p = 0; p < 64; p++) { const a = (p < 32 ? Math.floor(t / 64) : t % 64) * Math.pow(1e4, -(p % 32) / 32); rp[t * 128 + 2 * p] = Math.cos(a); rp[t * 128 + 2 * p + 1] = Math.sin(a); }
    return [{ w_enc: 1, w_rows: N, w_cols: K, wr0: 0, x_mode: 1, st_off: 0, pv_off: 0, pv_stride: K, ev_off: 0, M, N, K, epi: 4,
      h_Ltot: M, h_Hq: 24, h_Hkv: 24, h_rowOff: 0, h_eps: 1e-6, h_rope_mode: 0 },
      { w: records('q4', N, K, 8), x: bytesOf(x), st: bytesOf(st), pv: bytesOf(pv), ev: bytesOf(ev), rope: bytesOf(rp), y: new Uint8Array(N * M * 2) }]; },
  dit_up: (M) => { const K = 3072, rows = 24576;
    return [{ w_enc: 1, w_rows: rows, w_cols: K, wr0: 0, wr1: rows / 2, x_mode: 0, M, N: rows, K, epi: 3, act: 1 },
      { w: records('q4', rows, K, 9), x: bytesOf(randnF16(M * K, 10)), y: new Uint8Array(M * rows) }]; },
  conv3: (M) => { const T = 13, H = 92, W = 160, C = 128, N = 128, K = 27 * C;
    return [{ w_enc: 3, w_rows: N, w_cols: K, wr0: 0, x_mode: 4, M, N, K, epi: 0, c_Hi: H, c_Wi: W, c_Ci: C, c_Ho: H, c_Wo: W, c_stride: T, c_padT: 0, c_padL: 0, c_ks: 1 },
      { w: bytesOf(randnF16(N * K, 11).map((h) => f2h(0.02 * H2F[h]))), x: bytesOf(randnF16(T * H * W * C, 12)), y: new Uint8Array(M * N * 2) }]; },
};

function bench(config, rows, targetS) {
  const [a, b] = CONFIGS[config](rows);
  const t0 = process.hrtime.bigint();
  const Wd = gemmRows(a, b, 0, 1);                       // the weights are decoded once per call, then row 0
  const t1 = process.hrtime.bigint();
  gemmRows(a, b, 1, rows, Wd);
  const t2 = process.hrtime.bigint();
  // decode time = first row minus one plain row (measured on the other rows, or a second pass of row 0)
  let rowMs;
  if (rows > 1) rowMs = Number(t2 - t1) / 1e6 / (rows - 1);
  else { const t3 = process.hrtime.bigint(); gemmRows(a, b, 0, 1, Wd); rowMs = Number(process.hrtime.bigint() - t3) / 1e6; }
  const firstMs = Number(t1 - t0) / 1e6;
  // whole calls (decode + every row) repeated until targetS seconds have passed: the timed sample
  let calls = 1, totalMs = firstMs + Number(t2 - t1) / 1e6;
  const t4 = process.hrtime.bigint();
  while (targetS > 0 && Number(process.hrtime.bigint() - t4) / 1e9 + totalMs / 1e3 < targetS) {
    const d = gemmRows(a, b, 0, 1);
    gemmRows(a, b, 1, rows, d);
    calls++;
  }
  if (calls > 1) totalMs += Number(process.hrtime.bigint() - t4) / 1e6;
  const cpus = os.cpus();
  console.log(JSON.stringify({ config, rows, ms: totalMs, calls, ms_per_call: totalMs / calls, deq_ms: Math.max(0, firstMs - rowMs),
    ms_per_row: rowMs, node: process.version, cpu: cpus.length ? cpus[0].model : '?', host_cores: cpus.length }));
}

function check(dir) {
  const a = JSON.parse(fs.readFileSync(path.join(dir, 'spec.json'), 'utf8'));
  const b = {};
  for (const f of fs.readdirSync(dir)) if (f.endsWith('.bin')) b[f.slice(0, -4)] = new Uint8Array(fs.readFileSync(path.join(dir, f)));
  gemmRows(a, b, 0, a.M);
  fs.writeFileSync(path.join(dir, 'y_js.bin'), b.y);
}

if (process.argv[2] === 'bench') bench(process.argv[3], parseInt(process.argv[4] || '1', 10), parseFloat(process.argv[5] || '0'));
else if (process.argv[2] === 'check') check(process.argv[3]);
