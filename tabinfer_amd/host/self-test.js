'use strict';
// selfTestKernels (models/qwen3.js:2753-3219, exported at :5529-5534): every launcher of the
// decode path on small deterministic inputs against an f64 restatement here, as
// [{name, ok, err}] with err the max abs error relative to the result's max (or 0/1 for
// index and distribution checks) and ok = err < tol (1e-3 unless stated).
//
// The int4 weights come from quantizeInt4Bf16 on the GPU and are read back, and so are
// the int8 activations quantQ8 / rmsnormQ leave in the engine's _dp4 scratch and the KV
// rows kvQuantWrite stores; the references dequantize what the kernels consumed. The
// quantizers themselves are checked as round trips (within half a step of the input).
const { f32ToF16 } = require('./ti-engine');

// f16 bits -> value (exact)
function h2f(h) {
  const s = h & 0x8000 ? -1 : 1, e = (h >>> 10) & 31, m = h & 1023;
  if (e === 0) return s * m * Math.pow(2, -24);
  if (e === 31) return m ? NaN : s * Infinity;
  return s * (1 + m / 1024) * Math.pow(2, e - 15);
}

function selfTestKernels(engine) {
  const { E, L } = engine;
  const TI = E.TI, ctx = E.ctx;
  const out = [];
  const check = (name, err, tol) => out.push({ name, ok: err < (tol || 1e-3), err });
  const bufs = [];
  const f32buf = (a) => { const b = E.createBuffer(a.length * 4); E.writeBuffer(b, 0, Float32Array.from(a)); bufs.push(b); return b; };
  const f16buf = (a) => { const b = E.createBuffer(a.length * 2); E.writeBuffer(b, 0, Uint16Array.from(a, f32ToF16)); bufs.push(b); return b; };
  const u32buf = (a) => { const b = E.createBuffer(a.length * 4); E.writeBuffer(b, 0, Uint32Array.from(a)); bufs.push(b); return b; };
  const zbuf = (bytes) => { const b = E.createBuffer(bytes); E.fillU32(b, 0, Math.ceil(bytes / 4)); bufs.push(b); return b; };
  const rd32 = (b, n) => E.readF32(b, n);
  const rdu = (b, n) => E.readU32Range(b, 0, n);
  const rd16 = (b, n) => new Uint16Array(E.readBytes(b, 0, n * 2));
  const relErr = (got, want) => {
    let m = 1e-30, e = 0;
    for (let i = 0; i < want.length; i++) { m = Math.max(m, Math.abs(want[i])); e = Math.max(e, Math.abs(got[i] - want[i])); }
    return e / m;
  };
  const r16 = (a) => Array.from(a, (v) => h2f(f32ToF16(v)));   // values as the f16 buffers hold them
  const dp4 = engine._dp4;
  const int8At = (words, k) => { const b = (words[k >> 2] >>> (8 * (k & 3))) & 0xff; return b > 127 ? b - 256 : b; };
  const actQ8 = (K) => {                               // what quantQ8 / rmsnormQ left: codes x scales
    const xq = rdu(dp4.xq, K / 4), xs = rd32(dp4.xs, K / 32);
    return Array.from({ length: K }, (_, k) => int8At(xq, k) * xs[k >> 5]);
  };
  // a GPU-quantized int4 matrix and its dequantized values
  const int4 = (N, K, seed) => {
    const bf = new Uint16Array(N * K), f = new Float32Array(1), u = new Uint32Array(f.buffer);
    const src = new Float32Array(N * K);
    for (let i = 0; i < N * K; i++) { f[0] = 0.05 * Math.sin(i * 0.37 + seed) * Math.cos(i * 0.011 * seed); bf[i] = u[0] >>> 16; u[0] = bf[i] << 16; src[i] = f[0]; }
    const stage = E.createBuffer(N * K * 2); bufs.push(stage);
    E.writeBuffer(stage, 0, bf);
    const rec = { pack: zbuf(N * K / 2), scales: zbuf(N * K / 16), N, K };
    TI.quant_int4_bf16(ctx, stage, rec.pack, rec.scales, N, K);
    const pk = rdu(rec.pack, N * K / 8), sc = rd16(rec.scales, N * K / 32);
    const W = new Float64Array(N * K);
    for (let n = 0; n < N; n++) for (let k = 0; k < K; k++) {
      const nib = ((pk[n * K / 8 + (k >> 3)] >>> (4 * (k & 7))) & 15) - 8;
      W[n * K + k] = nib * h2f(sc[n * K / 32 + (k >> 5)]);
    }
    return { rec, W, src, sc };
  };
  const mv = (W, x, N, K) => Array.from({ length: N }, (_, n) => { let s = 0; for (let k = 0; k < K; k++) s += W[n * K + k] * x[k]; return s; });
  const silu = (g) => g / (1 + Math.exp(-g));

  try {
    // --- rmsnorm (f32 out) and rmsnormQ (fused norm + int8 quantize, decode) ---
    {
      const T = 3, H = 512, eps = 1e-6;
      const x = Array.from({ length: T * H }, (_, i) => Math.sin(i * 0.07)), w = Array.from({ length: H }, (_, i) => 0.5 + 0.5 * Math.cos(i * 0.03));
      const wr = r16(w), y = zbuf(T * H * 4);
      L.rmsnorm(f32buf(x), f16buf(w), y, T, H, eps);
      const want = [];
      for (let t = 0; t < T; t++) {
        let ss = 0; for (let i = 0; i < H; i++) ss += x[t * H + i] ** 2;
        const inv = 1 / Math.sqrt(ss / H + eps);
        for (let i = 0; i < H; i++) want.push(x[t * H + i] * inv * wr[i]);
      }
      check('rmsnorm', relErr(rd32(y, T * H), want), 1e-5);
      L.rmsnormQ(f32buf(x.slice(0, H)), f16buf(w), H, eps);
      check('rmsnormQ', relErr(actQ8(H), want.slice(0, H)), 2e-2);   // int8 per group: 1/254 of the group max
    }
    // --- quantizeInt4Bf16 round trip, gemvDP4A (int4 x int8), gemvQ (int4 x f32) ---
    {
      const N = 96, K = 256;
      const { rec, W, src, sc } = int4(N, K, 3);
      let worst = 0;
      for (let i = 0; i < N * K; i++) worst = Math.max(worst, Math.abs(W[i] - src[i]) / Math.max(h2f(sc[i >> 5]), 1e-30));
      // within half a step of its group, plus the f16 rounding of the step (|q| <= 8: 8 * 2^-11)
      check('quantizeInt4Bf16 round trip', worst, 0.5 + 8 / 2048 + 1e-4);
      const x = Array.from({ length: K }, (_, i) => Math.cos(i * 0.13) * 2);
      const xb = f32buf(x), y = zbuf(N * 4);
      L.quantQ8(xb, K);
      const xa = actQ8(K);
      check('quantQ8 round trip', relErr(xa, x), 1 / 250);
      L.gemvDP4_only(rec.pack, rec.scales, y, N, K, false);
      check('gemvDP4A', relErr(rd32(y, N), mv(W, xa, N, K)));
      L.gemvQ(xb, rec.pack, rec.scales, y, N, K, false);
      check('gemvQ', relErr(rd32(y, N), mv(W, x, N, K)));
      // gate/up + SiLU on the same activation
      const u = int4(N, K, 5), sw = zbuf(N * 4);
      L.quantQ8(xb, K);
      L.gateUpSiluDP4_only(rec, u.rec, sw, N, K);
      const g = mv(W, xa, N, K), up = mv(u.W, xa, N, K);
      check('gateUpSiluQ', relErr(rd32(sw, N), g.map((v, i) => silu(v) * up[i])));
      // linearQ, T = 5 tokens (the batched path quantizes each token's row itself)
      const T = 5, xs = Array.from({ length: T * K }, (_, i) => Math.sin(i * 0.21));
      const yt = zbuf(T * N * 4);
      L.linearQ(f32buf(xs), rec, yt, T, N, K, false);
      const want = [];
      for (let t = 0; t < T; t++) for (const v of mv(W, xs.slice(t * K, (t + 1) * K), N, K)) want.push(v);
      check('gemmDP4A (linearQ, T = 5)', relErr(rd32(yt, T * N), want), 2e-2);
    }
    // --- embedGather, swiglu ---
    {
      const V = 50, H = 64, emb = Array.from({ length: V * H }, (_, i) => Math.sin(i * 0.3));
      const er = r16(emb), ids = [3, 0, 49, 7], y = zbuf(ids.length * H * 4);
      L.embedGather(u32buf(ids), { buf: f16buf(emb), vocab: V }, y, ids.length, H, 0);
      check('embedGather', relErr(rd32(y, ids.length * H), [].concat(...ids.map((id) => er.slice(id * H, (id + 1) * H)))), 1e-7);
      const n = 300, g = Array.from({ length: n }, (_, i) => 3 * Math.sin(i * 0.1)), u = Array.from({ length: n }, (_, i) => Math.cos(i * 0.2)), sy = zbuf(n * 4);
      engine.Moe.swiglu(f32buf(g), f32buf(u), sy, n);
      check('swiglu', relErr(rd32(sy, n), g.map((v, i) => silu(v) * u[i])), 1e-5);
    }
    // --- ropeQK (per-head RMSNorm + split-half RoPE), kvQuantWrite round trip, attention ---
    {
      const nHq = 4, nKv = 2, hd = 64, T = 3, pos0 = 5, theta = 1e6, eps = 1e-6;
      const x = Array.from({ length: T * nHq * hd }, (_, i) => Math.sin(i * 0.05) + 0.3 * Math.cos(i * 0.7));
      const w = Array.from({ length: hd }, (_, i) => 1 + 0.1 * Math.sin(i)), wr = r16(w), y = zbuf(x.length * 4);
      L.ropeQK(f32buf(x), f16buf(w), y, T, nHq, hd, pos0, theta, eps);
      const want = [];
      for (let t = 0; t < T; t++) for (let h = 0; h < nHq; h++) {
        const r = x.slice((t * nHq + h) * hd, (t * nHq + h + 1) * hd);
        let ss = 0; for (const v of r) ss += v * v;
        const inv = 1 / Math.sqrt(ss / hd + eps), nr = r.map((v, i) => v * inv * wr[i]);
        for (let i = 0; i < hd; i++) {
          const j = i % (hd / 2), a = (pos0 + t) * Math.pow(theta, -2 * j / hd);
          want.push(i < hd / 2 ? nr[i] * Math.cos(a) - nr[i + hd / 2] * Math.sin(a) : nr[i] * Math.cos(a) + nr[i - hd / 2] * Math.sin(a));
        }
      }
      check('ropeQK', relErr(rd32(y, x.length), want), 1e-5);

      const S = 300, row = nKv * hd;
      const kv = { kq: zbuf(S * row), ks: zbuf(S * row / 8), vq: zbuf(S * row), vs: zbuf(S * row / 8) };
      const K = Array.from({ length: S * row }, (_, i) => Math.sin(i * 0.013) * (1 + (i % 7))), Vv = Array.from({ length: S * row }, (_, i) => Math.cos(i * 0.029));
      L.kvQuantWrite(f32buf(K), f32buf(Vv), kv, S, nKv, hd, 0);
      const kq = rdu(kv.kq, S * row / 4), ks = rd32(kv.ks, S * row / 32), vq = rdu(kv.vq, S * row / 4), vs = rd32(kv.vs, S * row / 32);
      const Kd = Array.from({ length: S * row }, (_, i) => int8At(kq, i) * ks[i >> 5] / 127);
      const Vd = Array.from({ length: S * row }, (_, i) => int8At(vq, i) * vs[i >> 5] / 127);
      check('kvQuantWrite round trip', Math.max(relErr(Kd, K), relErr(Vd, Vv)), 1 / 200);
      const attend = (q, npos) => {         // q [nHq][hd] against positions [0, npos)
        const o = [];
        for (let h = 0; h < nHq; h++) {
          const g = Math.floor(h / (nHq / nKv)), sc = [];
          for (let p = 0; p < npos; p++) { let d = 0; for (let i = 0; i < hd; i++) d += q[h * hd + i] * Kd[p * row + g * hd + i]; sc.push(d / Math.sqrt(hd)); }
          const mx = Math.max(...sc), e = sc.map((v) => Math.exp(v - mx)), z = e.reduce((a, b) => a + b, 0);
          for (let i = 0; i < hd; i++) { let s = 0; for (let p = 0; p < npos; p++) s += e[p] * Vd[p * row + g * hd + i]; o.push(s / z); }
        }
        return o;
      };
      const q = Array.from({ length: nHq * hd }, (_, i) => 2 * Math.sin(i * 0.41));
      const o = zbuf(nHq * hd * 4);
      L.attnDecodeStreamQ8(f32buf(q), kv.kq, kv.ks, kv.vq, kv.vs, o, S, nHq, nKv, hd, 0);
      check('attnQ8 decode (GPU-quantized KV)', relErr(rd32(o, nHq * hd), attend(q, S)));
      L.attnDecodeStreamQ8(f32buf(q), kv.kq, kv.ks, kv.vq, kv.vs, o, 5, nHq, nKv, hd, 16);   // more splits than keys
      check('attnDecodeStream (empty split)', relErr(rd32(o, nHq * hd), attend(q, 5)));
      const Tq = 6, p0 = 40, qs = Array.from({ length: Tq * nHq * hd }, (_, i) => Math.cos(i * 0.17)), oc = zbuf(Tq * nHq * hd * 4);
      L.attnCausalQ8(f32buf(qs), kv, oc, Tq, p0, nHq, nKv, hd);
      const wc = [];
      for (let t = 0; t < Tq; t++) for (const v of attend(qs.slice(t * nHq * hd, (t + 1) * nHq * hd), p0 + t + 1)) wc.push(v);
      check('attnQ8 prefill (GPU-quantized KV)', relErr(rd32(oc, Tq * nHq * hd), wc));
    }
    // --- argmax: one stage, two stages (N >= 16384) with the reference's tie order ---
    {
      const ob = zbuf(16);
      const amax = (vals) => { L.argmaxKernel(f32buf(vals), ob, vals.length, 0); return rdu(ob, 1)[0]; };
      const a1 = Array.from({ length: 1000 }, (_, i) => Math.sin(i * 1.3)); a1[777] = 5;
      check('argmax', amax(a1) === 777 ? 0 : 1);
      const a2 = new Array(20000).fill(-1); a2[300] = 3; a2[16394] = 3;   // (i >> 8) & 63: slot 1 for 300, slot 0 for 16394
      check('argmax 2-stage (tie order)', amax(a2) === 16394 ? 0 : 1);
    }
    // --- Gumbel-max sampling: frequencies follow softmax(logits / T) (the reference's test) ---
    {
      const N = 1024, base = new Array(N).fill(-100); base[5] = 2; base[9] = 1;
      const ab = f32buf(base), ob = zbuf(16);
      let seed = 0x9E3779B9 >>> 0, c5 = 0, c9 = 0, other = 0;
      const draw = (t) => {
        seed = (Math.imul(seed, 1664525) + 1013904223) >>> 0;
        E.writeBuffer(ab, 0, Float32Array.from(base));
        TI.gumbel_noise(ctx, ab, N, seed, t);
        L.argmaxKernel(ab, ob, N, 0);
        return rdu(ob, 1)[0];
      };
      for (let i = 0; i < 240; i++) { const v = draw(1.0); if (v === 5) c5++; else if (v === 9) c9++; else other++; }
      const ratio = c5 / Math.max(1, c9);
      check('gumbel T=1 distribution', other === 0 && ratio > 1.6 && ratio < 4.6 ? 0 : 1);
      let det = 0;
      for (let i = 0; i < 10; i++) if (draw(0.02) === 5) det++;
      check('gumbel T→0 ≈ greedy', det === 10 ? 0 : 1);
    }
  } finally {
    E.sync();
    for (const b of bufs) E.destroy(b);
  }
  return out;
}

module.exports = { selfTestKernels };
