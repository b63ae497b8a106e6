'use strict';
// ti-engine.js — the engine object and kernel launchers of TabInfer's decode path, over
// the MI355X library (tabinfer.node -> libtabinfer.so).
//
// The reference's launchers are closures inside models/qwen3.js / models/lfm25.js that
// dispatch WGSL pipelines through engine/webgpu-engine.js. Here the launchers keep their
// names, argument order and meaning; GPU buffers are opaque device handles from
// E.createBuffer; an int4 weight record is {pack, scales, N, K} as in
// models/qwen3.js:3508-3514. Shape errors are thrown by the library as JS exceptions.
const path = require('path');

const ADDON = path.join(__dirname, 'tabinfer.node');
let TI;
try {
  TI = require(ADDON);
} catch (e) {
  throw new Error('tabinfer.node is not built (' + ADDON + '): run `python -m tabinfer_amd.build` (' + e.message + ')');
}

const ACT_CAP = 65536;    // widest activation the quantQ8 scratch holds (the library's own limit)

// engine/webgpu-engine.js:217-236: f32 -> f16 bits with the +0x1000 rounding the engine's
// converter uses (scales of the int3 requant).
const _f32 = new Float32Array(1), _u32 = new Uint32Array(_f32.buffer);
function engineF32ToF16(v) {
  _f32[0] = v;
  const x = _u32[0], sign = (x >>> 16) & 0x8000;
  let mant = x & 0x7fffff;
  const exp = (x >>> 23) & 0xff;
  if (exp === 255) return sign | (mant ? 0x7e00 : 0x7c00);
  const e = exp - 127 + 15;
  if (e >= 31) return sign | 0x7c00;
  if (e <= 0) {
    if (e < -10) return sign;
    mant = (mant | 0x800000) >>> (1 - e);
    return sign | ((mant + 0x1000) >>> 13);
  }
  return sign | (e << 10) | ((mant + 0x1000) >>> 13);
}

// models/qwen3.js:3357-3374: f32 -> f16 bits, the half-up rounding of the qwen3 loader
// (norms, embeddings).
function f32ToF16(v) {
  _f32[0] = v;
  const x = _u32[0], sign = (x >>> 16) & 0x8000;
  const exp = (x >>> 23) & 0xff, mant = x & 0x7fffff;
  if (exp === 0xff) return sign | (mant ? 0x7e00 : 0x7c00);
  const e = exp - 127 + 15;
  if (e >= 31) return sign | 0x7c00;
  if (e <= 0) {
    if (e < -10) return sign;
    const m = mant | 0x800000, shift = 14 - e;
    let half = m >>> shift;
    if ((m >>> (shift - 1)) & 1) half += 1;
    return sign | half;
  }
  let half = (e << 10) | (mant >>> 13);
  if ((mant >>> 12) & 1) half += 1;
  return sign | half;
}

// bf16 bits -> f16 bits through the exact bf16 -> f32 widening (models/qwen3.js:3386-3391)
function bf16ToF16bits(u16) {
  const out = new Uint16Array(u16.length);
  for (let i = 0; i < u16.length; i++) { _u32[0] = u16[i] << 16; out[i] = f32ToF16(_f32[0]); }
  return out;
}

function createEngine({ device = 0 } = {}) {
  const ctx = TI.init(device);
  const U = (v) => (v == null ? null : v);
  const b01 = (acc) => (acc ? 1 : 0);

  // ---- E: the engine surface the launchers sit on (engine/webgpu-engine.js) ----------
  const E = {
    TI, ctx,
    createBuffer(bytes) { return TI.buf_alloc(ctx, Math.max(4, Math.ceil(bytes))); },
    destroy(buf) { TI.buf_free(buf); },
    view(buf, byteOff, bytes) { return bytes == null ? TI.buf_view(buf, byteOff) : TI.buf_view(buf, byteOff, bytes); },
    bytes(buf) { return TI.buf_bytes(buf); },
    writeBuffer(buf, off, data) { TI.buf_write(ctx, buf, off, data); },
    readBytes(buf, off, bytes) { return TI.buf_read(ctx, buf, off, bytes); },
    readF32(buf, n, off = 0) { return new Float32Array(TI.buf_read(ctx, buf, off, n * 4)); },
    readU32Range(buf, from, n) { return new Uint32Array(TI.buf_read(ctx, buf, from * 4, n * 4)); },
    copyBuffer(src, soff, dst, doff, bytes) { TI.buf_copy(ctx, dst, doff, src, soff, bytes); },
    fillU32(buf, value, count) { TI.buf_fill_u32(ctx, buf, value >>> 0, count); },
    sync() { TI.sync(ctx); },
    drain() { return TI.sync_async(ctx); },
    // E.beginBatch(Infinity) / E.endBatch(): every call in between becomes one replayable graph
    beginBatch() { TI.graph_begin(ctx); },
    endBatch() { return TI.graph_end(ctx); },
    launch(graph) { TI.graph_launch(ctx, graph); },
    destroyGraph(graph) { TI.graph_destroy(graph); },
    mark(slot) { TI.event_record(ctx, slot); },
    elapsedMs(a, b) { return TI.event_elapsed_ms(ctx, a, b); },
    shutdown() { TI.shutdown(ctx); },
  };

  // quantQ8's output lives in engine scratch, as the reference's _dp4 (models/qwen3.js:405-420)
  const _dp4 = { xq: E.createBuffer(ACT_CAP), xs: E.createBuffer(ACT_CAP / 32 * 4), xsum: E.createBuffer(ACT_CAP / 16 * 4) };

  // ---- int4 records -------------------------------------------------------------------------
  function int4Record(N, K) {
    return { pack: E.createBuffer(N * K / 2), scales: E.createBuffer(N * K / 32 * 2), N, K, int4: true };
  }
  // quantizeInt4Bf16 (models/qwen3.js:3405-3426) on the GPU: bf16 rows already on the
  // device -> rec (rows [row0, row0 + rows) of it)
  function quantizeInt4Bf16(bf16Buf, rec, row0 = 0, rows = rec.N) {
    const K = rec.K;
    const pack = row0 ? E.view(rec.pack, row0 * K / 2) : rec.pack;
    const sc = row0 ? E.view(rec.scales, row0 * K / 32 * 2) : rec.scales;
    TI.quant_int4_bf16(ctx, bf16Buf, pack, sc, rows, K);
  }

  // quantizeTernaryBf16 (models/qwen3.js:3435-3469) on the GPU: bf16 rows on the device ->
  // a ternary record {pack, scales, N, K, tern: true}, or null where the tensor is not
  // ternary (the caller then quantizes to int4, as the reference's loader does)
  const _ternFlag = E.createBuffer(4);
  function quantizeTernaryBf16(bf16Buf, N, K) {
    const rec = { pack: E.createBuffer(N * K / 4), scales: E.createBuffer(N * K / 32 * 2), N, K, tern: true };
    E.fillU32(_ternFlag, 0, 1);
    TI.quant_tern_bf16(ctx, bf16Buf, rec.pack, rec.scales, N, K, _ternFlag);
    if (new Uint32Array(E.readBytes(_ternFlag, 0, 4))[0] === 0) return rec;
    E.destroy(rec.pack);
    E.destroy(rec.scales);
    return null;
  }
  // gemvTern_only (:548-556): the ternary GEMV against the activation quantQ8 left in _dp4
  function gemvTern_only(wrec, yBuf, N, K, acc) {
    TI.gemv_tern2(ctx, _dp4.xq, _dp4.xs, _dp4.xsum, wrec.pack, wrec.scales, yBuf, N, K, b01(acc));
  }

  // ---- models/qwen3.js launchers ---------------------------------------------------------------
  const L = {
    quantizeInt4Bf16, int4Record, quantizeTernaryBf16, gemvTern_only,
    // projGemv (:558-561): the kind router of the decode call sites sharing one activation
    projGemv(wrec, yBuf, N, K, acc) {
      if (wrec.tern) return gemvTern_only(wrec, yBuf, N, K, acc);
      return TI.gemv_q4_q8(ctx, _dp4.xq, _dp4.xs, wrec.pack, wrec.scales, yBuf, N, K, b01(acc));
    },
    quantQ8(xBuf, K) { TI.quant_act_q8(ctx, xBuf, _dp4.xq, _dp4.xs, _dp4.xsum, K); },                       // :414
    rmsnormQ(xBuf, wBuf, H, eps) { TI.rmsnorm_q8(ctx, xBuf, wBuf, _dp4.xq, _dp4.xs, _dp4.xsum, H, eps); },  // :614
    rmsnorm(xBuf, wBuf, yBuf, T, H, eps) { TI.rmsnorm(ctx, xBuf, wBuf, yBuf, T, H, eps); },                // :81
    gemvDP4_only(packBuf, scBuf, yBuf, N, K, acc) {                                                        // :422
      TI.gemv_q4_q8(ctx, _dp4.xq, _dp4.xs, packBuf, scBuf, yBuf, N, K, b01(acc));
    },
    gemvQ(xBuf, packBuf, scBuf, yBuf, N, K, acc /* , NR: a WGSL tile knob */) {                           // :314
      TI.gemv_q4_f32(ctx, xBuf, packBuf, scBuf, yBuf, N, K, b01(acc));
    },
    gateUpSiluDP4_only(gRec, uRec, swiBuf, I, H /* , NR */) {                                              // :861
      if (gRec.tern) {                                                                                       // :862-870
        TI.gateup_silu_tern2(ctx, _dp4.xq, _dp4.xs, _dp4.xsum, gRec.pack, gRec.scales, uRec.pack, uRec.scales, swiBuf, I, H);
        return;
      }
      TI.gateup_silu_q4(ctx, _dp4.xq, _dp4.xs, gRec.pack, gRec.scales, uRec.pack, uRec.scales, swiBuf, I, H);
    },
    linearQ(xBuf, wrec, yBuf, T, N, K, acc) {                                                              // :1588
      if (wrec.tern) {        // :1594-1598: quantQ8 + the ternary GEMV, token by token (no ternary GEMM here)
        for (let t = 0; t < T; t++) {
          TI.quant_act_q8(ctx, T > 1 ? E.view(xBuf, t * K * 4) : xBuf, _dp4.xq, _dp4.xs, _dp4.xsum, K);
          gemvTern_only(wrec, T > 1 ? E.view(yBuf, t * N * 4) : yBuf, N, K, acc);
        }
        return;
      }
      TI.linear_q4(ctx, xBuf, wrec.pack, wrec.scales, yBuf, T, N, K, b01(acc));
    },
    attnPrepQ8(qBuf, kBuf, vBuf, qwBuf, kwBuf, qrBuf, kv, nHq, nKv, hd, posBase, theta, eps) {             // :2297
      TI.attn_prep_q8(ctx, qBuf, kBuf, vBuf, qwBuf, kwBuf, qrBuf, kv.kq, kv.ks, kv.vq, kv.vs, nHq, nKv, hd, posBase, theta, eps);
    },
    attnDecodeStreamQ8(qBuf, kqBuf, ksBuf, vqBuf, vsBuf, oBuf, S, nHq, nKv, hd, nsplitOverride) {         // :2165
      TI.attn_decode_q8(ctx, qBuf, kqBuf, ksBuf, vqBuf, vsBuf, oBuf, S, nHq, nKv, hd, nsplitOverride | 0);
    },
    kvQuantWrite(krBuf, vBuf, kv, T, nKv, hd, posBase) {                                                   // :2211
      TI.kv_write_q8(ctx, krBuf, vBuf, kv.kq, kv.ks, kv.vq, kv.vs, T, nKv, hd, posBase);
    },
    ropeQK(xBuf, wBuf, outBuf, T, nH, hd, pos0, theta, eps) {                                              // :1700
      if (xBuf === outBuf) throw new Error('ropeQK: x and out must not alias');                            // :1754
      TI.rope_qk(ctx, xBuf, U(wBuf), outBuf, T, nH, hd, pos0, theta, eps);
    },
    argmaxKernel(logitsBuf, outBuf, N, outPos) { TI.argmax(ctx, logitsBuf, N, outBuf, outPos); },          // :2681
    embedGather(idsBuf, embRec, yBuf, T, H, idOff) {                                                       // :1663
      TI.embed(ctx, idsBuf, embRec.buf, yBuf, T, H, idOff | 0, embRec.vocab);
    },
    attnCausalQ8(qrBuf, kv, oBuf, T, pos0, nHq, nKv, hd) {                                                 // :2534-2577
      TI.attn_causal_q8(ctx, qrBuf, kv.kq, kv.ks, kv.vq, kv.vs, oBuf, T, pos0, nHq, nKv, hd);
    },
  };

  // ---- ternary (native/crates/n2-kernels/src/tern.rs, cpu/kernel/src/lib.rs) --------------------
  const Tern = {
    // gemv_tern(out, codes, scales, act, xsum, n, k): out in units of 1/scale
    gemv_tern(outBuf, codesBuf, scalesBuf, actBuf, xsumBuf, n, k) { TI.tern_gemv(ctx, outBuf, codesBuf, scalesBuf, actBuf, xsumBuf, n, k); },
    // several matrices over one activation (q/k/v, gate/up) in one launch: [{codes, scales, out, n}]
    gemv_tern_multi(mats, actBuf, xsumBuf, k) {
      TI.tern_gemv_multi(ctx, actBuf, xsumBuf, k, mats.map((m) => m.codes), mats.map((m) => m.scales), mats.map((m) => m.out), mats.map((m) => m.n));
    },
    gemm_tern(outBuf, outStride, codesBuf, scalesBuf, actBuf, xsumBuf, n, k, b) {
      TI.tern_gemm(ctx, outBuf, outStride, codesBuf, scalesBuf, actBuf, xsumBuf, n, k, b);
    },
    // quantize_act_into (mode 'n2') or the WASM quantize (mode 'wasm'); the scale lands in scaleBuf
    quantize_act(xBuf, actBuf, xsumBuf, scaleBuf, k, mode = 'n2') {
      TI.quant_act_tern(ctx, xBuf, actBuf, xsumBuf, scaleBuf, k, mode === 'wasm' ? 1 : 0);
    },
  };

  // ---- models/lfm25.js int3 MoE launchers ----------------------------------------------------
  // an int3 expert record: {pack, scales, nE, N, K} with the experts' rows stacked
  function int3Record(nE, N, K) {
    const g = nE * N * K / 32;
    return { pack: E.createBuffer(g * 12), scales: E.createBuffer(g * 2), nE, N, K, int3: true };
  }
  const Moe = {
    int3Record,
    _requant43(rec4, rec3, rows) { TI.requant43(ctx, rec4.pack, rec4.scales, rows, rec4.K, rec3.pack, rec3.scales); },  // :833
    router(logitsBuf, biasBuf, idxBuf, wtBuf, T, nE, K) { TI.router(ctx, logitsBuf, U(biasBuf), T, nE, K, idxBuf, wtBuf); }, // :143
    idxGemv3(xBuf, rec, idxBuf, yBuf, pairs, N, Kc, inStride, xdiv) {                                      // :1976
      TI.moe_gemv_q3(ctx, xBuf, rec.pack, rec.scales, idxBuf, yBuf, pairs, N, Kc, inStride, xdiv, rec.nE);
    },
    moeGemm3(srcBuf, srcRows, wrec, ridxBuf, yBuf, P, N, Kc, srcDiv, nE) {                                 // :1635
      TI.moe_gemm_q3(ctx, srcBuf, srcRows, wrec.pack, wrec.scales, ridxBuf, yBuf, P, N, Kc, srcDiv, nE || wrec.nE);
    },
    swiglu(gBuf, uBuf, yBuf, n) { TI.swiglu(ctx, gBuf, uBuf, yBuf, n); },                                 // :1843
    moeCombine(xBuf, oBuf, wtBuf, H, K, T) { TI.moe_combine(ctx, xBuf, oBuf, wtBuf, H, K, T || 1); },      // :1996
  };

  return { E, L, Tern, Moe, _dp4 };
}

module.exports = { createEngine, f32ToF16, engineF32ToF16, bf16ToF16bits, TI };
