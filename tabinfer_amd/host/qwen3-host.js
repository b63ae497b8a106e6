'use strict';
// qwen3-host.js — the Qwen3 decode API of TabInfer (models/qwen3.js, exported at
// :5529-5534: forward, generate, runConversation, loadModel, ...) over the MI355X library.
//
// The model-level forward runs in the native decoder object (ti_qwen3_*): a T-token
// forward for prefill chunks and a device-position decode step that reads nothing from
// the host, captured once into a HIP graph and replayed per token (the reference's
// GPU-resident token chaining, models/qwen3.js:3951-3959 and decodeLoop :4414-4435).
//
// Tokenization: loadModel({tokenizer}) takes a path to a local tokenizer.json (or its
// directory; tokenizer.js, the reference's TOK), or any object with encodeChat(messages)
// -> ids, decode(ids) -> string and isStop(id) -> bool; with neither, the tokenizer.json
// beside the safetensors file is used when there is one, else prompts are arrays of token
// ids and decode() returns them.
const fs = require('fs');
const path = require('path');
const { createEngine, bf16ToF16bits, f32ToF16 } = require('./ti-engine');
const { loadTokenizer } = require('./tokenizer');
const { selfTestKernels } = require('./self-test');
const QC = require('./quant-cache');
const CONV = require('./conversation');

// models/qwen3.js CONFIGS (Qwen3-0.6B / 1.7B geometry)
const CONFIGS = {
  '0.6B': { layers: 28, hidden: 1024, intermediate: 3072, n_heads: 16, n_kv_heads: 8, head_dim: 128, vocab: 151936 },
  '1.7B': { layers: 28, hidden: 2048, intermediate: 6144, n_heads: 16, n_kv_heads: 8, head_dim: 128, vocab: 151936 },
};
const GEN_BATCH = 32;        // decode steps per readback (models/qwen3.js:4535)
const PIPE_DEPTH = 3;        // batches in flight, so the GPU never waits for a readback (:4537)
const PIPE_SLOT0 = 56;       // event slots PIPE_SLOT0 .. + PIPE_DEPTH - 1 mark the batches' readbacks
const PREFILL_CHUNK = 256;   // prefill tokens per forward (models/qwen3.js:5250) ...
const ATTN_ROWS = 4096;      // ... within the library's T * n_heads <= 4096 (ti_qwen3_config)
const STAGE_BYTES = 64 << 20;

// ---- safetensors ----------------------------------------------------------------------------
function readSafetensorsHeader(file) {
  const fd = fs.openSync(file, 'r');
  try {
    const lenBuf = Buffer.alloc(8);
    fs.readSync(fd, lenBuf, 0, 8, 0);
    const n = Number(lenBuf.readBigUInt64LE(0));
    if (n <= 0 || n > (100 << 20)) throw new Error('safetensors: bad header length ' + n + ' in ' + file);
    const hb = Buffer.alloc(n);
    fs.readSync(fd, hb, 0, n, 8);
    const hdr = JSON.parse(hb.toString('utf8'));
    const tensors = {};
    for (const [name, info] of Object.entries(hdr)) {
      if (name === '__metadata__') continue;
      tensors[name] = { dtype: info.dtype, shape: info.shape, begin: 8 + n + info.data_offsets[0], end: 8 + n + info.data_offsets[1], file };
    }
    return tensors;
  } finally {
    fs.closeSync(fd);
  }
}

function readRange(t, off, bytes) {
  const fd = fs.openSync(t.file, 'r');
  try {
    const b = Buffer.alloc(bytes);
    let got = 0;
    while (got < bytes) {
      const r = fs.readSync(fd, b, got, bytes - got, t.begin + off + got);
      if (r <= 0) throw new Error('safetensors: short read in ' + t.file);
      got += r;
    }
    return b;
  } finally {
    fs.closeSync(fd);
  }
}

function toF16Bits(t, buf) {
  const n = buf.length / (t.dtype === 'F32' ? 4 : 2);
  if (t.dtype === 'BF16') return bf16ToF16bits(new Uint16Array(buf.buffer, buf.byteOffset, n));
  if (t.dtype === 'F16') return new Uint16Array(buf.buffer.slice(buf.byteOffset, buf.byteOffset + buf.length));
  if (t.dtype === 'F32') {
    const f = new Float32Array(buf.buffer, buf.byteOffset, n), out = new Uint16Array(n);
    for (let i = 0; i < n; i++) out[i] = f32ToF16(f[i]);
    return out;
  }
  throw new Error('unsupported dtype ' + t.dtype);
}

// toolPreamble (:5294-5320): Qwen3's own (Hermes) tool block, appended to the system prompt,
// the text its chat template renders (the model was trained on exactly this wording)
function claimSystemBlock(ids, sysIds, cachedIds, anchorIds) {
  if (!sysIds || sysIds.length < 16) return false;
  const P = sysIds.length;
  const covers = (a, n) => { if (!a || a.length < n) return false; for (let i = 0; i < n; i++) if (a[i] !== sysIds[i]) return false; return true; };
  if (!covers(ids, P)) return false;
  if (covers(cachedIds, P)) return false;
  return !!anchorIds && anchorIds.length === P && covers(anchorIds, P);
}

// ---- the model ----------------------------------------------------------------------------------
function createQwen3Host({ device = 0 } = {}) {
  const eng = createEngine({ device });
  const { E } = eng;
  const TI = E.TI, ctx = E.ctx;
  let M = null;          // native decoder
  let C = null;          // its config
  let TOK = null;
  let _devPos = -1;      // the device-side position as this host last left it
  let _decodeGraph = null, _decodeSplits = -1;
  let _cachedIds = null; // prefix cache: the ids whose KV rows are resident
  let _toolRunner = null;
  let _lastGenStats = null;
  let _lastLoadCached = false;
  let _sysAnchor = null; // {ids}: KV rows [0, ids.length) hold this system block (:5363-5395)

  function tensorNames(cfg) {
    const names = ['model.embed_tokens.weight', 'model.norm.weight', 'lm_head.weight'];
    for (let l = 0; l < cfg.layers; l++) {
      const p = 'model.layers.' + l + '.';
      for (const n of ['self_attn.q_proj.weight', 'self_attn.k_proj.weight', 'self_attn.v_proj.weight', 'self_attn.o_proj.weight',
        'mlp.gate_proj.weight', 'mlp.up_proj.weight', 'mlp.down_proj.weight', 'input_layernorm.weight',
        'post_attention_layernorm.weight', 'self_attn.q_norm.weight', 'self_attn.k_norm.weight']) names.push(p + n);
    }
    return names;
  }

  // bf16 [N, K] rows from `readRows(row0, rows) -> Uint8Array` -> int4 pack/scales on the GPU
  function quantizeInto(dst, N, K, readRows, stage) {
    const rowsPer = Math.max(1, Math.min(N, Math.floor(STAGE_BYTES / (K * 2))));
    for (let r = 0; r < N; r += rowsPer) {
      const nr = Math.min(rowsPer, N - r);
      E.writeBuffer(stage, 0, readRows(r, nr));
      TI.quant_int4_bf16(ctx, stage, E.view(dst.data, r * K / 2), E.view(dst.scales, r * K / 32 * 2), nr, K);
    }
  }

  function loadWeights(files, onProgress) {
    const all = {};
    for (const f of files) Object.assign(all, readSafetensorsHeader(f));
    const names = tensorNames(C);
    const stage = E.createBuffer(STAGE_BYTES);
    try {
      names.forEach((name, i) => {
        let t = all[name];
        if (!t && name === 'lm_head.weight') t = all['model.embed_tokens.weight'];   // tied embeddings
        if (!t) throw new Error('loadModel: checkpoint has no tensor ' + name);
        const dst = TI.qwen3_tensor(M, name);
        if (dst.scales) {
          if (t.dtype !== 'BF16') throw new Error('quant path expects BF16 for ' + name);   // models/qwen3.js:3502
          const [N, K] = t.shape;
          if (N * K / 2 !== dst.dataBytes) throw new Error('loadModel: ' + name + ' has shape ' + t.shape + ', the model expects ' + (dst.dataBytes * 2) + ' weights');
          quantizeInto(dst, N, K, (r0, nr) => readRange(t, r0 * K * 2, nr * K * 2), stage);
        } else {
          const bits = toF16Bits(t, readRange(t, 0, t.end - t.begin));
          if (bits.byteLength !== dst.dataBytes) throw new Error('loadModel: ' + name + ' size mismatch');
          E.writeBuffer(dst.data, 0, bits);
        }
        if (onProgress) onProgress({ phase: 'parse', pct: Math.round(100 * (i + 1) / names.length) });
      });
      E.sync();
    } finally {
      E.destroy(stage);
    }
  }

  // seeded synthetic weights: bf16 N(0, 0.02) projections quantized on the GPU, norms 1.0,
  // f16 N(0, 1) embeddings (for benchmarks and smoke runs without a checkpoint)
  function randomWeights(seed) {
    let s = (seed >>> 0) || 1;
    const rnd = () => { s ^= s << 13; s >>>= 0; s ^= s >>> 17; s ^= s << 5; s >>>= 0; return s / 4294967296; };
    const gauss = () => Math.sqrt(-2 * Math.log(rnd() + 1e-12)) * Math.cos(2 * Math.PI * rnd());
    const stage = E.createBuffer(STAGE_BYTES);
    const f = new Float32Array(1), u = new Uint32Array(f.buffer);
    try {
      for (const name of tensorNames(C)) {
        const dst = TI.qwen3_tensor(M, name);
        if (dst.scales) {
          const n = dst.dataBytes * 2, K = name.endsWith('down_proj.weight') ? C.intermediate
            : name.endsWith('o_proj.weight') ? C.n_heads * C.head_dim : C.hidden;
          quantizeInto(dst, n / K, K, (r0, nr) => {
            const b = new Uint16Array(nr * K);
            for (let i = 0; i < b.length; i++) { f[0] = 0.02 * gauss(); b[i] = u[0] >>> 16; }
            return b;
          }, stage);
        } else {
          const n = dst.dataBytes / 2, b = new Uint16Array(n);
          const emb = name === 'model.embed_tokens.weight';
          for (let i = 0; i < n; i++) b[i] = emb ? f32ToF16(gauss()) : 0x3c00;
          E.writeBuffer(dst.data, 0, b);
        }
      }
      E.sync();
    } finally {
      E.destroy(stage);
    }
  }

  // the tensors of the decoder as quant-cache segments, in stream order
  function cacheSegments() {
    const segs = [];
    for (const name of tensorNames(C)) {
      const t = TI.qwen3_tensor(M, name);
      if (t.scales) {
        const K = name.endsWith('down_proj.weight') ? C.intermediate : name.endsWith('o_proj.weight') ? C.n_heads * C.head_dim : C.hidden;
        const N = t.dataBytes * 2 / K;
        const meta = { kind: 'int4', shape: [N, K], numel: N * K, N, K };
        segs.push(Object.assign({ name, role: 'pack', len: t.dataBytes, buf: t.data }, meta));
        segs.push(Object.assign({ name, role: 'scales', len: t.scaleBytes, buf: t.scales }, meta));
      } else {
        const numel = t.dataBytes / 2;
        const shape = name === 'model.embed_tokens.weight' ? [C.vocab, C.hidden] : [numel];
        segs.push({ name, role: 'buf', len: t.dataBytes, buf: t.data, kind: 'f16', shape, numel });
      }
    }
    return segs;
  }

  // the fast load (models/qwen3.js:3675-3717): every segment of a valid cache written
  // straight into the decoder's buffers; false when the directory holds no usable cache
  function loadQuantCache(dir, variant, onProgress, source) {
    const bufs = new Map(cacheSegments().map((s) => [s.name + '.' + s.role, s]));
    return QC.readQuantCache(dir, variant, C, (seg, off, bytes) => E.writeBuffer(bufs.get(seg.name + '.' + seg.role).buf, off, bytes), {
      onProgress,
      source,
      check: (seg) => {
        const mine = bufs.get(seg.name + '.' + seg.role);
        if (!mine || mine.len !== seg.len) throw new Error('quant cache: segment ' + seg.name + '.' + seg.role + ' does not fit this model');
      },
    });
  }

  // the writer (:3629-3664): the quantized bytes read back from the GPU, one tensor at a time
  function writeQuantCache(dir, variant, source) {
    E.sync();
    return QC.writeQuantCache(dir, variant, C, cacheSegments(), (seg) => new Uint8Array(E.readBytes(seg.buf, 0, seg.len)), { source });
  }

  // loadModel({variant, nCtx, config, safetensors, random, tokenizer, quantCache, onProgress})
  // (models/qwen3.js:3719): allocates the decoder for `nCtx` positions and fills it. With
  // quantCache (a directory), a valid cache of this variant and geometry is loaded instead
  // of the checkpoint; after a checkpoint load the cache is (re)written. When safetensors
  // are named, only a cache quantized from those same files is read (path, size,
  // modification time and header hash), so another checkpoint of the same geometry is a
  // miss. A cache that cannot be read falls back to the checkpoint (:3752-3759); a failed
  // write only warns. With no usable source of weights (a cache miss and neither
  // safetensors nor random) loadModel throws and leaves no model loaded.
  async function loadModel(opts = {}) {
    if (M && !opts.reload) return;
    if (M) unload();
    const base = opts.config || CONFIGS[opts.variant || '0.6B'];
    if (!base) throw new Error('loadModel: unknown variant ' + opts.variant);
    const variant = opts.variant || (opts.config ? 'custom' : '0.6B');
    const maxCtx = opts.nCtx || base.max_ctx || 4096;
    const chunk = Math.max(1, Math.min(PREFILL_CHUNK, Math.floor(ATTN_ROWS / base.n_heads), maxCtx));
    C = Object.assign({ rope_theta: 1e6, rms_eps: 1e-6 }, base, { max_ctx: maxCtx, max_tokens: chunk });
    M = TI.qwen3_create(ctx, C);
    _temp = 0;                           // a new decoder samples greedily until told otherwise
    _sysAnchor = null;
    TOK = typeof opts.tokenizer === 'string' ? loadTokenizer(opts.tokenizer) : (opts.tokenizer || null);
    if (!TOK && opts.safetensors) {
      const beside = path.join(path.dirname([].concat(opts.safetensors)[0]), 'tokenizer.json');
      if (fs.existsSync(beside)) TOK = loadTokenizer(beside);
    }
    const files = opts.safetensors ? [].concat(opts.safetensors) : null;
    let source = null;
    if (files && opts.quantCache) {
      try { source = QC.checkpointIdentity(files); } catch (e) { unload(); throw e; }
    }
    let cached = false;
    if (opts.quantCache) {
      try { cached = loadQuantCache(opts.quantCache, variant, opts.onProgress, source); } catch (e) {
        console.warn('[qwen3] quant cache load failed, loading the checkpoint:', (e && e.message) || e);
      }
    }
    if (!cached) {
      if (files) {
        loadWeights(files, opts.onProgress);
        if (opts.quantCache) {
          try { writeQuantCache(opts.quantCache, variant, source); } catch (e) {
            console.warn('[qwen3] quant cache write failed (the next load quantizes again):', (e && e.message) || e);
          }
        }
      } else if (opts.random != null) randomWeights(opts.random);
      else {
        unload();
        throw new Error('loadModel: no weights: ' + (opts.quantCache ? 'no usable quant cache in ' + opts.quantCache + ', and ' : '') +
          'neither safetensors nor random was given');
      }
    }
    E.sync();
    _lastLoadCached = cached;
    _devPos = -1;
    _cachedIds = null;
  }

  function unload() {
    if (_decodeGraph) { E.destroyGraph(_decodeGraph); _decodeGraph = null; _decodeSplits = -1; }
    if (_pipe) { E.sync(); for (const b of _pipe) TI.host_free(b.buffer); _pipe = null; }
    if (M) { TI.qwen3_destroy(M); M = null; }
  }

  function need() { if (!M) throw new Error('no model loaded: call loadModel() first'); }
  // the decoder's sampling temperature (device-side, read by every step; 0 = greedy)
  let _temp = 0;
  function setTemp(t) { if (t !== _temp) { TI.qwen3_sampling(ctx, M, t); _temp = t; } }
  function setPos(pos) { if (_devPos !== pos) { TI.qwen3_set_pos(ctx, M, pos); _devPos = pos; } }
  function readTok(pos) { return TI.qwen3_read_tokens(ctx, M, pos, 1)[0]; }

  function logitsNow() { return new Float32Array(E.readBytes(TI.qwen3_logits(M), 0, C.vocab * 4)); }

  // distStats over the last logits: logprob of tok, top-k alternatives, entropy (nats)
  function distStats(logits, tok, k) {
    let mx = -Infinity;
    for (let i = 0; i < logits.length; i++) if (logits[i] > mx) mx = logits[i];
    let z = 0;
    for (let i = 0; i < logits.length; i++) z += Math.exp(logits[i] - mx);
    const lz = Math.log(z) + mx;
    let ent = 0;
    for (let i = 0; i < logits.length; i++) { const lp = logits[i] - lz; ent -= Math.exp(lp) * lp; }
    const idx = Array.from(logits.keys()).sort((a, b) => logits[b] - logits[a]).slice(0, k);
    return { logprob: logits[tok] - lz, alts: idx.map((i) => ({ id: i, logprob: logits[i] - lz })), entropy: ent };
  }

  // forward(idsArray, posBase, {chain, submitOnly, logprobs}) -> next token id (:3938).
  // A caller's forward may overwrite any KV rows, so it drops the prefix caches; the
  // host's own prefill goes through fwd, which keeps them.
  async function forward(idsArray, posBase, opts) {
    _cachedIds = null;
    _sysAnchor = null;
    return fwd(idsArray, posBase, opts);
  }
  async function fwd(idsArray, posBase, opts) {
    need();
    const chain = !!(opts && opts.chain), submitOnly = !!(opts && opts.submitOnly);
    setTemp(opts && opts.temp > 0 ? +opts.temp : 0);   // :4052, Gumbel-max in the lm_head
    let T;
    if (chain) {
      T = 1;
      setPos(posBase);
      TI.qwen3_decode(ctx, M);
    } else {
      const ids = Int32Array.from(idsArray);
      T = ids.length;
      if (T < 1 || T > C.max_tokens) throw new Error('forward: T=' + T + ' outside [1, ' + C.max_tokens + ']');
      TI.qwen3_forward(ctx, M, ids, T, posBase);
    }
    _devPos = posBase + T;
    if (submitOnly) return undefined;
    await E.drain();
    const tok = readTok(posBase + T);
    if (opts && opts.logprobs) return Object.assign({ tok }, distStats(logitsNow(), tok, 5));
    return tok;
  }

  // the captured step for a loop starting at pos: its attention split count follows the
  // context (qwen3_decode_splits), so a loop at a position of another tier captures anew,
  // after the earlier graph's replays have drained
  function decodeGraph(pos) {
    const ns = TI.qwen3_decode_splits(M, pos);
    if (_decodeGraph && _decodeSplits === ns) return _decodeGraph;
    if (_decodeGraph) { E.sync(); E.destroyGraph(_decodeGraph); _decodeGraph = null; }
    TI.qwen3_set_pos(ctx, M, pos);   // the capture reads the position last set on the host
    _devPos = pos;
    E.beginBatch();
    try { TI.qwen3_decode(ctx, M); } finally { _decodeGraph = E.endBatch(); }
    _decodeSplits = ns;
    return _decodeGraph;
  }

  // decodeLoop (:4414-4435): batches of GEN_BATCH graph replays of the device-position step,
  // each followed by a queued readback of the tokens it chained; PIPE_DEPTH batches stay in
  // flight, and the host consumes the oldest while the GPU runs the newer ones. Stops on
  // emitTok() === false, maxTokens or the cache end; batches still in flight then run out
  // (as the reference's discarded batches do) before their buffers are reused.
  let _pipe = null;
  async function decodeLoop(pos, maxTokens, emitTok, signal, count, temp) {
    const g = decodeGraph(pos);
    if (!_pipe) _pipe = Array.from({ length: PIPE_DEPTH }, () => new Int32Array(TI.host_alloc(GEN_BATCH * 4)));
    setTemp(temp > 0 ? +temp : 0);
    setPos(pos);
    let submitted = 0, seq = 0;
    const submitBatch = () => {
      if (signal && signal.aborted) return null;
      const K = Math.min(GEN_BATCH, C.max_ctx - 1 - pos, maxTokens + GEN_BATCH - submitted);
      if (K <= 0) return null;
      const base = pos, i = seq++ % PIPE_DEPTH;
      for (let k = 0; k < K; k++) E.launch(g);
      pos += K; submitted += K; _devPos = pos;
      TI.qwen3_read_tokens_async(ctx, M, base + 1, K, _pipe[i]);
      TI.event_record(ctx, PIPE_SLOT0 + i);
      return { K, buf: _pipe[i], done: TI.event_wait_async(ctx, PIPE_SLOT0 + i) };
    };
    const inflight = [];
    try {
      while (inflight.length < PIPE_DEPTH) { const b = submitBatch(); if (!b) break; inflight.push(b); }
      while (inflight.length) {
        const cur = inflight.shift();
        await cur.done;
        const toks = cur.buf.slice(0, cur.K);              // copied out before the buffer is reused
        let stop = !!(signal && signal.aborted);
        if (!stop) for (let k = 0; k < cur.K; k++) { if (!emitTok(toks[k]) || count() >= maxTokens) { stop = true; break; } }
        if (stop) break;
        const b = submitBatch(); if (b) inflight.push(b);
      }
    } finally {
      for (const b of inflight) await b.done.catch(() => {});
    }
  }

  function encode(x) {
    if (Array.isArray(x) || ArrayBuffer.isView(x)) return Array.from(x);
    if (!TOK) throw new Error('a text prompt needs loadModel({tokenizer})');
    return TOK.encodeChat(typeof x === 'string' ? [{ role: 'user', content: x }] : x);
  }
  const decode = (ids) => (TOK ? TOK.decode(ids) : ids.slice());
  // the text each emitted token completes (a tokenizer without a stream decoder: its decode of the token)
  const textStream = () => (TOK && TOK.streamDecoder ? TOK.streamDecoder()
    : { push: (t) => (TOK ? TOK.decode([t]) : String(t)), flush: () => '' });
  const isStop = (t) => !!(TOK && TOK.isStop && TOK.isStop(t));

  // prefill ids[from..L) in chunks of up to PREFILL_CHUNK (C.max_tokens); returns the token
  // after the last; a temperature applies to the last chunk's token only (:4553-4556)
  async function prefill(ids, from, signal, temp) {
    let tok;
    for (let off = from; off < ids.length; off += C.max_tokens) {
      if (signal && signal.aborted) throw abortError();
      const last = off + C.max_tokens >= ids.length;
      tok = await fwd(ids.slice(off, Math.min(off + C.max_tokens, ids.length)), off, last && temp ? { temp } : undefined);
    }
    return tok;
  }

  function abortError() { const e = new Error('aborted'); e.name = 'AbortError'; return e; }

  function checkFits(L) {
    if (L + 64 > C.max_ctx) throw new Error('prompt too long: ' + L + ' tokens — exceeds the context limit (' + C.max_ctx + ').');
  }

  // generate(prompt, {maxTokens, onToken, onStats, signal}) (:4538-4569)
  async function generate(prompt, { maxTokens = 64, onToken, onStats, signal, temperature } = {}) {
    need();
    const temp = temperature > 0 ? +temperature : 0;
    _cachedIds = null;
    _sysAnchor = null;                   // the one-shot path prefills from position 0 (:4540)
    const ids = encode(prompt);
    const L = ids.length;
    checkFits(L);
    const t0 = Date.now();
    const tok0 = await prefill(ids, 0, signal, temp);
    const ms = Date.now() - t0;
    _lastGenStats = { prefillTokens: L, prefillMs: ms, prefillTps: +(L / Math.max(ms, 1e-3) * 1000).toFixed(1) };
    if (onStats) { try { onStats(_lastGenStats); } catch (_) { /* caller's hook */ } }
    const out = [];
    const sd = textStream();
    const emit = (t) => {
      if (isStop(t)) return false;
      out.push(t);
      if (onToken) { const x = TOK ? sd.push(t) : t; if (x !== '') { try { onToken(x); } catch (_) { /* caller's hook */ } } }
      return true;
    };
    if (emit(tok0)) await decodeLoop(L, maxTokens, emit, signal, () => out.length, temp);
    if (onToken && TOK) { const x = sd.flush(); if (x) { try { onToken(x); } catch (_) { /* caller's hook */ } } }
    return decode(out);
  }

  // _streamIds (:5199-5292) without grammar masking: prefix-cache reuse, chunked prefill of
  // the rest, then the batched decode loop
  async function streamIds(ids, { maxTokens, onToken, signal, temperature }) {
    const temp = temperature > 0 ? +temperature : 0;
    const L = ids.length;
    checkFits(L);
    let lcp = 0;
    if (_cachedIds) { const n = Math.min(_cachedIds.length, L - 1); while (lcp < n && _cachedIds[lcp] === ids[lcp]) lcp++; }
    _cachedIds = null;   // from here on rows lcp.. are being overwritten
    if (_sysAnchor && lcp < _sysAnchor.ids.length) _sysAnchor = null;
    let tok0;
    try { tok0 = await prefill(ids, lcp, signal, temp); } catch (e) {
      _sysAnchor = null;                 // the KV prefix is now partial (:5257-5259)
      throw e;
    }
    const out = [];
    const sd = textStream();
    const emitTok = (t) => { if (isStop(t)) return false; out.push(t); if (onToken) { const x = sd.push(t); if (x) onToken(x); } return true; };
    if (emitTok(tok0)) await decodeLoop(L, maxTokens, emitTok, signal, () => out.length, temp);
    if (onToken) { const x = sd.flush(); if (x) onToken(x); }
    // Rows [0, L) hold the prompt. The step at position L + j wrote the row of out[j] and
    // produced out[j + 1], so rows exist for out[0 .. n-2]; the last emitted token's row
    // is written only if a later step ran, which a stop at maxTokens or the cache end skips.
    _cachedIds = ids.concat(out.slice(0, Math.max(0, out.length - 1)));
    return out;
  }

  // The system-prompt KV anchor (:5363-5395): after round 0 of a conversation, KV rows
  // [0, P) hold the system block (system prompt + tool preamble, P tokens, no generation
  // prompt); a later conversation with the same system block whose prefix cache no longer
  // covers it claims those rows instead of prefilling them again. Any prefill that starts
  // below P drops the anchor first (its rows are being rewritten); a successful round 0
  // records it again.
  const startsWith = (ids, pre) => !!pre && ids.length >= pre.length && pre.every((t, i) => ids[i] === t);
  function sysCacheClaim(ids, sysIds, emit) {
    if (!claimSystemBlock(ids, sysIds, _cachedIds, _sysAnchor && _sysAnchor.ids)) return false;
    _cachedIds = sysIds;
    emit({ type: 'info', message: 'Using cached system prompt…' });
    return true;
  }

  // runConversation({provider, messages, systemPrompt, tools, convId, signal}, emit)
  // (models/qwen3.js:5397-5522): the system block (system prompt + tool preamble) and the
  // rendered messages form the transcript; conversation.js runs the rounds over streamIds,
  // with the system-prompt KV anchor claimed before round 0 and recorded after it.
  async function runConversation({ provider, messages, systemPrompt, tools, convId, signal } = {}, emit) {
    const unusable = !M ? 'no model loaded: call loadModel() first' : (!TOK ? 'runConversation needs loadModel({tokenizer})' : null);
    if (unusable) {
      emit({ type: 'error', message: CONV.ERROR_PREFIX + unusable });
      emit({ type: 'agent_done' });
      return;
    }
    const offered = (Array.isArray(tools) ? tools : []).filter((t) => t && t.type === 'function');
    const sysText = [(systemPrompt && typeof systemPrompt === 'object') ? (systemPrompt.content || '') : (systemPrompt || ''),
      CONV.toolPreamble(offered)].filter(Boolean).join('\n\n');
    const transcript = sysText ? [{ role: 'system', content: sysText }] : [];
    for (const m of (messages || [])) if (m && m.role) transcript.push(CONV.renderMessage(m));
    const sysIds = sysText ? TOK.encodeChat([{ role: 'system', content: sysText }], { addGenerationPrompt: false }) : null;
    const maxTokens = (provider && (provider.maxTokens | 0)) || C.max_ctx;
    const deps = {
      encode: (msgs) => TOK.encodeChat(msgs),
      stream: (ids, onText) => streamIds(ids, { maxTokens, signal, onToken: onText }),
      runTool: _toolRunner,
      hooks: {
        beforeFirst: (ids) => sysCacheClaim(ids, sysIds, emit),
        afterFirst: (ids) => { _sysAnchor = sysIds && sysIds.length >= 16 && startsWith(ids, sysIds) ? { ids: sysIds } : null; },
      },
    };
    await CONV.converse({ transcript, toolsOffered: offered.length > 0, ctxLimit: C.max_ctx, convId, signal }, deps, emit);
  }

  return {
    CONFIGS, engine: eng, loadModel, unload, forward, generate, runConversation, decodeLoop,
    setToolRunner(fn) { _toolRunner = fn; },
    lastGenStats: () => _lastGenStats,
    loadedFromCache: () => _lastLoadCached,
    selfTestKernels: () => selfTestKernels(eng),        // models/qwen3.js:2753, exported at :5529
    tokenizer: () => TOK,
    config: () => C,
    model: () => M,
    readTokens: (from, n) => TI.qwen3_read_tokens(ctx, M, from, n),
    logits: () => logitsNow(),
    shutdown() { unload(); E.shutdown(); },
  };
}

module.exports = { createQwen3Host, CONFIGS, readSafetensorsHeader, toolPreamble: CONV.toolPreamble, renderMessage: CONV.renderMessage, claimSystemBlock, GEN_BATCH,
  PIPE_DEPTH, PREFILL_CHUNK };
