'use strict';
// Drives the JS host from a spec written by the Python tests:
//   node tests/js/run_spec.js <dir>
// <dir>/spec.json:
//   buffers: {name: {file: "x.bin"} | {bytes: n}}            device buffers (files are raw bytes)
//   calls:   [{fn: "L.gemvDP4_only", args: [...]}, {read: name, bytes, out}, {read_dp4: "xq", bytes, out}]
//            an argument is a number/boolean/null, {buf: name}, {rec: {pack, scales, N, K}},
//            {kv: {kq, ks, vq, vs}}, {emb: {buf, vocab}}, {rec3: {pack, scales, nE}} or {trec: name}
//            (a record made by {tern_quant: name, src: buffer, N, K}: L.quantizeTernaryBf16)
//   selftest: true   host.selfTestKernels() -> result.selftest
//   model:   {config, nCtx, safetensors, prompt, maxTokens, dump: [tensor names]}   (optional)
//            gens: [{prompt, maxTokens, temperature}]   generate() runs on a freshly loaded model
//            prefix: {first, second, maxTokens}   conversation `second` after `first` (prefix
//                    cache reuse) and again cold on a reloaded model
//            qcache: {dir, dump, prompt, maxTokens}   load from safetensors writing the quant
//                    cache, then from the cache alone, then after a manifest of another geometry
//            tokchat: {tokenizer, text, system, maxTokens}   generate() and runConversation on text
//   kvw:     {config, nCtx, layer, T, pos, kr, v}   a randomly initialised model: qwen3_kv_layout,
//            then qwen3_kv_write of buffers kr, v at pos; the layer's K/V code rows and scales
//            [pos, pos + T) before and after are written to kvw_{before,after}.{kq,ks,vq,vs}
// Writes <dir>/result.json (and the files named by `read`).
const fs = require('fs');
const path = require('path');
const { createQwen3Host } = require(path.join(__dirname, '..', '..', 'tabinfer_amd', 'host', 'qwen3-host.js'));

async function main() {
  const dir = process.argv[2];
  const spec = JSON.parse(fs.readFileSync(path.join(dir, 'spec.json'), 'utf8'));
  const host = createQwen3Host({ device: 0 });
  const { E, L, Tern, Moe, _dp4 } = host.engine;
  const groups = { L, Tern, Moe };
  const bufs = {};
  const result = { calls: 0 };
  for (const [name, b] of Object.entries(spec.buffers || {})) {
    if (b.file) {
      const data = fs.readFileSync(path.join(dir, b.file));
      bufs[name] = E.createBuffer(data.length);
      E.writeBuffer(bufs[name], 0, new Uint8Array(data.buffer, data.byteOffset, data.length));
    } else {
      bufs[name] = E.createBuffer(b.bytes);
      E.fillU32(bufs[name], 0, Math.ceil(b.bytes / 4));
    }
  }
  const B = (n) => { if (!(n in bufs)) throw new Error('spec: no buffer ' + n); return bufs[n]; };
  const trecs = {};
  const arg = (a) => {
    if (a === null || typeof a !== 'object') return a;
    if ('buf' in a) return B(a.buf);
    if ('rec' in a) return { pack: B(a.rec.pack), scales: B(a.rec.scales), N: a.rec.N, K: a.rec.K };
    if ('kv' in a) return { kq: B(a.kv.kq), ks: B(a.kv.ks), vq: B(a.kv.vq), vs: B(a.kv.vs) };
    if ('emb' in a) return { buf: B(a.emb.buf), vocab: a.emb.vocab };
    if ('rec3' in a) return { pack: B(a.rec3.pack), scales: B(a.rec3.scales), nE: a.rec3.nE };
    if ('trec' in a) { if (!trecs[a.trec]) throw new Error('spec: no ternary record ' + a.trec); return trecs[a.trec]; }
    throw new Error('spec: bad argument ' + JSON.stringify(a));
  };
  for (const c of spec.calls || []) {
    if (c.fn) {
      const [g, f] = c.fn.split('.');
      if (!groups[g] || typeof groups[g][f] !== 'function') throw new Error('spec: no launcher ' + c.fn);
      groups[g][f](...c.args.map(arg));
      result.calls++;
    } else if (c.read) {
      fs.writeFileSync(path.join(dir, c.out), Buffer.from(E.readBytes(B(c.read), c.offset || 0, c.bytes)));
    } else if (c.read_dp4) {
      fs.writeFileSync(path.join(dir, c.out), Buffer.from(E.readBytes(_dp4[c.read_dp4], 0, c.bytes)));
    } else if (c.tern_quant) {            // L.quantizeTernaryBf16 -> a named record (or null)
      const rec = L.quantizeTernaryBf16(B(c.src), c.N, c.K);
      result[c.tern_quant] = !!rec;
      if (rec) {
        trecs[c.tern_quant] = rec;
        fs.writeFileSync(path.join(dir, c.tern_quant + '.pack'), Buffer.from(E.readBytes(rec.pack, 0, c.N * c.K / 4)));
        fs.writeFileSync(path.join(dir, c.tern_quant + '.scales'), Buffer.from(E.readBytes(rec.scales, 0, c.N * c.K / 16)));
      }
    }
  }
  if (spec.selftest) result.selftest = host.selfTestKernels();
  if (spec.model) {
    const m = spec.model;
    await host.loadModel({ config: m.config, nCtx: m.nCtx, safetensors: m.safetensors });
    result.forward = await host.forward(m.prompt, 0);
    const gen = await host.generate(m.prompt, { maxTokens: m.maxTokens });
    result.generate = Array.from(gen);
    result.dumps = {};
    for (const name of m.dump || []) {
      const t = E.TI.qwen3_tensor(host.model(), name);
      const d = Buffer.from(E.readBytes(t.data, 0, t.dataBytes));
      const s = t.scales ? Buffer.from(E.readBytes(t.scales, 0, t.scaleBytes)) : null;
      fs.writeFileSync(path.join(dir, name + '.data'), d);
      if (s) fs.writeFileSync(path.join(dir, name + '.scales'), s);
      result.dumps[name] = !!s;
    }
    const events = [];
    m.chat && (await runChat(host, m, events));
    result.events = events;
    if (m.gens) {
      result.gens = [];
      for (const g of m.gens) {
        await host.loadModel({ config: m.config, nCtx: m.nCtx, safetensors: m.safetensors, reload: true });
        const out = await host.generate(g.prompt, { maxTokens: g.maxTokens, temperature: g.temperature });
        result.gens.push(Array.from(out));
      }
    }
    if (m.prefix) result.prefix = await runPrefix(host, m);
    if (m.qcache) result.qcache = await runQcache(host, m, dir);
    if (m.tokchat) result.tokchat = await runTokChat(host, m);
  }
  if (spec.kvw) result.kvw = await runKvWrite(host, spec.kvw, B, dir);
  E.sync();
  fs.writeFileSync(path.join(dir, 'result.json'), JSON.stringify(result));
  host.shutdown();
}

async function runKvWrite(host, k, B, dir) {
  const { E } = host.engine;
  await host.loadModel({ config: k.config, nCtx: k.nCtx, random: 7, reload: true });
  const model = host.model();
  const slots = E.TI.qwen3_kv_layout(model);
  const kv = E.TI.qwen3_kv(model, k.layer);
  const hd = k.config.head_dim, nKv = k.config.n_kv_heads;
  const dump = (tag) => {
    const rowc = slots * hd, rows = nKv * (hd / 32) * 4;
    for (const [n, bytes] of [['kq', rowc], ['vq', rowc], ['ks', rows], ['vs', rows]])
      fs.writeFileSync(path.join(dir, 'kvw_' + tag + '.' + n), Buffer.from(E.readBytes(kv[n], k.pos * bytes, k.T * bytes)));
  };
  E.sync();
  dump('before');
  E.TI.qwen3_kv_write(E.ctx, model, k.layer, B(k.kr), B(k.v), k.T, k.pos);
  E.sync();
  dump('after');
  return { slots, kvSlots: kv.slots };
}

// a toy tokenizer over raw ids: encodeChat joins the messages' id lists
async function runChat(host, m, events) {
  const tok = {
    encodeChat: (msgs) => [].concat(...msgs.map((x) => x.content.split(' ').map(Number))),
    decode: (ids) => ids.map((i) => '<' + i + '>').join(''),
    isStop: (id) => id === m.chat.stop,
  };
  await host.loadModel({ config: m.config, nCtx: m.nCtx, safetensors: m.safetensors, tokenizer: tok, reload: true });
  await host.runConversation({ provider: { maxTokens: m.maxTokens }, messages: [{ role: 'user', content: m.prompt.join(' ') }] },
    (ev) => events.push(ev));
}

// runConversation over id "text": the tokens of `second` after `first` ran (its KV rows reused
// by the prefix cache) and of `second` on a reloaded model (cold prefill)
async function runPrefix(host, m) {
  const tok = {
    encodeChat: (msgs) => [].concat(...msgs.map((x) => x.content.split(' ').filter((w) => w).map(Number))),
    decode: (ids) => ids.map((i) => ' ' + i).join(''),
    isStop: () => false,
  };
  const conv = async (msgs) => {
    const ev = [];
    await host.runConversation({ provider: { maxTokens: m.prefix.maxTokens }, messages: msgs }, (e) => ev.push(e));
    return ev.filter((e) => e.type === 'delta' && e.delta.content).map((e) => e.delta.content).join('').trim();
  };
  const load = () => host.loadModel({ config: m.config, nCtx: m.nCtx, safetensors: m.safetensors, tokenizer: tok, reload: true });
  await load();
  const a1 = await conv(m.prefix.first);
  const second = m.prefix.first.concat([{ role: 'assistant', content: a1 }], m.prefix.second);
  const warm = await conv(second);
  await load();
  const cold = await conv(second);
  return { first: a1, warm, cold };
}

// the quantized-weights cache: a checkpoint load writes it (tensors dumped as a.*), a load
// from the cache alone reads it (b.*); a manifest edited to another geometry is no cache
async function runQcache(host, m, dir) {
  const { E } = host.engine;
  const q = m.qcache;
  const base = { config: m.config, nCtx: m.nCtx, quantCache: q.dir, reload: true };
  const dump = (tag) => {
    for (const name of q.dump) {
      const t = E.TI.qwen3_tensor(host.model(), name);
      fs.writeFileSync(path.join(dir, tag + '.' + name + '.data'), Buffer.from(E.readBytes(t.data, 0, t.dataBytes)));
      if (t.scales) fs.writeFileSync(path.join(dir, tag + '.' + name + '.scales'), Buffer.from(E.readBytes(t.scales, 0, t.scaleBytes)));
    }
  };
  const out = { fromCache: [], gens: [] };
  await host.loadModel(Object.assign({ safetensors: m.safetensors }, base));
  out.fromCache.push(host.loadedFromCache());
  dump('a');
  out.gens.push(Array.from(await host.generate(q.prompt, { maxTokens: q.maxTokens })));
  await host.loadModel(base);                          // no checkpoint: the cache alone
  out.fromCache.push(host.loadedFromCache());
  dump('b');
  out.gens.push(Array.from(await host.generate(q.prompt, { maxTokens: q.maxTokens })));
  const mf = path.join(q.dir, 'v1', 'custom', 'manifest');
  const man = JSON.parse(fs.readFileSync(mf, 'utf8'));
  man.config.vocab += 1;
  fs.writeFileSync(mf, JSON.stringify(man));
  await host.loadModel(Object.assign({ safetensors: m.safetensors }, base));   // a miss: the checkpoint, the cache rewritten
  out.fromCache.push(host.loadedFromCache());
  await host.loadModel(base);
  out.fromCache.push(host.loadedFromCache());
  out.gens.push(Array.from(await host.generate(q.prompt, { maxTokens: q.maxTokens })));
  out.manifest = JSON.parse(fs.readFileSync(mf, 'utf8'));
  // another checkpoint of the same geometry through the same cache: a miss, its own weights
  // (dumped as c.*), and the cache then holds it (a cache-only load gives c.* again as d.*)
  if (q.safetensorsB) {
    await host.loadModel(Object.assign({ safetensors: q.safetensorsB }, base));
    out.fromCache.push(host.loadedFromCache());
    dump('c');
    await host.loadModel(base);
    out.fromCache.push(host.loadedFromCache());
    dump('d');
    out.manifestB = JSON.parse(fs.readFileSync(mf, 'utf8'));
  }
  // no usable weights: an empty cache directory and no checkpoint is an error, no model stays loaded
  try {
    await host.loadModel({ config: m.config, nCtx: m.nCtx, quantCache: path.join(dir, 'empty-cache'), reload: true });
    out.noWeights = null;
  } catch (e) { out.noWeights = e.message; }
  out.modelAfterNoWeights = host.model() === null;
  return out;
}

// text through the tokenizer: generate()'s streamed pieces and result, the prompt length,
// and a conversation's usage and content
async function runTokChat(host, m) {
  const t = m.tokchat;
  await host.loadModel({ config: m.config, nCtx: m.nCtx, safetensors: m.safetensors, tokenizer: t.tokenizer, reload: true });
  const pieces = [];
  const text = await host.generate(t.text, { maxTokens: t.maxTokens, onToken: (x) => pieces.push(x) });
  const out = { text, pieces, prefill: host.lastGenStats().prefillTokens, events: [] };
  await host.runConversation({ provider: { maxTokens: t.maxTokens }, systemPrompt: t.system,
    messages: [{ role: 'user', content: t.text }] }, (ev) => out.events.push(ev));
  return out;
}

main().catch((e) => { console.error(e && e.stack ? e.stack : e); process.exit(1); });
