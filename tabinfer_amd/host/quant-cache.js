'use strict';
// The quantized-weights cache (models/qwen3.js:3340-3351, 3626-3717) on a local directory:
// after a checkpoint has been quantized, its GPU-ready bytes (int4 packs and f16 scales,
// f16 tensors) are written as one byte stream cut into 64 MiB chunk files plus a JSON
// manifest; a later load reads the chunks and writes their slices straight into the
// decoder's buffers, with no safetensors parse and no quantization.
//
//   <dir>/v1/<variant>/manifest   {ver, variant, qgroup, chunkSize, nChunks, totalBytes,
//                                  config: {numLayers, hidden, nHeads, nKvHeads, headDim,
//                                  intermediate, vocab}, segs: [{name, role, off, len,
//                                  kind, shape, numel, N, K}]}
//   <dir>/v1/<variant>/c0, c1, ...  the stream: every segment starts 16-byte aligned
//
// The manifest also records `source`, the checkpoint the bytes were quantized from (each
// safetensors file's resolved path, size, modification time and a SHA-256 of its header;
// the reference needs no such field because its variant fixes the download URL). A load
// that names a checkpoint reads the cache only when the checkpoint's identity matches; a
// load from the cache alone accepts any source.
//
// The manifest is the commit point, as in the reference: removed before a write starts,
// written after the last chunk, so a cache whose write was cut short is never read. A
// manifest that does not match (version, variant, group size, chunk size, the model's
// dims) reads as no cache. No device calls here: segment bytes come from `get(seg)` and
// go to `put(seg, offset, bytes)`, so the format is testable without a GPU.
const fs = require('fs');
const path = require('path');
const crypto = require('crypto');

const QCACHE_VER = 1;
const QCHUNK = 64 * 1024 * 1024;
const QGROUP = 32;
const ceil16 = (n) => (n + 15) & ~15;

// the dims that fix the quantized layout (models/qwen3.js:3627), under the reference's names
function configKey(c) {
  return { numLayers: c.layers, hidden: c.hidden, nHeads: c.n_heads, nKvHeads: c.n_kv_heads, headDim: c.head_dim,
    intermediate: c.intermediate, vocab: c.vocab };
}

// the identity of a checkpoint (one or more safetensors files, in load order)
function checkpointIdentity(files) {
  return {
    files: [].concat(files).map((f) => {
      const abs = path.resolve(f);
      const st = fs.statSync(abs);
      const fd = fs.openSync(abs, 'r');
      try {
        const lenBuf = Buffer.alloc(8);
        if (fs.readSync(fd, lenBuf, 0, 8, 0) !== 8) throw new Error('safetensors: ' + abs + ' is shorter than its header length');
        const n = Number(lenBuf.readBigUInt64LE(0));
        if (!(n > 0 && n <= st.size - 8)) throw new Error('safetensors: bad header length ' + n + ' in ' + abs);
        const hb = Buffer.alloc(n);
        if (fs.readSync(fd, hb, 0, n, 8) !== n) throw new Error('safetensors: short header read in ' + abs);
        return { path: abs, size: st.size, mtimeMs: st.mtimeMs, header: crypto.createHash('sha256').update(lenBuf).update(hb).digest('hex') };
      } finally {
        fs.closeSync(fd);
      }
    }),
  };
}

function sameSource(a, b) {
  if (!a || !b || !Array.isArray(a.files) || !Array.isArray(b.files) || a.files.length !== b.files.length) return false;
  return a.files.every((f, i) => {
    const g = b.files[i];
    return !!g && f.path === g.path && f.size === g.size && f.mtimeMs === g.mtimeMs && f.header === g.header;
  });
}

function cacheDir(dir, variant) { return path.join(dir, 'v' + QCACHE_VER, variant); }

// writeQuantCache(dir, variant, config, segs, get, {source}): segs = [{name, role, len, kind,
// shape, numel, N, K}] in stream order, get(seg) -> Uint8Array of seg.len bytes, source =
// checkpointIdentity(...) of the checkpoint they came from (null: unknown). chunkSize is for
// tests (a manifest records it; a reader accepts only QCHUNK).
function writeQuantCache(dir, variant, config, segs, get, { chunkSize = QCHUNK, source = null } = {}) {
  const d = cacheDir(dir, variant);
  fs.mkdirSync(d, { recursive: true });
  const mf = path.join(d, 'manifest');
  if (fs.existsSync(mf)) fs.unlinkSync(mf);                      // invalidate first
  let buf = Buffer.alloc(chunkSize), used = 0, idx = 0, off = 0;
  const flush = () => {
    if (!used) return;
    fs.writeFileSync(path.join(d, 'c' + idx), buf.subarray(0, used));
    idx++;
    used = 0;
  };
  const write = (u8) => {
    let src = 0;
    while (src < u8.length) {
      if (used === chunkSize) flush();
      const n = Math.min(chunkSize - used, u8.length - src);
      buf.set(u8.subarray(src, src + n), used);
      used += n;
      src += n;
    }
  };
  const out = [];
  for (const s of segs) {
    const pad = ceil16(off) - off;
    if (pad) { write(new Uint8Array(pad)); off += pad; }
    const bytes = get(s);
    if (bytes.length !== s.len) throw new Error('quant cache: ' + s.name + '.' + s.role + ' has ' + bytes.length + ' bytes, expected ' + s.len);
    out.push({ name: s.name, role: s.role, off, len: s.len, kind: s.kind, shape: s.shape, numel: s.numel, N: s.N, K: s.K });
    write(bytes);
    off += s.len;
  }
  flush();
  const manifest = { ver: QCACHE_VER, variant, qgroup: QGROUP, chunkSize, nChunks: idx, totalBytes: off,
    config: configKey(config), source: source || null, segs: out };
  fs.writeFileSync(mf + '.tmp', JSON.stringify(manifest));
  fs.renameSync(mf + '.tmp', mf);                                 // the commit point
  return manifest;
}

// the manifest of a usable cache for (variant, config), or null; with a source (the
// checkpoint the caller would otherwise load) the manifest must record the same one
// (chunkSize: tests only)
function readManifest(dir, variant, config, { chunkSize = QCHUNK, source = null } = {}) {
  let m;
  try { m = JSON.parse(fs.readFileSync(path.join(cacheDir(dir, variant), 'manifest'), 'utf8')); } catch (_) { return null; }
  if (!m || m.ver !== QCACHE_VER || m.variant !== variant || m.qgroup !== QGROUP || m.chunkSize !== chunkSize) return null;
  const want = configKey(config);
  for (const k in want) if (!m.config || m.config[k] !== want[k]) return null;
  if (!Array.isArray(m.segs)) return null;
  if (source && !sameSource(source, m.source)) return null;
  return m;
}

// readQuantCache(dir, variant, config, put, {onProgress, check, source}) -> false when there
// is no usable cache, else true after every segment's bytes went to put(seg, offset, bytes).
// check(seg) may reject a manifest whose segments do not fit the caller's buffers (it
// throws); chunks are read one at a time (peak host memory: one chunk). chunkSize: tests.
function readQuantCache(dir, variant, config, put, { onProgress, check, chunkSize = QCHUNK, source = null } = {}) {
  const m = readManifest(dir, variant, config, { chunkSize, source });
  if (!m) return false;
  if (check) for (const s of m.segs) check(s);
  const d = cacheDir(dir, variant);
  let first = 0;
  for (let c = 0; c < m.nChunks; c++) {
    const u8 = fs.readFileSync(path.join(d, 'c' + c));
    const c0 = c * m.chunkSize, c1 = c0 + u8.length;
    if (c + 1 < m.nChunks ? u8.length !== m.chunkSize : c1 !== m.totalBytes) throw new Error('quant cache: chunk ' + c + ' has ' + u8.length + ' bytes');
    while (first < m.segs.length && m.segs[first].off + m.segs[first].len <= c0) first++;
    for (let i = first; i < m.segs.length; i++) {
      const s = m.segs[i];
      if (s.off >= c1) break;
      const a = Math.max(s.off, c0), b = Math.min(s.off + s.len, c1);
      if (b > a) put(s, a - s.off, u8.subarray(a - c0, b - c0));
    }
    if (onProgress) onProgress({ phase: 'parse', pct: Math.round((c + 1) / m.nChunks * 100) });
  }
  return true;
}

function dropQuantCache(dir, variant) {
  const mf = path.join(cacheDir(dir, variant), 'manifest');
  if (fs.existsSync(mf)) fs.unlinkSync(mf);
}

module.exports = { writeQuantCache, readQuantCache, readManifest, dropQuantCache, configKey, cacheDir, checkpointIdentity,
  sameSource, QCHUNK, QGROUP, QCACHE_VER };
