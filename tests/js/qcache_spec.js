'use strict';
// node tests/js/qcache_spec.js <dir>: exercises host/quant-cache.js on in-memory segments
// (no GPU) and host/qwen3-host.js's claimSystemBlock; prints one JSON object of results.
const fs = require('fs');
const path = require('path');
const QC = require(path.join(__dirname, '..', '..', 'tabinfer_amd', 'host', 'quant-cache.js'));
const { claimSystemBlock } = require(path.join(__dirname, '..', '..', 'tabinfer_amd', 'host', 'qwen3-host.js'));
const dir = process.argv[2];
const cfg = { layers: 2, hidden: 64, intermediate: 128, n_heads: 4, n_kv_heads: 2, head_dim: 16, vocab: 300 };
let s = 12345;
const rnd = () => { s ^= s << 13; s >>>= 0; s ^= s >>> 17; s ^= s << 5; s >>>= 0; return s; };
const lens = [4096, 512, 1000, 3, 17, 2500, 0, 999, 64, 1, 3001];   // several straddle 1000-byte chunks
const segs = lens.map((len, i) => ({ name: 't' + i, role: i % 3 === 0 ? 'pack' : i % 3 === 1 ? 'scales' : 'buf',
  len, kind: i % 3 === 2 ? 'f16' : 'int4', shape: [len], numel: len, N: 1, K: len }));
const data = segs.map((g) => Uint8Array.from({ length: g.len }, () => rnd() & 0xff));
const res = {};
const man = QC.writeQuantCache(dir, 'T', cfg, segs, (g) => data[segs.indexOf(g)], { chunkSize: 1000 });
res.manifest = man;
res.files = fs.readdirSync(QC.cacheDir(dir, 'T')).sort();
// read back into fresh buffers
const back = segs.map((g) => new Uint8Array(g.len));
const puts = [];
res.read = QC.readQuantCache(dir, 'T', cfg, (g, off, bytes) => { back[segs.findIndex((x) => x.name === g.name)].set(bytes, off); puts.push([g.name, off, bytes.length]); }, { chunkSize: 1000 });
res.equal = back.every((b, i) => Buffer.compare(Buffer.from(b), Buffer.from(data[i])) === 0);
res.puts = puts;
// the production reader takes 64 MiB chunks only; other geometries, variants, versions: no cache
res.otherChunk = QC.readQuantCache(dir, 'T', cfg, () => { throw new Error('no'); });
res.otherCfg = QC.readQuantCache(dir, 'T', Object.assign({}, cfg, { hidden: 128 }), () => { throw new Error('no'); }, { chunkSize: 1000 });
res.otherVariant = QC.readQuantCache(dir, 'U', cfg, () => { throw new Error('no'); }, { chunkSize: 1000 });
// check() rejects a segment that does not fit
try { QC.readQuantCache(dir, 'T', cfg, () => {}, { chunkSize: 1000, check: (g) => { if (g.name === 't5') throw new Error('t5 does not fit'); } }); res.checkThrew = false; } catch (e) { res.checkThrew = e.message; }
// a truncated chunk is an error, not a silent short read
const c1 = path.join(QC.cacheDir(dir, 'T'), 'c1');
const keep = fs.readFileSync(c1);
fs.writeFileSync(c1, keep.subarray(0, 10));
try { QC.readQuantCache(dir, 'T', cfg, () => {}, { chunkSize: 1000 }); res.truncThrew = false; } catch (e) { res.truncThrew = e.message; }
fs.writeFileSync(c1, keep);
// a write cut short leaves no manifest: the next write removes the old one first
try { QC.writeQuantCache(dir, 'T', cfg, segs, (g) => { if (g.name === 't4') throw new Error('cut'); return data[segs.indexOf(g)]; }, { chunkSize: 1000 }); } catch (_) { /* expected */ }
res.afterCut = QC.readQuantCache(dir, 'T', cfg, () => {}, { chunkSize: 1000 });
// the checkpoint identity: two safetensors files with the same header (a fine-tune of the
// same geometry) are different sources; a cache written from A is read for A or for a load
// from the cache alone, never for B; touching A's modification time makes it a miss too
const st = (name, fill) => {
  const hdr = Buffer.from(JSON.stringify({ w: { dtype: 'F16', shape: [4, 4], data_offsets: [0, 32] } }));
  const len = Buffer.alloc(8); len.writeBigUInt64LE(BigInt(hdr.length));
  const f = path.join(dir, name);
  fs.writeFileSync(f, Buffer.concat([len, hdr, Buffer.alloc(32, fill)]));
  return f;
};
const fa = st('a.safetensors', 1), fb = st('b.safetensors', 2);
const ida = QC.checkpointIdentity([fa]), idb = QC.checkpointIdentity([fb]);
res.ident = { sameHeader: ida.files[0].header === idb.files[0].header, absolute: path.isAbsolute(ida.files[0].path),
  size: ida.files[0].size };
QC.writeQuantCache(dir, 'S', cfg, segs, (g) => data[segs.indexOf(g)], { chunkSize: 1000, source: ida });
const rd = (source) => QC.readQuantCache(dir, 'S', cfg, () => {}, { chunkSize: 1000, source });
res.sourceA = rd(ida);
res.sourceB = rd(idb);
res.sourceNone = rd(null);
res.sourceTwo = rd(QC.checkpointIdentity([fa, fb]));
const later = new Date(Date.now() + 5000);
fs.utimesSync(fa, later, later);
res.sourceTouched = rd(QC.checkpointIdentity([fa]));
res.manifestSource = JSON.parse(fs.readFileSync(path.join(QC.cacheDir(dir, 'S'), 'manifest'), 'utf8')).source;
fs.writeFileSync(path.join(dir, 'bad.safetensors'), Buffer.from([200, 0, 0, 0, 0, 0, 0, 0, 1, 2]));
try { QC.checkpointIdentity([path.join(dir, 'bad.safetensors')]); res.badHeader = false; } catch (e) { res.badHeader = e.message; }
// claimSystemBlock: the reference's conditions
const S = Array.from({ length: 20 }, (_, i) => 100 + i), P = S.concat([7, 8, 9]);
res.claim = [
  claimSystemBlock(P, S, null, S),                  // claim
  claimSystemBlock(P, S, S.concat([1]), S),         // the live cache covers it
  claimSystemBlock(P, S, S.slice(0, 5), S),         // the live cache covers part: claim
  claimSystemBlock([1].concat(P), S, null, S),      // the prompt does not begin with it
  claimSystemBlock(P, S, null, null),               // no anchor
  claimSystemBlock(P, S, null, S.slice(0, 19)),     // anchor of another block
  claimSystemBlock(P, S, null, S.slice(0, 19).concat([0])),
  claimSystemBlock(P.slice(0, 15).concat([1]), S.slice(0, 15), null, S.slice(0, 15)),   // under 16 tokens
  claimSystemBlock(P, null, null, S),
];
process.stdout.write(JSON.stringify(res));
