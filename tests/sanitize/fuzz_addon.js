'use strict';
// The N-API addon's argument marshalling under AddressSanitizer / UBSan, CPU only:
//   LD_PRELOAD=<libasan> node fuzz_addon.js <addon.node> <iterations> <seed>
// with the addon built with -fsanitize=address,undefined. Without a GPU every entry point
// that needs a device must end in a JS exception; the container entry points (cpubin_*)
// run for real. Checked: every export called with wrong argument counts and types (numbers
// out of range, NaN, BigInt, strings, typed arrays of every kind, detached and empty
// buffers, objects posing as handles); container handles used after close, closed twice,
// and views read after their container was closed. Any outcome other than a return value
// or a thrown Error is a failure; a sanitizer report aborts the process.
const path = require('path');
const T = require(path.resolve(process.argv[2]));
const iters = +(process.argv[3] || 2000);
let s = BigInt(process.argv[4] || 1) * 0x9E3779B97F4A7C15n & 0xFFFFFFFFFFFFFFFFn;
const rnd = () => { s ^= s << 13n; s &= 0xFFFFFFFFFFFFFFFFn; s ^= s >> 7n; s ^= s << 17n; s &= 0xFFFFFFFFFFFFFFFFn; return Number(s >> 11n) / 2 ** 53; };
const pick = (a) => a[Math.floor(rnd() * a.length)];

// a small valid container: one tensor of each kind
function container() {
  const hdr = JSON.stringify({ G: 64, tensors: {
    t: { kind: 'tern', N: 2, K: 64, codesOff: 0, codesLen: 32, scalesOff: 32, scalesLen: 8 },
    e: { kind: 'embed_f16', shape: [3, 4], off: 48, len: 24 },
    f: { kind: 'f32', shape: [4], off: 80, len: 16 } } });
  const b = Buffer.alloc(4 + hdr.length + 96);
  b.writeUInt32LE(hdr.length, 0);
  b.write(hdr, 4, 'utf8');
  for (let i = 4 + hdr.length; i < b.length; i++) b[i] = (i * 37) & 0xff;
  return new Uint8Array(b.buffer, b.byteOffset, b.length);
}

const detached = () => { const ab = new ArrayBuffer(16); try { structuredClone(ab, { transfer: [ab] }); } catch (_) { /* no structuredClone */ } return ab; };
const values = () => [
  undefined, null, true, 0, -1, 1, 7, 1.5, NaN, Infinity, -Infinity, 2 ** 31, -(2 ** 31) - 1, 2 ** 53, 2 ** 63, -(2 ** 63),
  1e308, 3n, -1n, 2n ** 64n, '', 'x', 'model.norm.weight', '\u0000', {}, [], [1, 2], () => 0, Symbol('s'),
  new Float32Array(0), new Float32Array(5), new Int32Array(3), new Uint16Array(8), new Uint8Array(1), new Int8Array(4),
  new Float64Array(2), new BigInt64Array(1), new ArrayBuffer(0), new ArrayBuffer(64), detached(),
  new DataView(new ArrayBuffer(8)), container(),
];

let calls = 0, threw = 0;
function call(name, args) {
  calls++;
  try { T[name](...args); } catch (e) {
    if (!(e instanceof Error)) { console.error('FAIL', name, 'threw a non-Error', e); process.exit(1); }
    threw++;
  }
}

const names = Object.keys(T).filter((k) => typeof T[k] === 'function');
// every export with no arguments, with one of each value, and with random lists
for (const n of names) {
  call(n, []);
  for (const v of values()) call(n, [v]);
}
for (let it = 0; it < iters; it++) {
  const n = pick(names);
  const k = Math.floor(rnd() * 12);
  const pool = values();
  const args = Array.from({ length: k }, () => pick(pool));
  call(n, args);
}

// container handles: valid use, use after close, double close, views outliving the handle
const c = T.cpubin_parse(container());
const sum = T.cpubin_summary(c);
if (!sum || sum.tensors !== 3 || sum.groupSize !== 64 || sum.blobBytes !== 96) { console.error('FAIL summary', sum); process.exit(1); }
const mustThrow = (name, args) => {
  let ok = false;
  try { T[name](...args); } catch (e) { ok = e instanceof Error; }
  if (!ok) { console.error('FAIL', name, 'did not throw'); process.exit(1); }
};
for (let i = 0; i < 3; i++) T.cpubin_tensor(c, T.cpubin_name(c, i));
mustThrow('cpubin_name', [c, 3]);
mustThrow('cpubin_name', [c, -1]);
mustThrow('cpubin_embed_row', [c, 'e', 3, 4]);
mustThrow('cpubin_embed_row', [c, 'e', 2 ** 62, 4]);
mustThrow('cpubin_embed_row', [c, 'e', 0, 5]);
mustThrow('cpubin_tensor', [c, 'nope']);
const row = T.cpubin_embed_row(c, 'e', 2, 4);
if (!(row instanceof Float32Array) || row.length !== 4) { console.error('FAIL embed_row', row); process.exit(1); }
const view = T.cpubin_tensor(c, 'f');
T.cpubin_close(c);
call('cpubin_close', [c]);            // a second close: a no-op or an Error, never a double free
mustThrow('cpubin_summary', [c]);
mustThrow('cpubin_name', [c, 0]);
mustThrow('cpubin_tensor', [c, 'f']);
mustThrow('cpubin_embed_row', [c, 'e', 0, 4]);
// a view taken before the close is still readable (it must own or keep its bytes)
const readView = (v) => {
  if (!v) return;
  for (const key of Object.keys(v)) {
    const x = v[key];
    if (ArrayBuffer.isView(x)) { let t = 0; for (let i = 0; i < x.length; i++) t += Number(x[i]); }
    else if (x instanceof ArrayBuffer) { const u = new Uint8Array(x); let t = 0; for (let i = 0; i < u.length; i++) t += u[i]; }
  }
};
readView(view);
if (global.gc) global.gc();
console.log(JSON.stringify({ ok: true, exports: names.length, calls, threw }));
