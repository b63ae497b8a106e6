'use strict';
// CPU-side checks of the JS host (no GPU needed):
//   node tests/js/cpu_checks.js <dir>
// reads <dir>/f32.bin (float32 values) and <dir>/tiny.safetensors, writes <dir>/out.json with
// the addon's exports, both f32 -> f16 converters over the values, the parsed safetensors
// header, the error raised by a call without a context, and the conversation's text renderings.
const fs = require('fs');
const path = require('path');
const HOST = path.join(__dirname, '..', '..', 'tabinfer_amd', 'host');
const eng = require(path.join(HOST, 'ti-engine.js'));
const { readSafetensorsHeader, toolPreamble, renderMessage } = require(path.join(HOST, 'qwen3-host.js'));

const dir = process.argv[2];
const raw = fs.readFileSync(path.join(dir, 'f32.bin'));
const f = new Float32Array(raw.buffer, raw.byteOffset, raw.length / 4);
const q3 = new Array(f.length), en = new Array(f.length);
for (let i = 0; i < f.length; i++) { q3[i] = eng.f32ToF16(f[i]); en[i] = eng.engineF32ToF16(f[i]); }
const bf = new Uint16Array(f.length);
const u = new Uint32Array(f.buffer.slice(f.byteOffset, f.byteOffset + f.length * 4));
for (let i = 0; i < f.length; i++) bf[i] = u[i] >>> 16;
let ctxError = null;
try { eng.TI.gemv_q4_q8(null, null, null, null, null, null, 1, 32, 0); } catch (e) { ctxError = e.constructor.name + ': ' + e.message; }
let initError = null;
try { const c = eng.TI.init(0); eng.TI.shutdown(c); } catch (e) { initError = { message: e.message, code: e.code }; }
const out = {
  exports: Object.keys(eng.TI).sort(),
  version: eng.TI.version(),
  f16_q3: q3, f16_eng: en, bf16_to_f16: Array.from(eng.bf16ToF16bits(bf)),
  header: readSafetensorsHeader(path.join(dir, 'tiny.safetensors')),
  ctxError, initError,
  preamble: toolPreamble([{ type: 'function', function: { name: 'get_time', parameters: { type: 'object', properties: {} } } },
    { type: 'other' }]),
  preambleNone: toolPreamble([]),
  rendered: [renderMessage({ role: 'tool', content: '42' }),
    renderMessage({ role: 'assistant', content: 'ok', tool_calls: [{ function: { name: 'f', arguments: '{"a":1}' } }] }),
    renderMessage({ role: 'user', content: [{ type: 'text', text: 'a' }, { type: 'image' }, { type: 'text', text: 'b' }] })],
};
fs.writeFileSync(path.join(dir, 'out.json'), JSON.stringify(out));
