'use strict';
// Qwen3's tokenizer from a local tokenizer.json (models/qwen3.js:3227-3320): byte-level BPE
// behind the checkpoint's Split pre-tokenizer, and the ChatML prompt with the special ids
// spliced in. Node.js, no dependencies; the host's loadModel({tokenizer: path}) uses it.
//
//   const tok = loadTokenizer('/models/Qwen3-0.6B');        // a directory or the file itself
//   tok.encodeText('Hello world') -> ids    tok.decode(ids) -> string
//   tok.encodeChat([{role, content}], {addGenerationPrompt}) -> ids    tok.isStop(id)
//
// The algorithm is the tokenizer format's own (GPT-2's byte-level BPE as Hugging Face
// tokenizers runs it): the text is split by the pre-tokenizer's regex; each piece's UTF-8
// bytes become visible characters through the byte map; the lowest-ranked adjacent pair
// is merged, leftmost first, until no ranked pair is left; each symbol is a vocabulary id.
const fs = require('fs');
const path = require('path');

// Qwen2/Qwen3's pre-tokenizer pattern (their tokenizer.json), for files that carry none
const QWEN_SPLIT = "(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\\r\\n\\p{L}\\p{N}]?\\p{L}+|\\p{N}| ?[^\\s\\p{L}\\p{N}]+[\\r\\n]*|\\s*[\\r\\n]+|\\s+(?!\\S)|\\s+";

// A tokenizer.json regex as a JS RegExp: JS has no inline (?i:...) group, so inside one
// every ASCII letter outside an escape becomes a two-case class ([sS]).
function jsRegex(pattern) {
  let out = '';
  let i = 0;
  while (i < pattern.length) {
    if (pattern.startsWith('(?i:', i)) {
      let depth = 1, j = i + 4, body = '';
      for (; j < pattern.length && depth > 0; j++) {
        const ch = pattern[j];
        if (ch === '\\') { body += ch + pattern[j + 1]; j++; continue; }
        if (ch === '(') depth++;
        else if (ch === ')') { depth--; if (depth === 0) break; }
        body += ch;
      }
      let folded = '';
      for (let k = 0; k < body.length; k++) {
        const ch = body[k];
        if (ch === '\\') { folded += ch + body[k + 1]; k++; continue; }
        folded += /[A-Za-z]/.test(ch) ? '[' + ch.toLowerCase() + ch.toUpperCase() + ']' : ch;
      }
      out += '(?:' + folded + ')';
      i = j + 1;
    } else if (pattern[i] === '\\') {
      out += pattern[i] + pattern[i + 1];
      i += 2;
    } else {
      out += pattern[i++];
    }
  }
  return new RegExp(out, 'gu');
}

// GPT-2's reversible byte -> character map: the printable Latin-1 bytes stand for
// themselves, the other 68 bytes take the characters from U+0100 upward, in byte order.
function byteMaps() {
  const keep = (b) => (b >= 0x21 && b <= 0x7e) || (b >= 0xa1 && b <= 0xac) || (b >= 0xae && b <= 0xff);
  const enc = new Array(256), dec = new Map();
  let extra = 0;
  for (let b = 0; b < 256; b++) {
    const ch = String.fromCharCode(keep(b) ? b : 256 + extra++);
    enc[b] = ch;
    dec.set(ch, b);
  }
  return { enc, dec };
}

// the Split pattern of the file's pre-tokenizer (a Split alone or inside a Sequence)
function splitPattern(pre) {
  if (!pre) return null;
  if (pre.type === 'Split' && pre.pattern) return pre.pattern.Regex || null;
  if (pre.type === 'Sequence') {
    for (const p of pre.pretokenizers || []) { const r = splitPattern(p); if (r) return r; }
  }
  return null;
}

function createTokenizer(json) {
  const j = typeof json === 'string' ? JSON.parse(json) : json;
  if (!j || !j.model || j.model.type !== 'BPE') throw new Error('tokenizer: a BPE tokenizer.json is required');
  const vocab = new Map(Object.entries(j.model.vocab));
  const idToTok = new Map();
  for (const [t, id] of vocab) idToTok.set(id, t);
  const special = new Map();                 // added-token content -> id
  for (const a of j.added_tokens || []) { special.set(a.content, a.id); vocab.set(a.content, a.id); idToTok.set(a.id, a.content); }
  const ranks = new Map();
  (j.model.merges || []).forEach((m, r) => {
    const [a, b] = Array.isArray(m) ? m : (() => { const i = m.indexOf(' ', 1); return [m.slice(0, i), m.slice(i + 1)]; })();
    ranks.set(a + '\u0000' + b, r);
  });
  const re = jsRegex(splitPattern(j.pre_tokenizer) || QWEN_SPLIT);
  const { enc: byteEnc, dec: byteDec } = byteMaps();
  const utf8 = new TextEncoder(), text = new TextDecoder();
  const cache = new Map();

  // the symbols of one byte-mapped piece after every ranked merge
  function bpe(piece) {
    const hit = cache.get(piece);
    if (hit) return hit;
    let w = Array.from(piece);
    while (w.length > 1) {
      let best = -1, bestRank = Infinity;
      for (let i = 0; i + 1 < w.length; i++) {
        const r = ranks.get(w[i] + '\u0000' + w[i + 1]);
        if (r !== undefined && r < bestRank) { bestRank = r; best = i; }
      }
      if (best < 0) break;
      w = w.slice(0, best).concat([w[best] + w[best + 1]], w.slice(best + 2));
    }
    if (cache.size < 65536) cache.set(piece, w);
    return w;
  }

  function encodeText(s) {
    const ids = [];
    for (const piece of String(s).match(re) || []) {
      let mapped = '';
      for (const b of utf8.encode(piece)) mapped += byteEnc[b];
      for (const sym of bpe(mapped)) {
        const id = vocab.get(sym);
        if (id !== undefined) ids.push(id);
      }
    }
    return ids;
  }

  const idOf = (content) => {
    const id = special.get(content);
    if (id === undefined) throw new Error('tokenizer: no special token ' + content);
    return id;
  };
  const IM_START = special.has('<|im_start|>') ? special.get('<|im_start|>') : null;
  const IM_END = special.has('<|im_end|>') ? special.get('<|im_end|>') : null;
  const EOT = special.has('<|endoftext|>') ? special.get('<|endoftext|>') : null;

  // ChatML: <|im_start|>role\ncontent<|im_end|>\n per message, then <|im_start|>assistant\n
  function encodeChat(messages, { addGenerationPrompt = true } = {}) {
    const start = idOf('<|im_start|>'), end = idOf('<|im_end|>');
    const ids = [];
    for (const m of messages || []) {
      ids.push(start);
      for (const t of encodeText(m.role + '\n' + (typeof m.content === 'string' ? m.content : ''))) ids.push(t);
      ids.push(end);
      for (const t of encodeText('\n')) ids.push(t);
    }
    if (addGenerationPrompt) {
      ids.push(start);
      for (const t of encodeText('assistant\n')) ids.push(t);
    }
    return ids;
  }

  // ids -> text: each id's symbols back to bytes, decoded as UTF-8 (characters outside the
  // byte map are dropped)
  function decode(ids) {
    const bytes = [];
    for (const id of ids) {
      const t = idToTok.get(id);
      if (t === undefined) continue;
      for (const ch of t) { const b = byteDec.get(ch); if (b !== undefined) bytes.push(b); }
    }
    return text.decode(Uint8Array.from(bytes));
  }

  // streamed output: each token's bytes through one streaming UTF-8 decoder, so a character
  // whose bytes span two tokens is emitted once whole (push(id) -> the text completed by id)
  function streamDecoder() {
    const sd = new TextDecoder();
    return {
      push(id) {
        const t = idToTok.get(id);
        if (t === undefined) return '';
        const bytes = [];
        for (const ch of t) { const b = byteDec.get(ch); if (b !== undefined) bytes.push(b); }
        return sd.decode(Uint8Array.from(bytes), { stream: true });
      },
      flush() { return sd.decode(); },
    };
  }

  return {
    encodeText, encodeChat, decode, streamDecoder,
    isStop: (id) => id === IM_END || id === EOT,   // models/qwen3.js:4534
    specialIds: () => new Set(special.values()),
    imStart: IM_START, imEnd: IM_END, endOfText: EOT,
    vocabSize: () => idToTok.size,
  };
}

// loadTokenizer(dirOrFile): tokenizer.json from a local checkpoint directory
function loadTokenizer(where) {
  const file = fs.existsSync(where) && fs.statSync(where).isDirectory() ? path.join(where, 'tokenizer.json') : where;
  return createTokenizer(fs.readFileSync(file, 'utf8'));
}

module.exports = { createTokenizer, loadTokenizer, jsRegex, byteMaps, QWEN_SPLIT };
