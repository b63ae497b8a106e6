'use strict';
// node tests/js/tok_spec.js <spec.json>: {tokenizer: path, texts: [..], chats: [[messages]]}
// -> stdout JSON {ids: [[..]], dec: [..], chat: [[..]], stop: [ids that isStop]}
const fs = require('fs');
const path = require('path');
const { loadTokenizer } = require(path.join(__dirname, '..', '..', 'tabinfer_amd', 'host', 'tokenizer.js'));
const spec = JSON.parse(fs.readFileSync(process.argv[2], 'utf8'));
const tok = loadTokenizer(spec.tokenizer);
const ids = spec.texts.map((t) => tok.encodeText(t));
const out = {
  ids,
  dec: ids.map((x) => tok.decode(x)),
  chat: (spec.chats || []).map((m) => tok.encodeChat(m)),
  chatNoGen: (spec.chats || []).map((m) => tok.encodeChat(m, { addGenerationPrompt: false })),
  stream: ids.map((x) => { const sd = tok.streamDecoder(); const parts = x.map((i) => sd.push(i)); parts.push(sd.flush()); return parts; }),
  stop: Array.from({ length: tok.vocabSize() + 8 }, (_, i) => i).filter((i) => tok.isStop(i)),
};
process.stdout.write(JSON.stringify(out));
