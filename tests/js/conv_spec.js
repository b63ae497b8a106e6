'use strict';
// CPU checks of the conversation driver (tabinfer_amd/host/conversation.js) with a scripted
// model in place of the decoder: node tests/js/conv_spec.js <out.json>
// Each case scripts the text pieces of every assistant turn and records the events, the
// prompts the driver encoded and what the tool runner saw.
const fs = require('fs');
const path = require('path');
const CONV = require(path.join(__dirname, '..', '..', 'tabinfer_amd', 'host', 'conversation.js'));

// encode: one "token" per character of the rendered transcript, so prompt lengths are checkable
const encode = (msgs) => Array.from(msgs.map((m) => '<' + m.role + '>' + m.content).join('|'));

async function run(name, turns, { tools = true, runner, transcript, signal, streamError } = {}) {
  const events = [], prompts = [], toolCalls = [];
  let round = 0;
  const deps = {
    encode: (msgs) => { prompts.push(msgs.map((m) => ({ role: m.role, content: m.content }))); return encode(msgs); },
    stream: async (ids, onText) => {
      if (streamError && round === streamError.round) { round++; throw new Error(streamError.message); }
      const pieces = turns[Math.min(round, turns.length - 1)];
      round++;
      for (const p of pieces) onText(p);
    },
    runTool: runner === null ? null : (runner || (async (n, a) => { toolCalls.push({ n, a }); return { result: 'R' + toolCalls.length }; })),
    hooks: { beforeFirst: (ids) => events.push({ type: '_before', n: ids.length }), afterFirst: (ids) => events.push({ type: '_after', n: ids.length }) },
  };
  let rejected = null;
  try {
    await CONV.converse({ transcript: transcript || [{ role: 'user', content: 'hi' }], toolsOffered: tools, ctxLimit: 4096, convId: 'c1', signal }, deps,
      (e) => events.push(JSON.parse(JSON.stringify(e))));
  } catch (e) { rejected = e.name + ': ' + e.message; }
  return { name, events, prompts, toolCalls, rejected };
}

(async () => {
  const out = [];
  // a plain answer, tags split across pieces, reasoning streamed apart from the content
  out.push(await run('plain', [['<thi', 'nk>why', ' so</th', 'ink>\n\nHel', 'lo', ' world']], { tools: false }));
  // a tool round: one valid call and one body that is not JSON, then an answer
  out.push(await run('tool', [
    ['<tool_call>\n{"name": "get_time", "arguments": {"tz": "UTC"}}\n</tool_call>', '<tool_call>not json</tool_call>'],
    ['It is noon.'],
  ]));
  // the runner throws: the error text becomes the tool result
  out.push(await run('tool_error', [['<tool_call>{"name": "f"}</tool_call>'], ['ok']],
    { runner: async () => { throw new Error('boom'); } }));
  // calls but no runner: the conversation stops after the first round
  out.push(await run('no_runner', [['<tool_call>{"name": "f", "arguments": {}}</tool_call>']], { runner: null }));
  // blank turns: nothing at all; reasoning cut off by the context
  out.push(await run('blank', [[]], { tools: false }));
  out.push(await run('cut_in_think', [['<think>step one', ' step two']], { tools: false }));
  // a model that always calls: 8 rounds at most
  out.push(await run('round_cap', [['<tool_call>{"name": "again", "arguments": {"i": 1}}</tool_call>']]));
  // the stream fails in round 1: error event, then agent_done
  out.push(await run('stream_error', [['<tool_call>{"name": "f"}</tool_call>'], ['x']], { streamError: { round: 1, message: 'device lost' } }));
  // an aborted signal rejects with AbortError and emits no agent_done
  out.push(await run('aborted', [['x']], { signal: { aborted: true } }));
  // the transcript grows by rendered messages: assistant calls and tool results as text
  out.push(await run('transcript', [['<tool_call>{"name": "f", "arguments": {"a": [1, 2]}}</tool_call>'], ['done']],
    { transcript: [{ role: 'system', content: 'S' }, { role: 'user', content: 'q' }] }));
  // parseToolCall on its own: ids number every body, arguments default to {}
  const parsed = [CONV.parseToolCall('{"name": "a"}', 2, 3), CONV.parseToolCall('{"arguments": {}}', 0, 0),
    CONV.parseToolCall('[1]', 0, 0), CONV.parseToolCall('{"name": "b", "arguments": {"x": "y"}}', 1, 0)];
  fs.writeFileSync(process.argv[2], JSON.stringify({ cases: out, parsed }));
})().catch((e) => { console.error(e); process.exit(1); });
