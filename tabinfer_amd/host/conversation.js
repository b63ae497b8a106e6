'use strict';
// conversation.js — the multi-round chat driver behind runConversation
// (models/qwen3.js:5397-5522 defines the contract kept here: the emit event types and
// their payload fields, the tool-call id format call_<round>_<k>, Hermes <tool_call> /
// <tool_response> text for re-prefill, at most 8 rounds when tools are offered).
//
// The driver knows nothing about the model. The caller hands it
//   encode(messages) -> ids          the chat template over the running transcript
//   stream(ids, onText) -> Promise    prefill + decode of one assistant turn, the decoded
//                                     text arriving in pieces through onText
//   hooks.beforeFirst(ids) / hooks.afterFirst(ids)   prefix-cache bookkeeping around round 0
//   runTool(name, args, convId, signal) -> {result, artifacts}   (optional)
// and it turns each assistant turn into events. A turn is handled in four steps:
//   1. stream    — the turn's text through a splitter (<think>, <tool_call>, plain text);
//   2. settle    — the turn's outcome: the answer text, the parsed calls, and a notice when
//                  the turn would otherwise be blank;
//   3. publish   — the outcome's events, in the order the UI consumes them;
//   4. act       — each call through the tool runner, its result appended to the transcript.
// The transcript only ever grows by rendered messages (renderMessage), so the next round's
// prompt extends the previous one and the decoder's prefix cache reuses its KV rows.

const MAX_TOOL_ROUNDS = 8;
const ERROR_PREFIX = 'Qwen3 dense: ';

// ---- the Hermes template (the text Qwen3's chat format was trained on) --------------------
function toolPreamble(tools) {
  const fns = (tools || []).filter((t) => t && t.type === 'function' && t.function);
  if (!fns.length) return '';
  const sigs = fns.map((t) => JSON.stringify({ type: 'function', function: t.function })).join('\n');
  return ['# Tools', '', 'You may call one or more functions to assist with the user query.', '',
    'You are provided with function signatures within <tools></tools> XML tags:', '<tools>', sigs, '</tools>', '',
    'For each function call, return a json object with function name and arguments within <tool_call></tool_call> XML tags:',
    '<tool_call>', '{"name": <function-name>, "arguments": <args-json-object>}', '</tool_call>'].join('\n');
}

// One chat message as plain text for the text-only encoder: tool results become a user
// turn in <tool_response>, an assistant turn's calls are appended as <tool_call> blocks.
function renderMessage(m) {
  let c = m.content;
  if (Array.isArray(c)) c = c.filter((p) => p && p.type === 'text').map((p) => p.text || '').join('\n');
  c = c == null ? '' : String(c);
  if (m.role === 'tool') return { role: 'user', content: '<tool_response>\n' + c + '\n</tool_response>' };
  if (m.role === 'assistant' && Array.isArray(m.tool_calls) && m.tool_calls.length) {
    const tc = m.tool_calls.map((t) => '<tool_call>\n{"name": "' + ((t.function && t.function.name) || '') + '", "arguments": ' +
      ((t.function && t.function.arguments) || '{}') + '}\n</tool_call>').join('\n');
    c = c ? c + '\n' + tc : tc;
  }
  return { role: m.role, content: c };
}

// ---- step 1: the streamed text, split three ways -------------------------------------------
// Text outside any tag goes to onContent, text inside <think>...</think> to onReasoning,
// a <tool_call>...</tool_call> body is kept whole in toolCalls. A tail the length of the
// longest tag is held back, so a tag split across two pieces is still found.
function makeRoundParser(onReasoning, onContent) {
  const p = { state: 'content', content: '', reasoning: '', toolCalls: [], buf: '' };
  const OPEN_T = '<think>', CLOSE_T = '</think>', OPEN_C = '<tool_call>', CLOSE_C = '</tool_call>';
  p.push = (text) => {
    p.buf += text;
    for (;;) {
      if (p.state === 'think') {
        const i = p.buf.indexOf(CLOSE_T);
        if (i < 0) { const keep = Math.max(0, p.buf.length - CLOSE_T.length); if (keep) { onReasoning(p.buf.slice(0, keep)); p.reasoning += p.buf.slice(0, keep); p.buf = p.buf.slice(keep); } return; }
        if (i) { onReasoning(p.buf.slice(0, i)); p.reasoning += p.buf.slice(0, i); }
        p.buf = p.buf.slice(i + CLOSE_T.length); p.state = 'content';
      } else if (p.state === 'tool') {
        const i = p.buf.indexOf(CLOSE_C);
        if (i < 0) return;
        p.toolCalls.push(p.buf.slice(0, i).trim()); p.buf = p.buf.slice(i + CLOSE_C.length); p.state = 'content';
      } else {
        const it = p.buf.indexOf(OPEN_T), ic = p.buf.indexOf(OPEN_C);
        const i = it < 0 ? ic : (ic < 0 ? it : Math.min(it, ic));
        if (i < 0) { const keep = Math.max(0, p.buf.length - OPEN_C.length); if (keep) { onContent(p.buf.slice(0, keep)); p.content += p.buf.slice(0, keep); p.buf = p.buf.slice(keep); } return; }
        if (i) { onContent(p.buf.slice(0, i)); p.content += p.buf.slice(0, i); }
        if (i === it) { p.buf = p.buf.slice(i + OPEN_T.length); p.state = 'think'; } else { p.buf = p.buf.slice(i + OPEN_C.length); p.state = 'tool'; }
      }
    }
  };
  p.flush = () => {
    if (p.buf) { if (p.state === 'think') { onReasoning(p.buf); p.reasoning += p.buf; } else if (p.state === 'content') { onContent(p.buf); p.content += p.buf; } }
    p.buf = '';
  };
  return p;
}

// ---- step 2: what a finished turn amounts to -------------------------------------------------
// A <tool_call> body is a call when it is a JSON object with a non-empty name; its arguments
// travel as a JSON string ({} when absent). The id numbers every body of the turn, parsed or
// not, so ids stay stable against the raw text.
function parseToolCall(body, round, k) {
  let obj = null;
  try { obj = JSON.parse(body); } catch (_) { return null; }
  if (!obj || typeof obj !== 'object' || !obj.name) return null;
  return { id: 'call_' + round + '_' + k, type: 'function', function: { name: obj.name, arguments: JSON.stringify(obj.arguments || {}) } };
}

function blankTurnNotice(cutInReasoning, ctxLimit) {
  if (cutInReasoning) {
    return '⚠️ No reply: the ' + ctxLimit + '-token context filled up while the model was still reasoning. ' +
      'Open a new chat, drop a long earlier message (a large tool output, say), or give the provider a larger **Context size**.';
  }
  return '⚠️ The model returned nothing for this turn. Send the message again, or open a new chat if the history is long.';
}

// The turn's outcome. A turn is never blank: no answer and no call gets a notice as its
// answer, worded by whether the turn ended inside its reasoning (the context ran out).
function settleTurn(split, round, ctxLimit) {
  const calls = split.toolCalls.map((body, k) => parseToolCall(body, round, k)).filter(Boolean);
  let answer = split.content.replace(/^\s+/, '');
  let notice = null;
  if (!answer && !calls.length) {
    notice = blankTurnNotice(split.state === 'think' || split.reasoning.length > 0, ctxLimit);
    answer = notice;
  }
  return { answer, calls, notice };
}

// ---- step 3: events ----------------------------------------------------------------------------
// The event sink. `status(null)` clears the host's status line; the first streamed piece of
// a round clears it once.
function eventSink(emit) {
  let cleared = false;
  const sink = {
    beginRound() { cleared = false; emit({ type: 'round_start' }); },
    status(message) { emit({ type: 'info', message }); },
    piece(field, text) {
      if (!cleared) { cleared = true; sink.status(null); }
      emit({ type: 'delta', delta: { [field]: text } });
    },
    raw: emit,
  };
  return sink;
}

// The events that close a turn, in order: the notice (as content), the calls (as one
// tool_calls delta), round_end, usage (the prompt's exact token count), message_added.
function turnEvents(outcome, promptTokens) {
  const evs = [];
  if (outcome.notice) evs.push({ type: 'delta', delta: { content: outcome.notice } });
  if (outcome.calls.length) {
    const tool_calls = outcome.calls.map((c, index) => ({ index, id: c.id, type: c.type, function: { name: c.function.name, arguments: c.function.arguments } }));
    evs.push({ type: 'delta', delta: { tool_calls } });
  }
  evs.push({ type: 'round_end', content: outcome.answer });
  evs.push({ type: 'usage', usage: { prompt_tokens: promptTokens, total_tokens: promptTokens } });
  evs.push({ type: 'message_added', message: assistantMessage(outcome) });
  return evs;
}

function assistantMessage(outcome) {
  const m = { role: 'assistant', content: outcome.answer };
  if (outcome.calls.length) m.tool_calls = outcome.calls;
  return m;
}

// ---- step 4: tools -----------------------------------------------------------------------------
const isAbort = (e) => !!e && e.name === 'AbortError';
function abortError() { const e = new Error('aborted'); e.name = 'AbortError'; return e; }
function throwIfAborted(signal) { if (signal && signal.aborted) throw abortError(); }

// One call through the runner: its text result (the error text when the runner throws;
// an abort propagates) and artifacts.
async function invokeTool(runTool, call, convId, signal) {
  let args = {};
  try { args = JSON.parse(call.function.arguments || '{}'); } catch (_) { args = {}; }
  try {
    const r = await runTool(call.function.name, args, convId, signal);
    return { text: r && r.result != null ? r.result : '', artifacts: r && r.artifacts };
  } catch (e) {
    if (isAbort(e)) throw e;
    return { text: 'Error: ' + ((e && e.message) || e), artifacts: undefined };
  }
}

// ---- the driver --------------------------------------------------------------------------------
// opts: {transcript (rendered messages, grows in place), toolsOffered, maxTokens, ctxLimit,
//        convId, signal}; deps: {encode, stream, runTool, hooks}. Resolves after agent_done;
// rejects only with an AbortError.
async function converse(opts, deps, emit) {
  const { transcript, toolsOffered, ctxLimit, convId, signal } = opts;
  const { encode, stream, runTool, hooks = {} } = deps;
  const ev = eventSink(emit);
  const rounds = toolsOffered ? MAX_TOOL_ROUNDS : 1;
  try {
    for (let round = 0; round < rounds; round++) {
      throwIfAborted(signal);
      ev.beginRound();
      const split = makeRoundParser((t) => ev.piece('reasoning', t), (t) => ev.piece('content', t));
      const ids = encode(transcript);
      if (round === 0 && hooks.beforeFirst) hooks.beforeFirst(ids);
      await stream(ids, (piece) => split.push(piece));
      if (round === 0 && hooks.afterFirst) hooks.afterFirst(ids);
      split.flush();
      throwIfAborted(signal);
      ev.status(null);
      const outcome = settleTurn(split, round, ctxLimit);
      for (const e of turnEvents(outcome, ids.length)) ev.raw(e);
      transcript.push(renderMessage(assistantMessage(outcome)));
      if (!outcome.calls.length) break;
      if (!runTool) { ev.status(null); break; }
      for (const call of outcome.calls) {
        throwIfAborted(signal);
        ev.raw({ type: 'tool_started', tc: call });
        const res = await invokeTool(runTool, call, convId, signal);
        ev.raw({ type: 'tool_result', id: call.id, result: res.text, artifacts: res.artifacts });
        const toolMsg = { role: 'tool', tool_call_id: call.id, content: res.text };
        transcript.push(renderMessage(toolMsg));
        ev.raw({ type: 'message_added', message: toolMsg });
      }
    }
  } catch (e) {
    if (isAbort(e)) throw e;
    ev.status(null);
    ev.raw({ type: 'error', message: ERROR_PREFIX + ((e && e.message) || e) });
  }
  ev.raw({ type: 'agent_done' });
}

module.exports = {
  converse, makeRoundParser, settleTurn, parseToolCall, turnEvents, toolPreamble, renderMessage, abortError,
  MAX_TOOL_ROUNDS, ERROR_PREFIX,
};
