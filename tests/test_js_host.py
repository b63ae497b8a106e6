"""CPU checks of the JavaScript host (tabinfer_amd/host): the N-API addon loads without a
GPU and exports every entry point of include/ti.h; its two f32 -> f16 converters equal the
oracle's restatements of models/qwen3.js:3357-3374 and engine/webgpu-engine.js:217-236
bit for bit; the safetensors reader parses a file written here; bad handles and a missing
device are JS exceptions."""
import json
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

from tabinfer_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ADDON = os.path.join(ROOT, "tabinfer_amd", "host", "tabinfer.node")
NODE = shutil.which("node")

pytestmark = pytest.mark.skipif(NODE is None, reason="node is not installed")


def write_safetensors(path, tensors):
    """tensors: name -> (dtype string, shape, raw bytes)."""
    hdr, off, blobs = {}, 0, []
    for name, (dt, shape, raw) in tensors.items():
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        off += len(raw)
        blobs.append(raw)
    h = json.dumps(hdr).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def f32_sweep(rng):
    edge = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 65519.996, 1e-8, -1e-8, 6.1e-5, 5.96e-8, 2.98e-8,
                     2.9802322e-08, 8.940697e-08, np.inf, -np.inf, np.nan, 1e30, -3.0e38, 0.33325195, 0.3334961],
                    np.float32)
    # f16 rounding boundaries: the midpoints between neighbouring f16 values, and one ulp either side
    h = rng.integers(0, 0x7bff, 4000).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float32)
    hi = (h + 1).view(np.float16).astype(np.float32)
    mid = ((lo.astype(np.float64) + hi.astype(np.float64)) / 2).astype(np.float32)
    near = np.concatenate([mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(-np.inf))])
    rnd = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    return np.concatenate([edge, near, -near, rnd]).astype(np.float32)


@pytest.fixture(scope="module")
def checks(tmp_path_factory):
    if not os.path.exists(ADDON):
        pytest.fail("tabinfer.node is not built: run python -m tabinfer_amd.build")
    d = tmp_path_factory.mktemp("jscpu")
    vals = f32_sweep(np.random.default_rng(3))
    vals.tofile(str(d / "f32.bin"))
    write_safetensors(str(d / "tiny.safetensors"), {
        "a.weight": ("BF16", (2, 3), np.arange(6, dtype=np.uint16).tobytes()),
        "b": ("F32", (4,), np.ones(4, np.float32).tobytes()),
    })
    r = subprocess.run([NODE, os.path.join(ROOT, "tests", "js", "cpu_checks.js"), str(d)],
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    assert r.returncode == 0, r.stdout
    out = json.load(open(str(d / "out.json")))
    return vals, out


def test_addon_exports_every_entry_point(checks):
    """Every entry point of ti.h that takes a context; the context-free no-allocation
    variant is for callers that cannot allocate, and a JS host always holds a context."""
    _, out = checks
    want = {n[len("ti_"):] for n in abi.header_functions() if not n.endswith("_noalloc")}
    missing = sorted(want - set(out["exports"]))
    assert not missing, missing
    assert out["version"] == abi.lib().ti_version()


def test_js_f16_converters_match_the_oracle(checks, orc):
    vals, out = checks
    q3 = np.array([orc.f32_to_f16_q3(v) for v in vals])
    en = np.array([orc.f32_to_f16_eng(v) for v in vals])
    assert np.array_equal(np.array(out["f16_q3"]), q3)
    assert np.array_equal(np.array(out["f16_eng"]), en)
    # the two converters do differ (ties), so the comparison above can tell them apart
    assert np.any(q3 != en)
    bf = (vals.view(np.uint32) >> 16).astype(np.uint32)
    want = np.array([orc.f32_to_f16_q3(np.uint32(b << 16).view(np.float32)) for b in bf])
    assert np.array_equal(np.array(out["bf16_to_f16"]), want)


def test_safetensors_header(checks):
    _, out = checks
    h = out["header"]
    assert h["a.weight"]["dtype"] == "BF16" and h["a.weight"]["shape"] == [2, 3]
    assert h["b"]["end"] - h["b"]["begin"] == 16
    assert h["b"]["begin"] == h["a.weight"]["end"]


def test_errors_are_exceptions(checks):
    _, out = checks
    assert out["ctxError"].startswith("TypeError") and "context" in out["ctxError"]
    if abi.device_count() == 0:
        assert out["initError"]["code"] == abi.TI_ERR_NO_DEVICE
        assert "no HIP device" in out["initError"]["message"]


def test_tool_preamble_and_message_rendering(checks):
    """toolPreamble (models/qwen3.js:5294-5320): Qwen3's Hermes tool block, each tool's
    {"type": "function", "function": ...} signature on its own line inside <tools>, non-function
    tools dropped, nothing without tools; message rendering (:5429-5441): tool results as
    <tool_response> user turns, assistant tool calls as <tool_call> blocks, text parts joined."""
    _, out = checks
    sig = '{"type":"function","function":{"name":"get_time","parameters":{"type":"object","properties":{}}}}'
    want = "\n".join(["# Tools", "", "You may call one or more functions to assist with the user query.", "",
                      "You are provided with function signatures within <tools></tools> XML tags:", "<tools>", sig,
                      "</tools>", "",
                      "For each function call, return a json object with function name and arguments within "
                      "<tool_call></tool_call> XML tags:",
                      "<tool_call>", '{"name": <function-name>, "arguments": <args-json-object>}', "</tool_call>"])
    assert out["preamble"] == want
    assert out["preambleNone"] == ""
    tool, asst, user = out["rendered"]
    assert tool == {"role": "user", "content": "<tool_response>\n42\n</tool_response>"}
    assert asst == {"role": "assistant", "content": 'ok\n<tool_call>\n{"name": "f", "arguments": {"a":1}}\n</tool_call>'}
    assert user == {"role": "user", "content": "a\nb"}


@pytest.fixture(scope="module")
def conv(tmp_path_factory):
    out = tmp_path_factory.mktemp("conv") / "conv.json"
    subprocess.run([NODE, os.path.join(ROOT, "tests", "js", "conv_spec.js"), str(out)], check=True, timeout=60)
    with open(out) as f:
        d = json.load(f)
    return {c["name"]: c for c in d["cases"]}, d["parsed"]


def kinds(case):
    return [e["type"] for e in case["events"] if not e["type"].startswith("_")]


def deltas(case, field):
    return "".join(e["delta"][field] for e in case["events"] if e["type"] == "delta" and field in e["delta"])


def test_conversation_plain_turn(conv):
    """One round without tools: reasoning and content stream apart (tags split across
    pieces), the status line clears at the first piece, usage counts the prompt exactly."""
    c = conv[0]["plain"]
    k = kinds(c)
    assert k[0] == "round_start" and k[1] == "info" and k[-1] == "agent_done"
    assert k[-5:] == ["info", "round_end", "usage", "message_added", "agent_done"]
    assert deltas(c, "reasoning") == "why so"
    assert deltas(c, "content") == "\n\nHello world"
    end = [e for e in c["events"] if e["type"] == "round_end"][0]
    assert end["content"] == "Hello world"                       # leading whitespace dropped
    usage = [e for e in c["events"] if e["type"] == "usage"][0]["usage"]
    assert usage == {"prompt_tokens": len("<user>hi"), "total_tokens": len("<user>hi")}
    assert [e["type"] for e in c["events"]].count("_before") == 1


def test_conversation_tool_round(conv):
    """A call is parsed, announced as one tool_calls delta, run, and its result re-enters
    the transcript as a <tool_response> user turn; a body that is not JSON is no call but
    still takes its index in the ids."""
    c = conv[0]["tool"]
    assert c["toolCalls"] == [{"n": "get_time", "a": {"tz": "UTC"}}]
    tcd = [e["delta"]["tool_calls"] for e in c["events"] if e["type"] == "delta" and "tool_calls" in e["delta"]]
    assert tcd == [[{"index": 0, "id": "call_0_0", "type": "function",
                     "function": {"name": "get_time", "arguments": '{"tz":"UTC"}'}}]]
    started = [e for e in c["events"] if e["type"] == "tool_started"]
    assert started[0]["tc"]["id"] == "call_0_0"
    res = [e for e in c["events"] if e["type"] == "tool_result"]
    assert res == [{"type": "tool_result", "id": "call_0_0", "result": "R1"}]
    added = [e["message"] for e in c["events"] if e["type"] == "message_added"]
    assert added[0]["role"] == "assistant" and added[0]["tool_calls"][0]["id"] == "call_0_0"
    assert added[1] == {"role": "tool", "tool_call_id": "call_0_0", "content": "R1"}
    assert added[2] == {"role": "assistant", "content": "It is noon."}
    second = c["prompts"][1]
    assert second[1] == {"role": "assistant",
                         "content": '<tool_call>\n{"name": "get_time", "arguments": {"tz":"UTC"}}\n</tool_call>'}
    assert second[2] == {"role": "user", "content": "<tool_response>\nR1\n</tool_response>"}
    assert kinds(c).count("round_start") == 2


def test_conversation_tool_errors_and_limits(conv):
    cases = conv[0]
    err = [e for e in cases["tool_error"]["events"] if e["type"] == "tool_result"][0]
    assert err["result"] == "Error: boom"
    k = kinds(cases["no_runner"])
    assert k[-3:] == ["message_added", "info", "agent_done"] and k.count("round_start") == 1
    assert kinds(cases["round_cap"]).count("round_start") == 8 and len(cases["round_cap"]["toolCalls"]) == 8
    se = cases["stream_error"]
    assert kinds(se)[-3:] == ["info", "error", "agent_done"]
    assert [e for e in se["events"] if e["type"] == "error"][0]["message"] == "Qwen3 dense: device lost"
    ab = cases["aborted"]
    assert ab["rejected"] == "AbortError: aborted" and ab["events"] == []


def test_conversation_never_blank(conv):
    """No answer and no call: the turn's content is a notice, and a turn cut off inside its
    reasoning names the context limit."""
    for name, needle in (("blank", "returned nothing"), ("cut_in_think", "4096-token context")):
        c = conv[0][name]
        end = [e for e in c["events"] if e["type"] == "round_end"][0]["content"]
        assert end.startswith("⚠️") and needle in end
        assert deltas(c, "content").endswith(end)
    assert deltas(conv[0]["cut_in_think"], "reasoning") == "step one step two"


def test_conversation_transcript_and_ids(conv):
    c = conv[0]["transcript"]
    assert c["prompts"][0] == [{"role": "system", "content": "S"}, {"role": "user", "content": "q"}]
    assert c["prompts"][1][2]["content"] == '<tool_call>\n{"name": "f", "arguments": {"a":[1,2]}}\n</tool_call>'
    parsed = conv[1]
    assert parsed[0] == {"id": "call_2_3", "type": "function", "function": {"name": "a", "arguments": "{}"}}
    assert parsed[1] is None and parsed[2] is None
    assert parsed[3]["function"]["arguments"] == '{"x":"y"}'
