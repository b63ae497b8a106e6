"""CPU checks of the JS host's quantized-weights cache format (tabinfer_amd/host/quant-cache.js;
models/qwen3.js:3340-3351, 3626-3717) and of its system-prompt anchor decision
(claimSystemBlock; :5378-5389), through tests/js/qcache_spec.js.

Pinned by construction, on seeded bytes: segments of odd sizes (0, 1, 3, 17, 999, ...)
written with 1000-byte chunks so that they straddle chunk boundaries come back byte for
byte; every segment starts 16-byte aligned in the stream and the manifest's totals agree
with the files; a manifest of another chunk size, geometry or variant reads as no cache; a
segment the caller rejects and a truncated chunk are errors; a write cut short leaves no
manifest (the manifest is removed first and written last). The anchor claims only for a
prompt that begins with a block of >= 16 tokens that the live prefix cache does not cover
and that the anchor records exactly."""
import json
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SPEC = os.path.join(HERE, "js", "qcache_spec.js")

pytestmark = pytest.mark.skipif(shutil.which("node") is None, reason="node is not installed")


@pytest.fixture(scope="module")
def res(tmp_path_factory):
    d = tmp_path_factory.mktemp("qc")
    r = subprocess.run(["node", SPEC, str(d)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout)


def test_round_trip_and_layout(res):
    m = res["manifest"]
    assert res["read"] and res["equal"]
    assert m["ver"] == 1 and m["qgroup"] == 32 and m["chunkSize"] == 1000 and m["variant"] == "T"
    assert m["config"] == {"numLayers": 2, "hidden": 64, "nHeads": 4, "nKvHeads": 2, "headDim": 16, "intermediate": 128,
                           "vocab": 300}
    off = 0
    for g in m["segs"]:
        assert g["off"] % 16 == 0 and g["off"] >= off and g["off"] - off < 16
        off = g["off"] + g["len"]
    assert m["totalBytes"] == off and m["nChunks"] == (off + 999) // 1000
    assert res["files"] == sorted(["manifest"] + ["c%d" % i for i in range(m["nChunks"])])
    # every byte of every segment arrived exactly once
    got = {}
    for name, o, n in res["puts"]:
        got.setdefault(name, []).append((o, n))
    for g in m["segs"]:
        parts = sorted(got.get(g["name"], []))
        pos = 0
        for o, n in parts:
            assert o == pos
            pos += n
        assert pos == g["len"]


def test_mismatches_and_failures(res):
    assert res["otherChunk"] is False and res["otherCfg"] is False and res["otherVariant"] is False
    assert "t5" in res["checkThrew"]
    assert "chunk 1" in res["truncThrew"]
    assert res["afterCut"] is False


def test_checkpoint_identity(res):
    """A cache records the checkpoint it was quantized from: a load naming another checkpoint
    of the same geometry (same safetensors header) or a changed file is a miss; a load from
    the cache alone reads it; a safetensors header that overruns its file is an error."""
    ident = res["ident"]
    hdr = json.dumps({"w": {"dtype": "F16", "shape": [4, 4], "data_offsets": [0, 32]}}, separators=(",", ":"))
    assert ident["sameHeader"] and ident["absolute"] and ident["size"] == 8 + len(hdr) + 32
    assert res["sourceA"] is True and res["sourceNone"] is True
    assert res["sourceB"] is False and res["sourceTwo"] is False and res["sourceTouched"] is False
    src = res["manifestSource"]
    assert len(src["files"]) == 1 and src["files"][0]["path"].endswith("a.safetensors")
    assert set(src["files"][0]) == {"path", "size", "mtimeMs", "header"}
    assert "bad header length" in res["badHeader"]


def test_system_block_claim(res):
    assert res["claim"] == [True, False, True, False, False, False, False, False, False]
