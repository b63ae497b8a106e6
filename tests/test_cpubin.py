"""The `.cpu.bin` container reader (ti_cpubin_*, native/docs/FORMAT.md), on the CPU.

The reference reader's own tests (native/crates/n2-core/src/binfmt.rs:406-482) are the
model: a synthetic container with a misaligned header round-trips; a codesLen that
disagrees with N*K/4 and a range past the blob are refused; the f16 known answers of the
embedding decode. Each further rule the reader enforces (G, kind, K % G, scalesLen, the
header overrunning the file, UTF-8, JSON, f32 alignment, embedding rows) gets its case, and
a file on disk goes through ti_cpubin_open as well as through ti_cpubin_parse.
"""
import json
import struct

import numpy as np
import pytest

from tabinfer_amd import abi


def container(tensors, blob, G=64, raw_header=None):
    h = raw_header if raw_header is not None else json.dumps(
        dict({"G": G} if G is not None else {}, tensors=tensors)).encode()
    return struct.pack("<I", len(h)) + h + bytes(blob)


def refused(data, needle):
    with pytest.raises(abi.TIError) as e:
        abi.CpuBin(data=data)
    assert e.value.code == abi.TI_ERR_INVALID
    assert needle in str(e.value), str(e.value)


def tern(N, K, codes_off, scales_off, **over):
    t = {"kind": "tern", "N": N, "K": K, "codesOff": codes_off, "codesLen": N * K // 4, "scalesOff": scales_off,
         "scalesLen": N * (K // 64) * 4}
    t.update(over)
    return t


def test_round_trips_a_synthetic_container():
    """binfmt.rs:424-457: 2 x 64 codes at 0, scales 1.5 / 2.5 at 32, a header length that is
    not a multiple of 4 (the blob must not inherit the misalignment)."""
    blob = bytes(i % 3 for i in range(32)) + struct.pack("<ff", 1.5, 2.5)
    data = container({"lm_head.weight": tern(2, 64, 0, 32)}, blob)
    assert (len(data) - 4 - 40) % 4 != 0
    with abi.CpuBin(data=data) as c:
        assert c.summary() == (64, 1, 40)
        t, codes, sc = c.tensor("lm_head.weight")
        assert (t.kind, t.N, t.K) == (abi.CpuBin.TERN, 2, 64)
        assert codes.tobytes() == blob[:32]
        assert list(sc.view(np.float32)) == [1.5, 2.5]


def test_rejects_a_shape_mismatch():
    """binfmt.rs:459-470: codesLen deliberately wrong for N*K/4."""
    refused(container({"w": tern(2, 64, 0, 32, codesLen=99)}, bytes(128)), "codesLen")


def test_rejects_an_overrunning_range():
    """binfmt.rs:472-481: an f32 tensor whose range runs past a 16-byte blob."""
    refused(container({"w": {"kind": "f32", "shape": [4], "off": 0, "len": 4096}}, bytes(16)), "overruns")


@pytest.mark.parametrize("data,needle", [
    (b"\x01\x00", "too short"),
    (struct.pack("<I", 100) + b"{}", "overruns the file"),
    (container({}, b"", raw_header=b"\xff\xfe{}"), "UTF-8"),
    (container({}, b"", raw_header=b'{"G": 64, "tensors": {'), "JSON"),
    (container({}, b"", raw_header=b'{"G": 64}'), "no `tensors`"),
    (container({"w": tern(2, 64, 0, 32)}, bytes(64), G=32), "G=32"),
    (container({"w": {"N": 1}}, bytes(64)), "missing `kind`"),
    (container({"w": {"kind": "q4"}}, bytes(64)), "unknown kind `q4`"),
    (container({"w": tern(2, 96, 0, 48, codesLen=48, scalesLen=8)}, bytes(128)), "not a multiple of G"),
    (container({"w": tern(2, 64, 0, 32, scalesLen=12)}, bytes(128)), "scalesLen"),
    (container({"w": tern(2, 64, 0, 112)}, bytes(116)), "overruns"),
    (container({"w": dict(tern(2, 64, 0, 32), N=-2)}, bytes(128)), "non-negative integer"),
    (container({"e": {"kind": "embed_f16", "shape": [2, "x"], "off": 0, "len": 8}}, bytes(16)), "shape"),
    # ranges and shapes near the 2^62 field limit: no sum or product may wrap past a check
    (container({"w": {"kind": "f32", "shape": [1], "off": 1 << 62, "len": 1 << 62}}, bytes(16)), "overruns"),
    (container({"w": {"kind": "f32", "shape": [1], "off": 8, "len": (1 << 62) - 4}}, bytes(16)), "overruns"),
    (container({"w": tern(1 << 40, 1 << 40, 0, 0, codesLen=0, scalesLen=0)}, bytes(16)), "overflows"),
])
def test_rejects_each_rule(data, needle):
    refused(data, needle)


def test_missing_g_defaults_to_64():
    blob = bytes(32) + struct.pack("<ff", 1.0, 1.0)
    with abi.CpuBin(data=container({"w": tern(2, 64, 0, 32)}, blob, G=None)) as c:
        assert c.summary()[0] == 64


def test_f32_views_must_be_aligned_whole_values():
    blob = bytes(64)
    with abi.CpuBin(data=container({"a": {"kind": "f32", "shape": [3], "off": 2, "len": 12},
                                    "b": {"kind": "f32", "shape": [3], "off": 0, "len": 10}}, blob)) as c:
        for name, needle in (("a", "not 4-byte aligned"), ("b", "whole number of f32")):
            with pytest.raises(abi.TIError) as e:
                c.tensor(name)
            assert needle in str(e.value)
        with pytest.raises(abi.TIError) as e:
            c.tensor("absent")
        assert "not in container" in str(e.value)


def test_embedding_rows_decode_f16_exactly():
    """The f16 known answers of binfmt.rs:406-422 through embed_row, and its range checks."""
    bits = [0x0000, 0x8000, 0x3C00, 0xBC00, 0x4000, 0x3800, 0x7C00, 0x7E00, 0x7BFF, 0x0001, 0x03FF, 0xFC00]
    want = [0.0, -0.0, 1.0, -1.0, 2.0, 0.5, np.inf, np.nan, 65504.0, 2.0 ** -24, 1023 * 2.0 ** -24, -np.inf]
    blob = struct.pack("<12H", *bits) + bytes(8)
    with abi.CpuBin(data=container({"model.embed_tokens.weight": {"kind": "embed_f16", "shape": [2, 6], "off": 0,
                                                                   "len": 24}}, blob)) as c:
        rows = np.concatenate([c.embed_row("model.embed_tokens.weight", r, 6) for r in range(2)])
        got = rows.astype(np.float64)
        w = np.array(want)
        assert np.array_equal(np.isnan(got), np.isnan(w))
        ok = ~np.isnan(w)
        assert np.array_equal(got[ok], w[ok])
        assert np.signbit(got[1]) and not np.signbit(got[0])
        assert np.array_equal(rows.view(np.uint32) >> 31, (np.array(bits) >> 15).astype(np.uint32))
        with pytest.raises(abi.TIError) as e:
            c.embed_row("model.embed_tokens.weight", 2, 6)
        assert "out of range" in str(e.value)
        with pytest.raises(abi.TIError) as e:
            c.embed_row("model.embed_tokens.weight", 0, 5)
        assert "embedding dim is 6" in str(e.value)
        # rows whose byte offset overflows a signed 64-bit product are out of range too
        for row in ((2 ** 63 - 1) // 6, (2 ** 63 - 1) // 12 + 1, 2 ** 62, -1):
            with pytest.raises(abi.TIError) as e:
                c.embed_row("model.embed_tokens.weight", row, 6)
            assert "out of range" in str(e.value)


def test_open_reads_a_file_and_sorts_names(tmp_path):
    """ti_cpubin_open (Container::open): header then blob streamed from disk; tensors come
    back in name order (the reference's BTreeMap); every kind's fields survive."""
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 256, 4 * 128 // 4, dtype=np.uint8).tobytes()
    scales = struct.pack("<8f", *np.arange(8, dtype=np.float32) + 0.25)
    norm = struct.pack("<4f", 1.0, 2.0, 3.0, 4.0)
    emb = struct.pack("<4H", 0x3C00, 0x4000, 0x4200, 0x4400)
    blob = codes + scales + norm + emb                     # 128 + 32 + 16 + 8: every entry 16-aligned but the last
    tensors = {"z.k": tern(4, 128, 0, 128), "a.norm": {"kind": "f32", "shape": [4], "off": 160, "len": 16},
               "m.emb": {"kind": "embed_f16", "shape": [1, 4], "off": 176, "len": 8}}
    p = tmp_path / "tiny.cpu.bin"
    p.write_bytes(container(tensors, blob))
    with abi.CpuBin(path=str(p)) as c:
        assert c.names() == ["a.norm", "m.emb", "z.k"]
        t, d, s = c.tensor("z.k")
        assert (t.N, t.K) == (4, 128) and d.tobytes() == codes and s.tobytes() == scales
        t, d, _ = c.tensor("a.norm")
        assert t.kind == abi.CpuBin.F32 and list(t.shape[:t.ndim]) == [4] and d.tobytes() == norm
        t, d, _ = c.tensor("m.emb")
        assert t.kind == abi.CpuBin.EMBED_F16 and list(t.shape[:t.ndim]) == [1, 4]
        assert list(c.embed_row("m.emb", 0, 4)) == [1.0, 2.0, 3.0, 4.0]
    with pytest.raises(abi.TIError) as e:
        abi.CpuBin(path=str(tmp_path / "absent.cpu.bin"))
    assert "cannot open" in str(e.value)
