"""Pins for the oracle's f16 converters and the int4 quantizer.

Independent checks: the reference's own f16 known-answer tests
(native/crates/n2-core/src/binfmt.rs:406-422), numpy's float16 cast (an
independent round-to-nearest implementation) on every non-tie value, the
reference converters' designed tie/carry behaviour on hand-built values, and the
quantizer's invariants and hand-built known answers (models/qwen3.js:3405-3426).
"""
import numpy as np
import pytest


def test_f16_to_f32_known_answers(orc):
    # binfmt.rs:406-422
    assert orc.f16_to_f32(0x0000) == 0.0
    assert np.signbit(orc.f16_to_f32(0x8000))
    assert orc.f16_to_f32(0x3C00) == 1.0
    assert orc.f16_to_f32(0xBC00) == -1.0
    assert orc.f16_to_f32(0x4000) == 2.0
    assert orc.f16_to_f32(0x3800) == 0.5
    assert np.isinf(orc.f16_to_f32(0x7C00))
    assert np.isnan(orc.f16_to_f32(0x7E00))
    assert abs(orc.f16_to_f32(0x7BFF) - 65504.0) < 1.0
    assert abs(orc.f16_to_f32(0x0001) - 5.9604645e-8) < 1e-14
    assert abs(orc.f16_to_f32(0x03FF) - 6.097555e-5) < 1e-10


def test_f16_to_f32_matches_numpy_on_all_finite_patterns(orc):
    hs = np.arange(0, 0x10000, 37, dtype=np.uint32)
    for h in hs:
        e = (h >> 10) & 0x1F
        if e == 31:
            continue
        assert orc.f16_to_f32(int(h)) == float(np.uint16(h).view(np.float16))


@pytest.mark.parametrize("conv", ["q3", "eng"])
def test_f32_to_f16_roundtrips_every_finite_f16(orc, conv):
    f = orc.f32_to_f16_q3 if conv == "q3" else orc.f32_to_f16_eng
    for h in range(0, 0x10000, 3):
        if ((h >> 10) & 0x1F) == 31:
            continue
        v = np.float32(np.uint16(h).view(np.float16))
        assert f(v) == h, hex(h)


def _is_tie(v32):
    """True if the f32 value lies exactly halfway between two f16 neighbours."""
    v = np.float32(v32)
    lo = np.float16(v)
    if np.float32(lo) == v or not np.isfinite(lo):
        return False
    a = np.float64(lo)
    b = np.float64(np.nextafter(lo, np.float16(np.inf) if v > np.float32(lo) else np.float16(-np.inf)))
    return abs(np.float64(v) - a) == abs(np.float64(v) - b)


def test_f32_to_f16_q3_matches_numpy_off_ties(orc):
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-7, 4, 4000),
                           rng.uniform(-1e-4, 1e-4, 2000).astype(np.float32)])
    for v in vals:
        if _is_tie(v):
            continue
        assert orc.f32_to_f16_q3(v) == int(np.float16(v).view(np.uint16)), v


def test_f32_to_f16_q3_ties_round_away_from_zero(orc):
    # 1 + 2^-11 is halfway between 0x3C00 and 0x3C01: RNE gives 0x3C00, the
    # reference's "+1 if bit 12" gives 0x3C01 (qwen3.js:3371-3372).
    assert orc.f32_to_f16_q3(np.float32(1.0 + 2.0 ** -11)) == 0x3C01
    assert orc.f32_to_f16_q3(np.float32(-(1.0 + 2.0 ** -11))) == 0xBC01
    # carry into the exponent: halfway between 0x3BFF and 2.0
    assert orc.f32_to_f16_q3(np.float32(1.99951171875)) == 0x4000
    # subnormal tie: halfway between 0x0001 and 0x0002
    assert orc.f32_to_f16_q3(np.float32(1.5 * 2.0 ** -24)) == 0x0002
    # overflow and underflow
    assert orc.f32_to_f16_q3(np.float32(1e6)) == 0x7C00
    assert orc.f32_to_f16_q3(np.float32(1e-8)) == 0x0000
    assert orc.f32_to_f16_q3(np.float32(np.nan)) == 0x7E00


def test_f32_to_f16_eng_quirks(orc):
    # engine/webgpu-engine.js:233: the mantissa carry (0x400) is OR-ed into
    # (e<<10). For an odd exponent field the carry is lost: [1.99951, 2) -> 1.0.
    assert orc.f32_to_f16_eng(np.float32(1.99951171875)) == 0x3C00
    assert orc.f32_to_f16_eng(np.float32(1.999755859375)) == 0x3C00
    # even exponent field (values in [0.5,1)): the OR equals an add -> 1.0 (correct)
    assert orc.f32_to_f16_eng(np.float32(0.999755859375)) == 0x3C00
    # off the carry and tie cases it agrees with numpy
    rng = np.random.default_rng(2)
    for v in rng.standard_normal(3000).astype(np.float32):
        m = np.float32(v).view(np.uint32) & 0x7FFFFF
        if _is_tie(v) or m >= 0x7FF000:
            continue
        assert orc.f32_to_f16_eng(v) == int(np.float16(v).view(np.uint16)), v


def _bf16(vals):
    return (np.asarray(vals, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _unpack(pack, N, K):
    w = pack.reshape(N, K // 8)
    sh = (np.arange(8, dtype=np.uint32) * 4)
    return ((w[:, :, None] >> sh) & 0xF).reshape(N, K).astype(np.int64)


def test_int4_known_answers(orc):
    K = 32
    # group maxabs 7 -> scale exactly 1.0 (0x3C00); codes are the values + 8
    vals = np.array([7, -7, 0, 1, -1, 3, -3, 2] * 4, np.float32)
    pack, sc = orc.quant_int4_bf16(_bf16(vals), 1, K)
    assert sc[0] == 0x3C00
    assert np.array_equal(_unpack(pack, 1, K)[0], vals.astype(np.int64) + 8)
    # nibble placement: k = 8w + i -> bits 4i of word w (qwen3.js:3421)
    assert (pack[0] & 0xF) == 15 and ((pack[0] >> 4) & 0xF) == 1 and ((pack[0] >> 8) & 0xF) == 8


def test_int4_ties_round_toward_plus_infinity(orc):
    """Math.round (qwen3.js:3419): a half rounds toward +Inf, so 2.5 -> 3 but -2.5 -> -2, and
    -0.5 -> -0, whose nibble is 8. Scales are exact here (maxabs 7 -> 1.0, maxabs 3.5 -> 0.5),
    so every w * inv is an exact half or whole number; ties to even, or away from zero,
    would give other nibbles."""
    K = 64
    g0 = [7, 2.5, -2.5, -0.5, 0.5, 3.5, -3.5, 1.5, -1.5, 0, -7, 6.5, -6.5]
    g1 = [3.5, 1.25, -1.25, -0.25, 0.25, -0.75, 0.75, -3.25, 3.25, 0]       # inv = 2
    vals = np.zeros(K, np.float32)
    vals[:len(g0)] = g0
    vals[32:32 + len(g1)] = g1
    pack, sc = orc.quant_int4_bf16(_bf16(vals), 1, K)
    assert sc[0] == 0x3C00 and sc[1] == 0x3800
    codes = _unpack(pack, 1, K)[0]
    want0 = [7, 3, -2, 0, 1, 4, -3, 2, -1, 0, -7, 7, -6]
    want1 = [7, 3, -2, 0, 1, -1, 2, -6, 7, 0]
    assert list(codes[:len(g0)] - 8) == want0
    assert list(codes[32:32 + len(g1)] - 8) == want1
    # the nibbles of -0.5 and 0.5 (k = 3, 4: word 0, bits 12 and 16)
    assert ((pack[0] >> 12) & 0xF) == 8 and ((pack[0] >> 16) & 0xF) == 9


def test_int4_zero_and_tiny_groups(orc):
    K = 64
    vals = np.zeros(K, np.float32)
    vals[32:] = np.float32(1e-9)         # maxabs/7 underflows f16 -> scale bits 0
    vals[33] = np.float32(-1e-9)
    vals[34] = 0.0
    pack, sc = orc.quant_int4_bf16(_bf16(vals), 1, K)
    codes = _unpack(pack, 1, K)[0]
    # all-zero group: 1e-8 -> f16 0, inv = +Inf, 0*Inf = NaN, (NaN+8)&15 = 0
    assert sc[0] == 0 and np.all(codes[:32] == 0)
    # tiny group: +w*Inf -> +Inf -> clamp 7 -> 15 ; -w -> -8 -> 0 ; 0 -> NaN -> 0
    assert sc[1] == 0
    assert codes[32] == 15 and codes[33] == 0 and codes[34] == 0


def test_int4_invariants_random(orc):
    rng = np.random.default_rng(3)
    N, K = 64, 256
    w32 = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    wb = _bf16(w32)
    wf = (wb.astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(N, K // 32, 32)
    pack, sc = orc.quant_int4_bf16(wb, N, K)
    q = _unpack(pack, N, K).reshape(N, K // 32, 32) - 8
    s = orc.f16_array_to_f64(sc).reshape(N, K // 32, 1)
    assert q.min() >= -8 and q.max() <= 7
    # scale bits = f16(f32(maxabs/7)) within the away-from-zero rounding: equal to
    # numpy's RNE cast except on exact ties
    mx = np.abs(wf).max(axis=2)
    for v, h in zip((mx / 7.0).astype(np.float32).ravel(), sc):
        if not _is_tie(v):
            assert int(np.float16(v).view(np.uint16)) == int(h)
    # the group's max element maps to +/-7, never -8
    am = np.abs(wf).argmax(axis=2)
    qm = np.take_along_axis(q, am[..., None], axis=2)[..., 0]
    assert np.all(np.abs(qm) == 7)
    # dequant error <= s/2 (+1 ulp) wherever the value is inside the clamp range
    err = np.abs(q * s - wf)
    inside = np.abs(wf / s) <= 7.5
    assert np.all(err[inside] <= s.repeat(32, axis=2)[inside] * (0.5 + 1e-9))
