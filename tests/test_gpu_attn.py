"""GPU parity for the int8-KV attention rows.

attnPrep / ropeQK / kvQuantWrite: KV codes, KV scales and RoPE'd rows are
bit-exact against the oracle. Split-KV decode attention: max relative
error <= 1e-3 (normwise) against the oracle's f64 softmax over the dequantized
cache, on the reference's own fixtures (models/qwen3.js:2901-2937: uneven and
empty splits) and at Qwen3 geometry for 4k and 32k contexts.
"""
import numpy as np
import pytest

from tabinfer_amd import abi

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def ctx():
    c = abi.Ctx(0)
    yield c
    c.close()


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def f16r(rng, n, scale=1.0):
    return (rng.standard_normal(n) * scale).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("nHq,nKv,hd,pos,theta", [(16, 8, 128, 0, 1e6), (16, 8, 128, 7, 1e6), (16, 8, 128, 4095, 1e6),
                                                  (16, 8, 128, 32767, 1e6), (4, 2, 128, 7, 10000.0), (2, 1, 64, 3, 1e6)])
def test_attn_prep_bit_exact(ctx, orc, nHq, nKv, hd, pos, theta):
    rng = np.random.default_rng(pos + hd)
    q, k, v = f16r(rng, nHq * hd, 2), f16r(rng, nKv * hd, 2), f16r(rng, nKv * hd, 3)
    qw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float16).view(np.uint16)
    kw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float16).view(np.uint16)
    eps = np.float32(1e-6)
    qr, kq, ks, vq, vs = orc.attn_prep_q8(q, k, v, qw, kw, nHq, nKv, hd, pos, theta, eps)
    cap = pos + 2
    row_w, row_g = nKv * hd // 4, nKv * hd // 32
    dq, dk, dv, dqw, dkw = ctx.upload(q), ctx.upload(k), ctx.upload(v), ctx.upload(qw), ctx.upload(kw)
    dqr = ctx.zeros(nHq * hd * 4)
    caches = [ctx.alloc(cap * row_w * 4), ctx.alloc(cap * row_g * 4), ctx.alloc(cap * row_w * 4), ctx.alloc(cap * row_g * 4)]
    for b in caches:
        ctx.fill_u32(b, 0xA5A5A5A5, b.nbytes // 4)
    ctx.call("ti_attn_prep_q8", dq, dk, dv, dqw, dkw, dqr, *caches, nHq, nKv, hd, pos, np.float32(theta), eps)
    assert np.array_equal(ctx.download(dqr, np.float32, nHq * hd), qr)
    gk = ctx.download(caches[0], np.uint32, cap * row_w).reshape(cap, row_w)
    gks = ctx.download(caches[1], np.uint32, cap * row_g).reshape(cap, row_g)
    gv = ctx.download(caches[2], np.uint32, cap * row_w).reshape(cap, row_w)
    gvs = ctx.download(caches[3], np.uint32, cap * row_g).reshape(cap, row_g)
    assert np.array_equal(gk[pos], kq) and np.array_equal(gv[pos], vq)
    assert np.array_equal(gks[pos].view(np.float32), ks) and np.array_equal(gvs[pos].view(np.float32), vs)
    # other rows untouched
    others = [r for r in range(cap) if r != pos]
    assert np.all(gk[others] == 0xA5A5A5A5) and np.all(gvs[others] == 0xA5A5A5A5)


def test_rope_qk_and_kv_write_bit_exact(ctx, orc):
    rng = np.random.default_rng(3)
    T, nH, nKv, hd, pos0 = 5, 4, 2, 128, 11
    x = f16r(rng, T * nH * hd, 2)
    w = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float16).view(np.uint16)
    dx, dw, dout = ctx.upload(x), ctx.upload(w), ctx.zeros(x.nbytes)
    ctx.call("ti_rope_qk", dx, dw, dout, T, nH, hd, pos0, np.float32(1e6), np.float32(1e-6))
    got = ctx.download(dout, np.float32, x.size).reshape(T, nH, hd)
    for t in range(T):
        for h in range(nH):
            ref = orc.rope_norm_row(x.reshape(T, nH, hd)[t, h], w, hd, pos0 + t, 1e6, 1e-6, True)
            assert np.array_equal(got[t, h], ref)
    # kvQuantWrite of T rows at pos (models/qwen3.js:2939-2963 fixture shape)
    T, nKv, hd, pos, cap = 3, 2, 64, 5, 16
    n = T * nKv * hd
    i = np.arange(n)
    kr = (np.sin(i * 0.13) * (1 + (i % 7))).astype(np.float32)
    vv = (np.cos(i * 0.09) * (1 + (i % 5))).astype(np.float32)
    capn = cap * nKv * hd
    caches = [ctx.zeros(capn), ctx.zeros(capn // 8), ctx.zeros(capn), ctx.zeros(capn // 8)]
    ctx.call("ti_kv_write_q8", ctx.upload(kr), ctx.upload(vv), *caches, T, nKv, hd, pos)
    off_w, off_g = pos * nKv * hd // 4, pos * nKv * hd // 32
    qk, sk = orc.kv_quant(kr)
    qv, sv = orc.kv_quant(vv)
    assert np.array_equal(ctx.download(caches[0], np.uint32, off_w + n // 4)[off_w:], qk)
    assert np.array_equal(ctx.download(caches[1], np.float32, off_g + n // 32)[off_g:], sk)
    assert np.array_equal(ctx.download(caches[2], np.uint32, off_w + n // 4)[off_w:], qv)
    assert np.array_equal(ctx.download(caches[3], np.float32, off_g + n // 32)[off_g:], sv)


def _run_attn(ctx, orc, Q, K, V, S, nHq, nKv, hd, nsplit):
    kq, ks = orc.kv_quant(K)
    vq, vs = orc.kv_quant(V)
    ref = orc.attn_decode_q8(Q, kq, ks, vq, vs, S, nHq, nKv, hd)
    bufs = [ctx.upload(a) for a in (Q, kq, ks, vq, vs)]
    dout = ctx.zeros(nHq * hd * 4)
    ctx.call("ti_attn_decode_q8", *bufs, dout, S, nHq, nKv, hd, nsplit)
    got = ctx.download(dout, np.float32, nHq * hd)
    for b in bufs:
        b.free()
    return got, ref


@pytest.mark.parametrize("S,nHq,nKv,hd,nsplit", [(333, 4, 2, 128, 5), (333, 4, 2, 128, 16), (333, 4, 2, 128, 0),
                                                 (100, 2, 1, 64, 16), (1, 16, 8, 128, 0), (700, 16, 8, 128, 3)])
def test_attn_decode_reference_fixtures(ctx, orc, S, nHq, nKv, hd, nsplit):
    Q = np.sin(np.arange(nHq * hd) * 0.017).astype(np.float32)
    K = np.cos(np.arange(S * nKv * hd) * 0.009).astype(np.float32)
    V = np.sin(np.arange(S * nKv * hd) * 0.004 + 0.7).astype(np.float32)
    got, ref = _run_attn(ctx, orc, Q, K, V, S, nHq, nKv, hd, nsplit)
    assert rel_err(got, ref) < TOL


@pytest.mark.parametrize("S,nsplit", [(4096, 0), (4096, 10), (32768, 0), (32768, 16), (8192, 0), (5000, 0)])
def test_attn_decode_qwen3_geometry(ctx, orc, S, nsplit):
    rng = np.random.default_rng(S + nsplit)
    nHq, nKv, hd = 16, 8, 128
    Q = f16r(rng, nHq * hd)
    K = f16r(rng, S * nKv * hd)
    V = f16r(rng, S * nKv * hd)
    got, ref = _run_attn(ctx, orc, Q, K, V, S, nHq, nKv, hd, nsplit)
    assert rel_err(got, ref) < TOL


def test_attn_decode_nsplit_invariance(ctx, orc):
    rng = np.random.default_rng(5)
    S, nHq, nKv, hd = 1500, 16, 8, 128
    Q, K, V = f16r(rng, nHq * hd), f16r(rng, S * nKv * hd), f16r(rng, S * nKv * hd)
    outs = [_run_attn(ctx, orc, Q, K, V, S, nHq, nKv, hd, ns)[0] for ns in (1, 2, 7, 64, 512)]
    for o in outs[1:]:
        assert rel_err(o, outs[0]) < 1e-5


def test_attn_errors(ctx):
    d = ctx.zeros(1 << 16)
    with pytest.raises(abi.TIError):
        ctx.call("ti_attn_decode_q8", d, d, d, d, d, d, 10, 16, 8, 96 + 1, 0)   # hd not multiple of 32
    with pytest.raises(abi.TIError):
        ctx.call("ti_attn_decode_q8", d, d, d, d, d, d, 10, 15, 8, 128, 0)      # nHq % nKv != 0
    with pytest.raises(abi.TIError):
        ctx.call("ti_rope_qk", d, d, d, 1, 1, 128, 0, np.float32(1e6), np.float32(1e-6))   # in-place


@pytest.mark.parametrize("T,pos0,nHq,nKv,hd", [(2, 0, 16, 8, 128), (8, 100, 16, 8, 128), (8, 4095, 16, 8, 128),
                                               (32, 1000, 16, 8, 128), (5, 63, 4, 2, 128), (8, 300, 8, 8, 128),
                                               (3, 40, 8, 2, 128), (4, 50, 4, 2, 64)])
def test_attn_causal_matches_oracle(ctx, orc, T, pos0, nHq, nKv, hd):
    """T queries at positions pos0..pos0+T-1 over one cache (query t sees keys
    [0, pos0+t]): the one-pass multi-query kernel (hd 128) and the per-query path (hd 64)
    against the oracle's f64 softmax."""
    rng = np.random.default_rng(T * 7 + pos0 + hd)
    S = pos0 + T
    K = rng.standard_normal(S * nKv * hd).astype(np.float32)
    V = rng.standard_normal(S * nKv * hd).astype(np.float32)
    kq, ks = orc.kv_quant(K)
    vq, vs = orc.kv_quant(V)
    Q = (rng.standard_normal(T * nHq * hd) * 2).astype(np.float32)
    bufs = [ctx.upload(a) for a in (Q, kq, ks, vq, vs)]
    out = ctx.upload(np.full(T * nHq * hd, np.nan, np.float32))
    ctx.call("ti_attn_causal_q8", *bufs, out, T, pos0, nHq, nKv, hd)
    got = ctx.download(out, np.float32, T * nHq * hd)
    ref = orc.attn_causal_q8(Q, kq, ks, vq, vs, T, pos0, nHq, nKv, hd)
    assert rel_err(got, ref) < TOL
    # each query row alone is the decode attention over its prefix
    for t in (0, T - 1):
        one = orc.attn_decode_q8(Q[t * nHq * hd:(t + 1) * nHq * hd], kq, ks, vq, vs, pos0 + t + 1, nHq, nKv, hd)
        assert rel_err(got.reshape(T, -1)[t], one) < TOL
    for b in bufs + [out]:
        b.free()
