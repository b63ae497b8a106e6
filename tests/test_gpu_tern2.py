"""GPU parity of the on-GPU ternary format (models/qwen3.js:3428-3469, 449-503, 747-810):
ti_quant_tern_bf16 bit-exact against the oracle (codes, scales, the not-ternary flag),
ti_gemv_tern2 and ti_gateup_silu_tern2 within 1e-3 of the oracle's f64 at the Bonsai-1.7B
shapes (q/k/v, o, gate/up, down, the 151936-row lm_head) and a shape of the generic kernel,
the accumulate mode included."""
import numpy as np
import pytest

from tabinfer_amd import abi
from tern2_data import ternary_bf16

pytestmark = pytest.mark.gpu

TOL = 1e-3


@pytest.fixture(scope="module")
def ctx():
    c = abi.Ctx(0)
    yield c
    c.close()


def rel(got, want):
    want = np.asarray(want, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - want).max() / max(np.abs(want).max(), 1e-30))


def quantize(ctx, w, N, K):
    wd = ctx.upload(w)
    pack, sc, flag = ctx.zeros(N * K // 4), ctx.zeros(N * K // 16), ctx.zeros(4)
    ctx.call("ti_quant_tern_bf16", wd, pack, sc, N, K, flag)
    out = (ctx.download(pack, np.uint32, N * K // 16), ctx.download(sc, np.uint16, N * K // 32),
           int(ctx.download(flag, np.uint32, 1)[0]))
    return out, (pack, sc)


@pytest.mark.parametrize("N,K", [(256, 2048), (64, 6144), (3, 192)])
def test_quantizer_bit_exact(ctx, orc, N, K):
    rng = np.random.default_rng(N + K)
    w = ternary_bf16(rng, N, K)
    (p, s, flag), _ = quantize(ctx, w, N, K)
    want = orc.quant_tern_bf16(w, N, K)
    assert flag == 0 and want is not None
    assert np.array_equal(p, want[0]) and np.array_equal(s, want[1])
    # a continuous tensor is not ternary, on both
    cont = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    cb = (cont.view(np.uint32) >> 16).astype(np.uint16)
    (_, _, flag), _ = quantize(ctx, cb, N, K)
    assert flag != 0 and orc.quant_tern_bf16(cb, N, K) is None
    # one group 3 ULPs off in the last row: rejected, 2 ULPs: accepted, as the oracle decides
    for ulps, ternary in ((3, False), (2, True)):
        w2 = w.copy()
        g = (N - 1) * K + K - 32
        m = int(w2[g:g + 32].max() & 0x7FFF) or 0x3C80
        w2[g:g + 32] = m
        w2[g + 5] = m - ulps
        (p2, s2, flag), _ = quantize(ctx, w2, N, K)
        want2 = orc.quant_tern_bf16(w2, N, K)
        assert (flag == 0) == ternary and (want2 is not None) == ternary
        if ternary:
            assert np.array_equal(p2, want2[0]) and np.array_equal(s2, want2[1])


def activation(ctx, orc, rng, K):
    x = rng.standard_normal(K).astype(np.float32)
    xq, xs, xsum = orc.quant_act_q8(x)
    return (xq, xs, xsum), (ctx.upload(xq), ctx.upload(xs), ctx.upload(xsum))


@pytest.mark.parametrize("N,K", [(2048, 2048), (1024, 2048), (2048, 6144), (151936, 2048), (100, 192), (40, 1024)])
def test_gemv_tern2(ctx, orc, N, K):
    rng = np.random.default_rng(N * 7 + K)
    w = ternary_bf16(rng, N, K)
    pack, sc = orc.quant_tern_bf16(w, N, K)
    (xq, xs, xsum), (dq, ds, dsum) = activation(ctx, orc, rng, K)
    dp, dsc = ctx.upload(pack), ctx.upload(sc)
    y = ctx.zeros(N * 4)
    ctx.call("ti_gemv_tern2", dq, ds, dsum, dp, dsc, y, N, K, 0)
    want = orc.gemv_tern2(xq, xs, pack, sc, N, K)
    got = ctx.download(y, np.float32, N)
    assert rel(got, want) < TOL
    # accumulate: y += W x
    ctx.call("ti_gemv_tern2", dq, ds, dsum, dp, dsc, y, N, K, 1)
    assert rel(ctx.download(y, np.float32, N), 2 * want) < TOL


@pytest.mark.parametrize("I,H", [(6144, 2048), (3072, 1024), (50, 320)])
def test_gateup_silu_tern2(ctx, orc, I, H):
    rng = np.random.default_rng(I + H)
    g, u = ternary_bf16(rng, I, H), ternary_bf16(rng, I, H)
    gp, gs = orc.quant_tern_bf16(g, I, H)
    up, us = orc.quant_tern_bf16(u, I, H)
    (xq, xs, xsum), (dq, ds, dsum) = activation(ctx, orc, rng, H)
    swi = ctx.zeros(I * 4)
    ctx.call("ti_gateup_silu_tern2", dq, ds, dsum, ctx.upload(gp), ctx.upload(gs), ctx.upload(up), ctx.upload(us), swi, I, H)
    want = orc.gateup_silu_tern2(xq, xs, gp, gs, up, us, I, H)
    assert rel(ctx.download(swi, np.float32, I), want) < TOL


def test_rejects_bad_arguments(ctx):
    b = ctx.zeros(1 << 16)
    with pytest.raises(abi.TIError):
        ctx.call("ti_gemv_tern2", b, b, b, b, b, b, 4, 96, 0)           # K % 64
    with pytest.raises(abi.TIError):
        ctx.call("ti_quant_tern_bf16", b, b, b, 4, 32, b)               # K % 64
