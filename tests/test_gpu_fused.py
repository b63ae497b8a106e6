"""GPU parity of the fused decode-step launches.

Each fused kernel is checked against the oracle composition of the reference
launchers it replaces:
  rmsnormQ + projGemv x3         (models/qwen3.js:3981-3984)
  quantQ8 + gemvDP4 + residual   (linearQ, :1588-1608)
  rmsnormQ + gateUpSiluDP4       (:4023-4024)
  rmsnorm + gemvQ + argmax       (:4037-4055)
  attnPrepQ8 + attnDecodeStreamQ8 + combine (:4001-4002)
The int8 activation codes are bit-exact; float outputs are within max relative
error 1e-3 (normwise) of the f64 oracle on the quantized operands; KV codes are
bit-exact against the oracle's attnPrepQ8 on the same f32 inputs.
"""
import ctypes as C

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


def bf16_normal(rng, n, std=0.02):
    w = (rng.standard_normal(n) * std).astype(np.float32)
    return (w.view(np.uint32) >> 16).astype(np.uint16)


def quantized(ctx, orc, rng, N, K):
    w = bf16_normal(rng, N * K)
    pack, sc = orc.quant_int4_bf16(w, N, K)
    return pack, sc, ctx.upload(pack), ctx.upload(sc)


def ptrs(bufs):
    arr = (C.c_void_p * len(bufs))()
    for i, b in enumerate(bufs):
        arr[i] = int(b)
    return arr


def ints(vals):
    arr = (C.c_int * len(vals))()
    for i, v in enumerate(vals):
        arr[i] = v
    return arr


@pytest.mark.parametrize("K,Ns,norm", [(1024, (2048, 1024, 1024), True), (2048, (2048, 1024, 1024), True),
                                        (2048, (4096,), True), (320, (200, 70), True), (1024, (96,), False),
                                        (6144, (2048,), False), (3072, (1024, 33, 7), True)])
def test_rmsnorm_gemv_matches_separate_launchers(ctx, orc, K, Ns, norm):
    rng = np.random.default_rng(K + sum(Ns))
    x = (rng.standard_normal(K) * 3).astype(np.float16).astype(np.float32)
    x[:32] = 0                                             # a zero group
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float16).view(np.uint16)
    eps = np.float32(1e-6)
    mats = [quantized(ctx, orc, rng, N, K) for N in Ns]
    ys = [ctx.zeros(N * 4) for N in Ns]
    dx, dn = ctx.upload(x), ctx.upload(nw)
    xq_o, xs_o = ctx.zeros(K), ctx.zeros(K // 8)
    ctx.call("ti_rmsnorm_gemv_q4", dx, dn if norm else None, eps, K, len(Ns), ptrs([m[2] for m in mats]),
             ptrs([m[3] for m in mats]), ptrs(ys), ints(Ns), xq_o, xs_o)
    if norm:
        oq, os_, _ = orc.rmsnorm_q8(x, nw, eps)
    else:
        oq, os_, _ = orc.quant_act_q8(x)
    assert np.array_equal(ctx.download(xq_o, np.uint32, K // 4), oq)
    assert np.array_equal(ctx.download(xs_o, np.float32, K // 32), os_)
    for (pack, sc, _, _), y, N in zip(mats, ys, Ns):
        ref = orc.gemv_q4_q8(oq, os_, pack, sc, N, K)
        assert rel_err(ctx.download(y, np.float32, N), ref) < TOL


@pytest.mark.parametrize("N,K", [(1024, 2048), (2048, 2048), (1024, 3072), (2048, 6144), (100, 320)])
def test_linear_t1_residual(ctx, orc, N, K):
    """linearQ at T=1, N < 16384 (one fused launch): y += W . quantQ8(x)."""
    rng = np.random.default_rng(N * 7 + K)
    x = rng.standard_normal(K).astype(np.float32)
    y0 = rng.standard_normal(N).astype(np.float32)
    pack, sc, dp, ds = quantized(ctx, orc, rng, N, K)
    dx, dy = ctx.upload(x), ctx.upload(y0)
    ctx.call("ti_linear_q4", dx, dp, ds, dy, 1, N, K, 1)
    xq, xs, _ = orc.quant_act_q8(x)
    ref = y0.astype(np.float64) + orc.gemv_q4_q8(xq, xs, pack, sc, N, K)
    assert rel_err(ctx.download(dy, np.float32, N), ref) < TOL


@pytest.mark.parametrize("I,H", [(3072, 1024), (6144, 2048), (130, 256), (1792, 2048), (96, 3072)])
def test_rmsnorm_gateup(ctx, orc, I, H):
    rng = np.random.default_rng(I + H)
    x = (rng.standard_normal(H) * 2).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(H)).astype(np.float16).view(np.uint16)
    eps = np.float32(1e-6)
    gp, gs, dgp, dgs = quantized(ctx, orc, rng, I, H)
    up, us, dup, dus = quantized(ctx, orc, rng, I, H)
    dswi = ctx.zeros(I * 4)
    ctx.call("ti_rmsnorm_gateup_silu_q4", ctx.upload(x), ctx.upload(nw), eps, dgp, dgs, dup, dus, dswi, I, H, None, None)
    xq, xs, _ = orc.rmsnorm_q8(x, nw, eps)
    ref = orc.gateup_silu_q4(xq, xs, gp, gs, up, us, I, H)
    got = ctx.download(dswi, np.float32, I)
    assert rel_err(got, ref) < TOL
    if I % 32 == 0:
        # the chunked kernel: the same swi, plus swi quantized as linearQ's quantQ8 would
        sw2, sq, ss = ctx.zeros(I * 4), ctx.zeros(I), ctx.zeros(I // 8)
        ctx.call("ti_rmsnorm_gateup_silu_q4", ctx.upload(x), ctx.upload(nw), eps, dgp, dgs, dup, dus, sw2, I, H, sq, ss)
        got2 = ctx.download(sw2, np.float32, I)
        assert rel_err(got2, ref) < TOL
        oq, os_, _ = orc.quant_act_q8(got2)
        assert np.array_equal(ctx.download(sq, np.uint32, I // 4), oq)
        assert np.array_equal(ctx.download(ss, np.float32, I // 32), os_)
        # swi itself may be omitted
        sq2, ss2 = ctx.zeros(I), ctx.zeros(I // 8)
        ctx.call("ti_rmsnorm_gateup_silu_q4", ctx.upload(x), ctx.upload(nw), eps, dgp, dgs, dup, dus, None, I, H, sq2, ss2)
        assert np.array_equal(ctx.download(sq2, np.uint32, I // 4), oq)


@pytest.mark.parametrize("N,K,tied", [(151936, 1024, (300, 16394)), (151936, 2048, (98765, 98766)),
                                      (1000, 256, (64, 128)), (1000, 256, (5, 261))])
def test_lm_head_argmax_ties(ctx, orc, N, K, tied):
    """The fused lm_head's argmax resolves equal logits as argmaxKernel does. The tied rows
    share one packed row with a single non-zero 32-group of large codes (every other group
    has code 8, i.e. 0): their logits are the same exact sum of one group's dot, so they
    are equal bit for bit whatever the reduction order."""
    rng = np.random.default_rng(K + tied[0])
    x = (rng.standard_normal(K) * 2).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float16).view(np.uint16)
    eps = np.float32(1e-6)
    pack, sc, _, _ = quantized(ctx, orc, rng, N, K)
    pack, sc = pack.reshape(N, K // 8).copy(), sc.reshape(N, K // 32).copy()
    row = np.full(K // 8, 0x88888888, np.uint32)
    normed = orc.rmsnorm(x, nw, 1, K, eps)
    g = int(np.argmax(np.abs(normed[:K - K % 32].reshape(-1, 32)).sum(axis=1)))
    signs = np.where(normed[32 * g:32 * g + 32] >= 0, 15, 1)            # q = +7 / -7 along the sign of x
    for w in range(4):
        row[4 * g + w] = sum(int(signs[8 * w + e]) << (4 * e) for e in range(8))
    for r in tied:
        pack[r], sc[r] = row, np.float16(0.5).view(np.uint16)
    pack, sc = pack.ravel(), sc.ravel()
    dp, ds = ctx.upload(pack), ctx.upload(sc)
    dl, hist = ctx.zeros(N * 4), ctx.zeros(16 * 4)
    ctx.call("ti_rmsnorm_lm_head_argmax", ctx.upload(x), ctx.upload(nw), eps, dp, ds, dl, N, K, hist, 5)
    got = ctx.download(dl, np.float32, N)
    assert got[tied[0]] == got[tied[1]] and got[tied[0]] == got.max()
    assert int(ctx.download(hist, np.uint32, 16)[5]) == orc.argmax(got)


@pytest.mark.parametrize("N,K", [(151936, 1024), (151936, 2048), (1000, 256)])
def test_lm_head_argmax(ctx, orc, N, K):
    rng = np.random.default_rng(N + K)
    x = (rng.standard_normal(K) * 2).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float16).view(np.uint16)
    eps = np.float32(1e-6)
    pack, sc, dp, ds = quantized(ctx, orc, rng, N, K)
    dl = ctx.zeros(N * 4)
    hist = ctx.zeros(16 * 4)
    ctx.call("ti_rmsnorm_lm_head_argmax", ctx.upload(x), ctx.upload(nw), eps, dp, ds, dl, N, K, hist, 5)
    normed = orc.rmsnorm(x, nw, 1, K, eps)
    ref = orc.gemv_q4_f32(normed, pack, sc, N, K)
    got = ctx.download(dl, np.float32, N)
    assert rel_err(got, ref) < TOL
    tok = int(ctx.download(hist, np.uint32, 16)[5])
    assert tok == int(np.argmax(got))                      # the kernel's own logits
    s = np.sort(ref)
    if s[-1] - s[-2] > 4 * TOL * np.max(np.abs(ref)):
        assert tok == int(np.argmax(ref))
    # a second launch reuses the completion counter (it must have been reset)
    ctx.call("ti_rmsnorm_lm_head_argmax", ctx.upload(x), ctx.upload(nw), eps, dp, ds, dl, N, K, hist, 6)
    assert int(ctx.download(hist, np.uint32, 16)[6]) == tok


def _tie_cases(rng):
    """(N, logits, expected index) for argmax: the reference's tie order across workgroups,
    threads and one thread's scan, heavy ties, and the values never selected."""
    cases = []
    for N, idx, want in [(151936, (300, 16394), 16394), (151936, (98765, 98766), 98766), (151936, (256, 512), 512),
                         (151936, (16384, 0), 0), (1000, (64, 128), 128), (1000, (5, 261), 5), (16384, (16383, 256), 256)]:
        x = rng.standard_normal(N).astype(np.float32)
        x[list(idx)] = 50.0                               # models/qwen3.js:3171-3180 known answer, tied
        cases.append((N, x, want))
    for N in (151936, 1000):
        x = rng.integers(-3, 4, N).astype(np.float32)
        cases.append((N, x, None))
    cases.append((151936, np.full(151936, -np.inf, np.float32), 0))
    x = np.full(1000, np.nan, np.float32)
    x[7] = -3.0e38
    x[9] = 1.0
    cases.append((1000, x, 9))
    return cases


def test_argmax_tie_order_and_embed(ctx, orc):
    rng = np.random.default_rng(9)
    hist = ctx.zeros(8 * 4)
    for N, logits, want in _tie_cases(rng):
        ref = orc.argmax(logits)
        if want is not None:
            assert ref == want, (N, want)
        ctx.call("ti_argmax", ctx.upload(logits), N, hist, 3)
        assert int(ctx.download(hist, np.uint32, 8)[3]) == ref, (N, ref)
    V, H = 100, 64
    emb = rng.standard_normal(V * H).astype(np.float16)
    ids = np.array([5, 0, 99, 1234], np.int32)               # the last id is past the vocabulary
    y = ctx.zeros(4 * H * 4)
    ctx.call("ti_embed", ctx.upload(ids), ctx.upload(emb.view(np.uint16)), y, 4, H, 0, V)
    got = ctx.download(y, np.float32, 4 * H).reshape(4, H)
    e = emb.astype(np.float32).reshape(V, H)
    assert np.array_equal(got[:3], e[[5, 0, 99]]) and np.array_equal(got[3], e[V - 1])


def f16r(rng, n, scale=1.0):
    return (rng.standard_normal(n) * scale).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("nHq,nKv,hd,S,max_splits", [(16, 8, 128, 1, 0), (16, 8, 128, 2, 0), (16, 8, 128, 333, 5),
                                                     (16, 8, 128, 333, 0), (16, 8, 128, 4096, 0),
                                                     (16, 8, 128, 32768, 0), (16, 8, 128, 5000, 64),
                                                     (8, 8, 128, 700, 0), (4, 2, 64, 100, 16), (2, 2, 64, 129, 3)])
def test_attn_step_matches_prep_plus_decode(ctx, orc, nHq, nKv, hd, S, max_splits):
    rng = np.random.default_rng(S * 3 + hd + nHq)
    pos = S - 1
    cap = S + 3
    row_w, row_g = nKv * hd // 4, nKv * hd // 32
    # cache rows [0, pos) from the oracle's KV quantizer on random rows
    kq = np.zeros((cap, row_w), np.uint32)
    ks = np.zeros((cap, row_g), np.float32)
    vq = np.zeros((cap, row_w), np.uint32)
    vs = np.zeros((cap, row_g), np.float32)
    if pos > 0:
        kq[:pos], ks[:pos] = [a.reshape(pos, -1) for a in orc.kv_quant(f16r(rng, pos * nKv * hd))]
        vq[:pos], vs[:pos] = [a.reshape(pos, -1) for a in orc.kv_quant(f16r(rng, pos * nKv * hd))]
    q, k, v = f16r(rng, nHq * hd, 2), f16r(rng, nKv * hd, 2), f16r(rng, nKv * hd, 2)
    qw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float16).view(np.uint16)
    kw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float16).view(np.uint16)
    theta, eps = np.float32(1e6), np.float32(1e-6)
    qr, kq_p, ks_p, vq_p, vs_p = orc.attn_prep_q8(q, k, v, qw, kw, nHq, nKv, hd, pos, theta, eps)
    kq[pos], ks[pos], vq[pos], vs[pos] = kq_p, ks_p, vq_p, vs_p
    ref = orc.attn_decode_q8(qr, kq.ravel(), ks.ravel(), vq.ravel(), vs.ravel(), S, nHq, nKv, hd)
    d = [ctx.upload(a) for a in (q, k, v, qw, kw)]
    cache = [ctx.upload(kq), ctx.upload(ks), ctx.upload(vq), ctx.upload(vs)]
    ctx.write(cache[0], np.full(row_w, 0xA5A5A5A5, np.uint32), pos * row_w * 4)   # row pos holds garbage
    ctx.write(cache[1], np.full(row_g, 0x7FC00000, np.uint32), pos * row_g * 4)   # (a NaN scale)
    out = ctx.zeros(nHq * hd * 4)
    oq, os_ = ctx.zeros(nHq * hd), ctx.zeros(nHq * hd // 8)
    for rep in range(2):                                   # the combine counter must be reset between launches
        ctx.call("ti_attn_step_q8", *d, *cache, out, nHq, nKv, hd, pos, cap, theta, eps, max_splits,
                 oq if rep else None, os_ if rep else None)
        got = ctx.download(out, np.float32, nHq * hd)
        assert rel_err(got, ref) < TOL, rep
    # the output quantized as o_proj's linearQ would (quantQ8), bit-exact on the f32 output
    rq, rs, _ = orc.quant_act_q8(got)
    assert np.array_equal(ctx.download(oq, np.uint32, nHq * hd // 4), rq)
    assert np.array_equal(ctx.download(os_, np.float32, nHq * hd // 32), rs)
    gk = ctx.download(cache[0], np.uint32, cap * row_w).reshape(cap, row_w)
    gks = ctx.download(cache[1], np.float32, cap * row_g).reshape(cap, row_g)
    gv = ctx.download(cache[2], np.uint32, cap * row_w).reshape(cap, row_w)
    assert np.array_equal(gk[pos], kq_p) and np.array_equal(gv[pos], vq_p)
    assert np.array_equal(gks[pos], ks_p)
    assert np.array_equal(gk[:pos], kq[:pos]) and np.all(gk[pos + 1:] == 0)


def test_attn_step_rejects_out_of_capacity(ctx):
    b = ctx.zeros(1 << 16)
    with pytest.raises(abi.TIError):
        ctx.call("ti_attn_step_q8", b, b, b, b, b, b, b, b, b, b, 16, 8, 128, 10, 10, np.float32(1e6),
                 np.float32(1e-6), 0, None, None)
