"""GPU parity for the int3 MoE expert path of LFM2.5 (models/lfm25.js).

- int4 -> int3 requant: planes and f16 scales bit-exact against the oracle.
- router: expert ids exact; weights within 1e-6 relative (sigmoid uses expf).
- pair-indexed int3 GEMV (f32 activation) and the expert-grouped int3 x int8 GEMM:
  max error <= 1e-4 of the output's max magnitude against the f64 oracle, the GEMM
  after the same per-32 int8 quantization, which is bit-exact (checked in
  test_gpu_gemv.py).
- combine and swiglu: bit-exact (same operation order in f32).
Shapes: LFM2.5-8B-A1B experts (hidden 2048, expert intermediate 1792, 32 experts,
top-4) at batch 1 and 16, plus ragged and edge cases.
"""
import numpy as np
import pytest

from tabinfer_amd import abi

pytestmark = pytest.mark.gpu

H, I, NE, TOPK = 2048, 1792, 32, 4


@pytest.fixture(scope="module")
def ctx():
    c = abi.Ctx(0)
    yield c
    c.close()


def norm_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def rand_planes(rng, rows, K):
    ng = rows * (K // 32)
    p3 = rng.integers(0, 2 ** 32, ng * 3, dtype=np.uint64).astype(np.uint32)
    s3 = rng.uniform(0.005, 0.02, ng).astype(np.float16).view(np.uint16)
    return p3, s3


def gpu_requant(ctx, pack4, sc4, rows, K):
    ng = rows * (K // 32)
    dp, ds = ctx.upload(pack4), ctx.upload(sc4)
    d3, dsc = ctx.zeros(ng * 12), ctx.zeros(ng * 2)
    ctx.call("ti_requant43", dp, ds, rows, K, d3, dsc)
    out = ctx.download(d3, np.uint32, ng * 3), ctx.download(dsc, np.uint16, ng)
    for b in (dp, ds, d3, dsc):
        b.free()
    return out


# ---- requant -------------------------------------------------------------------------
def test_requant43_expert_matrix(ctx, orc):
    rng = np.random.default_rng(5)
    rows, K = I, H
    w = (rng.standard_normal(rows * K) * 0.02).astype(np.float32)
    bf = (w.view(np.uint32) >> 16).astype(np.uint16)
    pack4, sc4 = orc.quant_int4_bf16(bf, rows, K)
    got = gpu_requant(ctx, pack4, sc4, rows, K)
    want = orc.requant43(pack4, sc4, rows, K)
    assert np.array_equal(got[0], want[0])
    assert np.array_equal(got[1], want[1])


def test_requant43_edge_groups(ctx, orc):
    rng = np.random.default_rng(6)
    rows, K = 64, 256
    ng = rows * K // 32
    q = rng.integers(-8, 8, (ng, 32))
    q[0] = 0                                             # all-zero group
    q[1] = rng.integers(-1, 2, 32)                       # m = 1
    q[2, :] = 0
    q[2, 0] = 7                                          # m = 7: ratio 4/7
    q[3] = np.tile([-8, 7, 2, -2], 8)                    # m = 8: .5 ties
    q[4] = np.tile([6, -6, 3, -3], 8)                    # m = 6: ratio 2/3
    words = ((q.reshape(-1, 8) + 8).astype(np.uint32) << (np.arange(8, dtype=np.uint32) * 4)).sum(1)
    pack4 = words.astype(np.uint32)
    sc4 = rng.uniform(1e-3, 0.1, ng).astype(np.float16).view(np.uint16)
    sc4[5] = 0x0001                                      # smallest subnormal
    sc4[6] = 0x7BFF                                      # 65504: s4*m/4 overflows f16 for m >= 5
    sc4[7] = 0x8400                                      # negative scale
    sc4[8] = 0x0000
    got = gpu_requant(ctx, pack4, sc4, rows, K)
    want = orc.requant43(pack4, sc4, rows, K)
    assert np.array_equal(got[0], want[0])
    assert np.array_equal(got[1], want[1])
    assert list(want[0][0:3]) == [0, 0, 0xFFFFFFFF]


# ---- router --------------------------------------------------------------------------
@pytest.mark.parametrize("T,nE,topk", [(1, NE, TOPK), (16, NE, TOPK), (3, 256, 8), (5, 64, 64), (2, 7, 3)])
def test_router_random(ctx, orc, T, nE, topk):
    rng = np.random.default_rng(T * 1000 + nE)
    logits = rng.standard_normal(T * nE).astype(np.float32)
    bias = (rng.standard_normal(nE) * 0.1).astype(np.float32)
    dl, db = ctx.upload(logits), ctx.upload(bias)
    di, dw = ctx.zeros(T * topk * 4), ctx.zeros(T * topk * 4)
    ctx.call("ti_router", dl, db, T, nE, topk, di, dw)
    idx, wt = ctx.download(di, np.int32, T * topk), ctx.download(dw, np.float32, T * topk)
    oi, ow = orc.router(logits, bias, T, nE, topk)
    assert np.array_equal(idx, oi)
    assert np.abs(wt - ow).max() <= 1e-6 * np.abs(ow).max()
    for b in (dl, db, di, dw):
        b.free()


def test_router_ties_and_null_bias(ctx, orc):
    logits = np.array([0.0, 2.0, 2.0, -1.0, 1.0, 2.0], np.float32)
    dl = ctx.upload(logits)
    di, dw = ctx.zeros(16), ctx.zeros(16)
    ctx.call("ti_router", dl, None, 1, 6, 4, di, dw)
    assert list(ctx.download(di, np.int32, 4)) == [1, 2, 5, 4]
    oi, ow = orc.router(logits, np.zeros(6, np.float32), 1, 6, 4)
    assert np.abs(ctx.download(dw, np.float32, 4) - ow).max() <= 1e-6
    for b in (dl, di, dw):
        b.free()


# ---- pair-indexed GEMV (T = 1) -------------------------------------------------------
def run_gemv(ctx, x, p3, s3, idx, pairs, N, K, in_stride, xdiv, nE, sentinel=np.nan):
    dx, d3, ds, di = ctx.upload(x), ctx.upload(p3), ctx.upload(s3), ctx.upload(idx)
    y0 = np.full(pairs * N, sentinel, np.float32)
    dy = ctx.upload(y0)
    ctx.call("ti_moe_gemv_q3", dx, d3, ds, di, dy, pairs, N, K, in_stride, xdiv, nE)
    y = ctx.download(dy, np.float32, pairs * N)
    for b in (dx, d3, ds, di, dy):
        b.free()
    return y


@pytest.mark.parametrize("N,K,pairs,xdiv,in_stride,nE", [
    (I, H, TOPK, TOPK, H, 8),        # gate / up at batch 1: one token, 4 pairs
    (H, I, TOPK, 1, I, 8),           # down: per-pair activation rows
    (37, 4096, 3, 1, 4104, 5),       # two groups per lane, padded row stride, ragged N
    (16, 32, 2, 2, 32, 3),           # one group
    (100, 2016, 6, 3, 2048, 4),      # gpr = 63
])
def test_moe_gemv_q3(ctx, orc, N, K, pairs, xdiv, in_stride, nE):
    rng = np.random.default_rng(N + K + pairs)
    p3, s3 = rand_planes(rng, nE * N, K)
    rows_x = (pairs - 1) // xdiv + 1
    x = rng.standard_normal(rows_x * in_stride).astype(np.float32)
    idx = rng.permutation(nE)[:pairs].astype(np.int32) if pairs <= nE else rng.integers(0, nE, pairs).astype(np.int32)
    y = run_gemv(ctx, x, p3, s3, idx, pairs, N, K, in_stride, xdiv, nE)
    want = orc.moe_gemv_q3(x, p3, s3, idx, pairs, N, K, in_stride, xdiv)
    assert norm_err(y, want) <= 1e-4


def test_moe_gemv_q3_wide_dynamic_range(ctx, orc):
    # activations spanning 2^-20 .. 2^10 inside one group: the exact fixed-point dot keeps
    # the small terms that a per-group int8 quantization would drop
    rng = np.random.default_rng(9)
    N, K, nE = 64, 256, 2
    p3, s3 = rand_planes(rng, nE * N, K)
    x = (rng.standard_normal(K) * np.exp2(rng.integers(-20, 10, K))).astype(np.float32)
    idx = np.array([1], np.int32)
    y = run_gemv(ctx, x, p3, s3, idx, 1, N, K, K, 1, nE)
    want = orc.moe_gemv_q3(x, p3, s3, idx, 1, N, K, K, 1)
    assert norm_err(y, want) <= 1e-5


def test_moe_gemv_q3_zero_and_bad_ids(ctx, orc):
    rng = np.random.default_rng(10)
    N, K, nE = 48, 128, 4
    p3, s3 = rand_planes(rng, nE * N, K)
    x = np.zeros(K, np.float32)
    idx = np.array([2, -1, 4, 0], np.int32)              # -1 and 4 are out of range
    y = run_gemv(ctx, x, p3, s3, idx, 4, N, K, K, 4, nE).reshape(4, N)
    assert np.all(y[0] == 0.0) and np.all(y[3] == 0.0)
    assert np.all(np.isnan(y[1])) and np.all(np.isnan(y[2]))   # untouched


# ---- expert-grouped GEMM (T > 1) -----------------------------------------------------
def run_gemm(ctx, src, src_rows, p3, s3, ridx, P, N, K, src_div, nE, sentinel=np.nan):
    ds_, d3, dsc, dr = ctx.upload(src), ctx.upload(p3), ctx.upload(s3), ctx.upload(ridx)
    dy = ctx.upload(np.full(P * N, sentinel, np.float32))
    ctx.call("ti_moe_gemm_q3", ds_, src_rows, d3, dsc, dr, dy, P, N, K, src_div, nE)
    y = ctx.download(dy, np.float32, P * N)
    for b in (ds_, d3, dsc, dr, dy):
        b.free()
    return y


def oracle_gemm(orc, src, src_rows, p3, s3, ridx, P, N, K, src_div):
    xq, xs = orc.quant_act_q8_t(src, src_rows, K)
    return orc.moe_gemm_q3(xq, xs, p3, s3, ridx, P, N, K, src_div)


def route(rng, orc, T, nE, topk):
    logits = rng.standard_normal(T * nE).astype(np.float32)
    idx, _ = orc.router(logits, np.zeros(nE, np.float32), T, nE, topk)
    return idx


@pytest.mark.parametrize("T,N,K,per_pair", [
    (16, I, H, False),     # gate / up at batch 16: 64 pairs, source row = token
    (16, H, I, True),      # down: source row = pair
    (5, 40, 4096, False),  # two groups per lane, ragged N
    (70, 96, 512, True),   # 280 pairs: more than one 256-id scan chunk
])
def test_moe_gemm_q3(ctx, orc, T, N, K, per_pair):
    rng = np.random.default_rng(T * 7 + N)
    nE = NE
    P = T * TOPK
    ridx = route(rng, orc, T, nE, TOPK)
    src_rows, src_div = (P, 1) if per_pair else (T, TOPK)
    p3, s3 = rand_planes(rng, nE * N, K)
    src = rng.standard_normal(src_rows * K).astype(np.float32)
    y = run_gemm(ctx, src, src_rows, p3, s3, ridx, P, N, K, src_div, nE)
    want = oracle_gemm(orc, src, src_rows, p3, s3, ridx, P, N, K, src_div)
    assert norm_err(y, want) <= 1e-4


def test_moe_gemm_q3_skewed_and_bad_ids(ctx, orc):
    rng = np.random.default_rng(11)
    nE, N, K, P = 8, 64, 256, 300
    ridx = np.full(P, 3, np.int32)                       # one expert takes almost everything
    ridx[::7] = 5
    ridx[10], ridx[299] = 8, -2                          # out of range: rows untouched
    p3, s3 = rand_planes(rng, nE * N, K)
    src = rng.standard_normal(P * K).astype(np.float32)
    y = run_gemm(ctx, src, P, p3, s3, ridx, P, N, K, 1, nE).reshape(P, N)
    good = (ridx >= 0) & (ridx < nE)
    r2 = np.where(good, ridx, 0).astype(np.int32)
    want = oracle_gemm(orc, src, P, p3, s3, r2, P, N, K, 1).reshape(P, N)
    assert norm_err(y[good], want[good]) <= 1e-4
    assert np.all(np.isnan(y[~good]))


def test_moe_gemm_matches_gemv_at_one_token(ctx, orc):
    # T = 1 through the GEMM (int8 activation) stays within int8 quantization error of
    # the f32-activation GEMV
    rng = np.random.default_rng(12)
    nE, N, K = 8, 256, 1024
    p3, s3 = rand_planes(rng, nE * N, K)
    x = rng.standard_normal(K).astype(np.float32)
    idx = np.array([1, 6, 2, 0], np.int32)
    yv = run_gemv(ctx, x, p3, s3, idx, 4, N, K, K, 4, nE)
    ym = run_gemm(ctx, x, 1, p3, s3, idx, 4, N, K, 4, nE)
    assert norm_err(ym, yv) <= 2e-2


# ---- swiglu and combine ----------------------------------------------------------------
def test_swiglu_and_combine_bit_exact(ctx, orc):
    rng = np.random.default_rng(13)
    T = 16
    g = rng.standard_normal(T * TOPK * I).astype(np.float32)
    u = rng.standard_normal(T * TOPK * I).astype(np.float32)
    dg, du, dy = ctx.upload(g), ctx.upload(u), ctx.zeros(g.nbytes)
    ctx.call("ti_swiglu", dg, du, dy, g.size)
    act = ctx.download(dy, np.float32, g.size)
    want = (g / (np.float32(1) + np.exp(-g)) * u).astype(np.float32)
    assert np.abs(act - want).max() <= 2e-6 * np.abs(want).max()
    x = rng.standard_normal(T * H).astype(np.float32)
    o = rng.standard_normal(T * TOPK * H).astype(np.float32)
    wt = rng.uniform(0, 0.5, T * TOPK).astype(np.float32)
    dx, do, dw = ctx.upload(x), ctx.upload(o), ctx.upload(wt)
    ctx.call("ti_moe_combine", dx, do, dw, H, TOPK, T)
    assert np.array_equal(ctx.download(dx, np.float32, T * H), orc.moe_combine(x, o, wt, H, TOPK, T))
    for b in (dg, du, dy, dx, do, dw):
        b.free()


# ---- one MoE block, end to end ---------------------------------------------------------
@pytest.mark.parametrize("T", [1, 16])
def test_moe_block(ctx, orc, T):
    """router -> experts (GEMV at T = 1, GEMM at T > 1) -> swiglu -> down -> combine,
    as models/lfm25.js:2145-2166 sequences them, against the oracle chain."""
    rng = np.random.default_rng(100 + T)
    nE, P = NE, T * TOPK
    w13 = [rand_planes(rng, nE * I, H) for _ in range(2)]
    w2 = rand_planes(rng, nE * H, I)
    normed = rng.standard_normal(T * H).astype(np.float32)
    logits = rng.standard_normal(T * nE).astype(np.float32)
    bias = (rng.standard_normal(nE) * 0.05).astype(np.float32)
    x = rng.standard_normal(T * H).astype(np.float32)
    d = {k: ctx.upload(v) for k, v in dict(normed=normed, logits=logits, bias=bias, x=x,
                                             p1=w13[0][0], s1=w13[0][1], p3=w13[1][0], s3=w13[1][1],
                                             p2=w2[0], s2=w2[1]).items()}
    for k, n in dict(idx=P, wt=P, gate=P * I, up=P * I, act=P * I, out=P * H).items():
        d[k] = ctx.zeros(n * 4)
    ctx.call("ti_router", d["logits"], d["bias"], T, nE, TOPK, d["idx"], d["wt"])
    if T == 1:
        ctx.call("ti_moe_gemv_q3", d["normed"], d["p1"], d["s1"], d["idx"], d["gate"], P, I, H, H, TOPK, nE)
        ctx.call("ti_moe_gemv_q3", d["normed"], d["p3"], d["s3"], d["idx"], d["up"], P, I, H, H, TOPK, nE)
        ctx.call("ti_swiglu", d["gate"], d["up"], d["act"], P * I)
        ctx.call("ti_moe_gemv_q3", d["act"], d["p2"], d["s2"], d["idx"], d["out"], P, H, I, I, 1, nE)
    else:
        ctx.call("ti_moe_gemm_q3", d["normed"], T, d["p1"], d["s1"], d["idx"], d["gate"], P, I, H, TOPK, nE)
        ctx.call("ti_moe_gemm_q3", d["normed"], T, d["p3"], d["s3"], d["idx"], d["up"], P, I, H, TOPK, nE)
        ctx.call("ti_swiglu", d["gate"], d["up"], d["act"], P * I)
        ctx.call("ti_moe_gemm_q3", d["act"], P, d["p2"], d["s2"], d["idx"], d["out"], P, H, I, 1, nE)
    ctx.call("ti_moe_combine", d["x"], d["out"], d["wt"], H, TOPK, T)
    got = ctx.download(d["x"], np.float32, T * H)
    idx, wt = orc.router(logits, bias, T, nE, TOPK)
    assert np.array_equal(ctx.download(d["idx"], np.int32, P), idx)
    if T == 1:
        g = orc.moe_gemv_q3(normed, *w13[0], idx, P, I, H, H, TOPK)
        u = orc.moe_gemv_q3(normed, *w13[1], idx, P, I, H, H, TOPK)
        a = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
        o = orc.moe_gemv_q3(a, *w2, idx, P, H, I, I, 1)
    else:
        g = oracle_gemm(orc, normed, T, *w13[0], idx, P, I, H, TOPK)
        u = oracle_gemm(orc, normed, T, *w13[1], idx, P, I, H, TOPK)
        a = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
        # Teacher forcing at the re-quantization point: the down projection quantizes the
        # expert activations to int8 again, and a code flips wherever the GPU's f32 value
        # and the oracle's f64 value sit on two sides of a rounding boundary. The GPU's own
        # activations are held to the oracle's first; then they enter the oracle's down
        # projection, which quantizes them by the same rule, so the block output is held
        # to the same bar as at T = 1.
        gact = ctx.download(d["act"], np.float32, P * I)
        assert norm_err(gact, a) <= 1e-4
        o = oracle_gemm(orc, gact, P, *w2, idx, P, H, I, 1)
    want = x.astype(np.float64) + (wt.astype(np.float64).reshape(T, TOPK, 1) * o.reshape(T, TOPK, H)).sum(1).ravel()
    assert norm_err(got - x, want - x) <= 1e-4
    for b in d.values():
        b.free()


def test_moe_shape_errors(ctx):
    d = ctx.zeros(4096)
    with pytest.raises(abi.TIError):
        ctx.call("ti_moe_gemv_q3", d, d, d, d, d, 1, 16, 48, 48, 1, 4)        # K % 32
    with pytest.raises(abi.TIError):
        ctx.call("ti_moe_gemv_q3", d, d, d, d, d, 1, 16, 8192, 8192, 1, 4)    # K > 4096
    with pytest.raises(abi.TIError):
        ctx.call("ti_moe_gemm_q3", d, 1, d, d, d, d, 4, 16, 64, 1, 4)         # pair 3 reads row 3 of 1
    with pytest.raises(abi.TIError):
        ctx.call("ti_router", d, None, 1, 300, 4, d, d)                       # nE > 256
    d.free()


# ---- the fused decode block ---------------------------------------------------------------
@pytest.mark.parametrize("H,I,nE,topk", [(H, I, NE, TOPK), (4096, 1024, 8, 2), (1024, 4096, 100, 8), (512, 256, 256, 1)])
def test_moe_decode_fused_matches_chain(ctx, orc, H, I, nE, topk):
    """ti_moe_decode_q3 (2 launches) against the oracle chain, and its routing against
    ti_router bit for bit."""
    rng = np.random.default_rng(H + I + nE + topk)
    w1, w3 = rand_planes(rng, nE * I, H), rand_planes(rng, nE * I, H)
    w2 = rand_planes(rng, nE * H, I)
    normed = rng.standard_normal(H).astype(np.float32)
    logits = rng.standard_normal(nE).astype(np.float32)
    bias = (rng.standard_normal(nE) * 0.05).astype(np.float32)
    x = rng.standard_normal(H).astype(np.float32)
    d = {k: ctx.upload(v) for k, v in dict(normed=normed, logits=logits, bias=bias, x=x, p1=w1[0], s1=w1[1],
                                             p3=w3[0], s3=w3[1], p2=w2[0], s2=w2[1]).items()}
    d["idx"], d["wt"], d["act"] = ctx.zeros(topk * 4), ctx.zeros(topk * 4), ctx.zeros(topk * I * 4)
    d["ridx"], d["rwt"] = ctx.zeros(topk * 4), ctx.zeros(topk * 4)
    ctx.call("ti_moe_decode_q3", d["x"], d["normed"], d["logits"], d["bias"], d["p1"], d["s1"], d["p3"], d["s3"],
             d["p2"], d["s2"], d["idx"], d["wt"], d["act"], H, I, nE, topk)
    ctx.call("ti_router", d["logits"], d["bias"], 1, nE, topk, d["ridx"], d["rwt"])
    idx = ctx.download(d["idx"], np.int32, topk)
    assert np.array_equal(idx, ctx.download(d["ridx"], np.int32, topk))
    assert np.array_equal(ctx.download(d["wt"], np.float32, topk), ctx.download(d["rwt"], np.float32, topk))
    oi, ow = orc.router(logits, bias, 1, nE, topk)
    assert np.array_equal(idx, oi)
    g = orc.moe_gemv_q3(normed, *w1, oi, topk, I, H, H, topk)
    u = orc.moe_gemv_q3(normed, *w3, oi, topk, I, H, H, topk)
    a = g / (1.0 + np.exp(-g)) * u
    assert norm_err(ctx.download(d["act"], np.float32, topk * I), a) <= 1e-4
    o = orc.moe_gemv_q3(a.astype(np.float32), *w2, oi, topk, H, I, I, 1)
    want = (ow.astype(np.float64)[:, None] * o.reshape(topk, H)).sum(0)
    got = ctx.download(d["x"], np.float32, H).astype(np.float64) - x
    assert norm_err(got, want) <= 1e-4
    for b in d.values():
        b.free()


def test_moe_decode_rejects_bad_shapes(ctx):
    dd = ctx.zeros(4096)
    args = [dd] * 13
    with pytest.raises(abi.TIError):
        ctx.call("ti_moe_decode_q3", *args, 2048, 1792, 32, 3)      # topk 3
    with pytest.raises(abi.TIError):
        ctx.call("ti_moe_decode_q3", *args, 2048, 1792, 300, 4)     # nE > 256
    with pytest.raises(abi.TIError):
        ctx.call("ti_moe_decode_q3", *args, 8192, 1792, 32, 4)      # H > 4096
    dd.free()


# ---- the fused T > 1 block ------------------------------------------------------------------
@pytest.mark.parametrize("T,H,I,nE,topk", [(16, H, I, NE, TOPK), (3, H, I, NE, TOPK), (8, 4096, 1024, 8, 2),
                                           (5, 1024, 4096, 100, 8)])
def test_moe_prefill_fused_matches_chain(ctx, orc, T, H, I, nE, topk):
    """ti_moe_prefill_q3 (5 launches) against the chain of separate calls it replaces
    (ti_router, ti_moe_gemm_q3 x 2, ti_swiglu, ti_moe_gemm_q3, ti_moe_combine): routing,
    gate/up, activations, expert outputs and the residual bit for bit; and the routing
    against the oracle's."""
    rng = np.random.default_rng(7 * T + H + I + nE + topk)
    P = T * topk
    w1, w3 = rand_planes(rng, nE * I, H), rand_planes(rng, nE * I, H)
    w2 = rand_planes(rng, nE * H, I)
    normed = rng.standard_normal(T * H).astype(np.float32)
    logits = rng.standard_normal(T * nE).astype(np.float32)
    bias = (rng.standard_normal(nE) * 0.05).astype(np.float32)
    x = rng.standard_normal(T * H).astype(np.float32)
    d = {k: ctx.upload(v) for k, v in dict(normed=normed, logits=logits, bias=bias, p1=w1[0], s1=w1[1], p3=w3[0],
                                             s3=w3[1], p2=w2[0], s2=w2[1]).items()}
    runs = []
    for fused in (True, False):
        b = dict(x=ctx.upload(x))
        for k, n in dict(idx=P, wt=P, gate=P * I, up=P * I, act=P * I, out=P * H).items():
            b[k] = ctx.zeros(n * 4)
        if fused:
            ctx.call("ti_moe_prefill_q3", b["x"], d["normed"], d["logits"], d["bias"], d["p1"], d["s1"], d["p3"],
                     d["s3"], d["p2"], d["s2"], b["idx"], b["wt"], b["gate"], b["up"], b["act"], b["out"],
                     T, H, I, nE, topk)
        else:
            ctx.call("ti_router", d["logits"], d["bias"], T, nE, topk, b["idx"], b["wt"])
            ctx.call("ti_moe_gemm_q3", d["normed"], T, d["p1"], d["s1"], b["idx"], b["gate"], P, I, H, topk, nE)
            ctx.call("ti_moe_gemm_q3", d["normed"], T, d["p3"], d["s3"], b["idx"], b["up"], P, I, H, topk, nE)
            ctx.call("ti_swiglu", b["gate"], b["up"], b["act"], P * I)
            ctx.call("ti_moe_gemm_q3", b["act"], P, d["p2"], d["s2"], b["idx"], b["out"], P, H, I, 1, nE)
            ctx.call("ti_moe_combine", b["x"], b["out"], b["wt"], H, topk, T)
        runs.append({k: ctx.download(v, np.int32 if k == "idx" else np.float32,
                                     {"x": T * H, "idx": P, "wt": P, "out": P * H}.get(k, P * I))
                     for k, v in b.items()})
        for v in b.values():
            v.free()
    for k in runs[0]:
        assert np.array_equal(runs[0][k].view(np.uint32), runs[1][k].view(np.uint32)), k
    oi, ow = orc.router(logits, bias, T, nE, topk)
    assert np.array_equal(runs[0]["idx"], oi)
    # the fused block against the oracle itself (models/lfm25.js:2145-2166), as
    # test_moe_block holds the chain: the expert activations first, then the block output
    # with the down projection teacher-forced on the GPU's activations (its int8
    # re-quantization is the only place an f32/f64 difference can flip a code)
    g = oracle_gemm(orc, normed, T, *w1, oi, P, I, H, topk)
    u = oracle_gemm(orc, normed, T, *w3, oi, P, I, H, topk)
    a = g / (1.0 + np.exp(-g)) * u
    assert norm_err(runs[0]["act"], a) <= 1e-4
    o = oracle_gemm(orc, runs[0]["act"], P, *w2, oi, P, H, I, 1)
    want = (ow.astype(np.float64).reshape(T, topk, 1) * o.reshape(T, topk, H)).sum(1).ravel()
    assert norm_err(runs[0]["x"].astype(np.float64) - x, want) <= 1e-4
    for v in d.values():
        v.free()


def test_moe_prefill_rejects_bad_shapes(ctx):
    d = ctx.zeros(4096)
    args = [d] * 16
    with pytest.raises(abi.TIError):
        ctx.call("ti_moe_prefill_q3", *args, 2, 48, 64, 8, 2)          # H % 32
    with pytest.raises(abi.TIError):
        ctx.call("ti_moe_prefill_q3", *args, 2, 64, 8192, 8, 2)        # I > 4096
    with pytest.raises(abi.TIError):
        ctx.call("ti_moe_prefill_q3", *args, 2, 64, 64, 300, 2)        # nE > 256
    with pytest.raises(abi.TIError):
        ctx.call("ti_moe_prefill_q3", *args, 0, 64, 64, 8, 2)          # T = 0
    d.free()
