"""ti_attn_decode_q8_noalloc (split partials in the library's file-scope device array,
nothing allocated) against ti_attn_decode_q8 (partials in the context's scratch): the same
kernels, so the outputs must agree bit for bit. Two calls in a row, the second smaller
(fewer heads and positions, fewer splits), so stale partials of the first call would show;
then an over-size call is refused. Both outputs are also held to the oracle (1e-3)."""
import ctypes as C

import numpy as np
import pytest

from tabinfer_amd import abi

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _hip():
    h = C.CDLL("libamdhip64.so")
    h.hipDeviceSynchronize.restype = C.c_int
    return h


def _case(ctx, orc, rng, S, nHq, nKv, hd):
    kq, ks = orc.kv_quant(rng.standard_normal(S * nKv * hd).astype(np.float16).astype(np.float32))
    vq, vs = orc.kv_quant(rng.standard_normal(S * nKv * hd).astype(np.float16).astype(np.float32))
    qr = rng.standard_normal(nHq * hd).astype(np.float32)
    ref = orc.attn_decode_q8(qr, kq, ks, vq, vs, S, nHq, nKv, hd)
    return [ctx.upload(a) for a in (qr, kq, ks, vq, vs)], ref


def rel_err(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / np.max(np.abs(ref)))


def test_noalloc_matches_context_path(orc):
    hip = _hip()
    lib = abi.lib()
    rng = np.random.default_rng(77)
    with abi.Ctx(0) as ctx:
        # (S, nHq, nKv, hd, nsplit): 16 heads x 256 splits = the whole array, then a smaller call
        for S, nHq, nKv, hd, nsplit in [(32768, 16, 8, 128, 0), (5000, 4, 2, 64, 7)]:
            print("[noalloc] case S=%d nHq=%d nKv=%d hd=%d nsplit=%d" % (S, nHq, nKv, hd, nsplit), flush=True)
            bufs, ref = _case(ctx, orc, rng, S, nHq, nKv, hd)
            a, b = ctx.zeros(nHq * hd * 4), ctx.zeros(nHq * hd * 4)
            ctx.call("ti_attn_decode_q8", *bufs, a, S, nHq, nKv, hd, nsplit)
            ctx.sync()
            abi.check(lib.ti_attn_decode_q8_noalloc(None, *[int(x) for x in bufs], int(b), S, nHq, nKv, hd, nsplit))
            assert hip.hipDeviceSynchronize() == 0
            ga = ctx.download(a, np.float32, nHq * hd)
            gb = ctx.download(b, np.float32, nHq * hd)
            assert np.array_equal(ga, gb)
            assert rel_err(gb, ref) < TOL
        # more head-splits than the array holds: refused before anything is launched
        rc = lib.ti_attn_decode_q8_noalloc(None, *[int(x) for x in bufs], int(b), 5000, 64, 8, 64, 65)
        assert rc == abi.TI_ERR_INVALID and b"scratch array" in lib.ti_last_error()
