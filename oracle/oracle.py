"""numpy wrapper over oracle/libti_oracle.so — the CPU oracle.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker. The product path
(tabinfer_amd/) never imports this module.

Each wrapper mirrors one C function in ti_oracle.h; the C file cites the
reference file:line each one restates.
"""
import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "libti_oracle.so")


def build(force=False):
    if force or not os.path.exists(_SO):
        subprocess.check_call(["make", "-s", "-C", _HERE, "-B" if force else "--no-print-directory"])


def _load():
    if not os.path.exists(_SO):
        build()
    return C.CDLL(_SO)


_L = _load()

_f = C.c_float
_i = C.c_int
_p = C.c_void_p


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def _sig(name, res, args):
    fn = getattr(_L, name)
    fn.restype = res
    fn.argtypes = args
    return fn


_sig("or_f32_to_f16_q3", C.c_uint16, [_f])
_sig("or_f32_to_f16_eng", C.c_uint16, [_f])
_sig("or_f16_to_f32", C.c_double, [C.c_uint16])
_sig("or_bf16_to_f32", _f, [C.c_uint16])
_sig("or_quant_int4_bf16", None, [_p, _i, _i, _p, _p])
_sig("or_quant_act_q8", None, [_p, _i, _p, _p, _p])
_sig("or_quant_act_q8_t", None, [_p, _i, _i, _p, _p])
_sig("or_rmsnorm_q8", None, [_p, _p, _i, _f, _p, _p, _p])
_sig("or_rmsnorm", None, [_p, _p, _i, _i, _f, _p])
_sig("or_group_dots_q4_q8", None, [_p, _p, _i, _i, _p])
_sig("or_gemv_q4_q8", None, [_p, _p, _p, _p, _i, _i, _p])
_sig("or_quant_tern_bf16", _i, [_p, _i, _i, _p, _p])
_sig("or_gemv_tern2", None, [_p, _p, _p, _p, _i, _i, _p])
_sig("or_gateup_silu_tern2", None, [_p, _p, _p, _p, _p, _p, _i, _i, _p])
_sig("or_gemv_q4_f32", None, [_p, _p, _p, _i, _i, _p])
_sig("or_gateup_silu_q4", None, [_p, _p, _p, _p, _p, _p, _i, _i, _p])
_sig("or_gemm_q4_q8", None, [_p, _p, _p, _p, _i, _i, _i, _p])
_sig("or_kv_quant", None, [_p, _i, _p, _p])
_sig("or_snorm_dequant", C.c_double, [C.c_uint32, _i, _f])
_sig("or_attn_prep_q8", None, [_p, _p, _p, _p, _p, _i, _i, _i, _i, _f, _f, _p, _p, _p, _p, _p])
_sig("or_rope_norm_row", None, [_p, _p, _i, _i, _f, _f, _i, _p])
_sig("or_attn_decode_q8", None, [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p])
_sig("or_attn_causal_q8", None, [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p])
_sig("or_attn_causal_q8_kvheads", None, [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p])
_sig("or_embed", None, [_p, _p, _i, _i, _p])
_sig("or_argmax", _i, [_p, _i])
_sig("or_pcg", C.c_uint32, [C.c_uint32])
_sig("or_seed_next", C.c_uint32, [C.c_uint32])
_sig("or_gumbel_noise", None, [_p, _i, C.c_uint32, _f])
_sig("or_tern_pack", None, [_p, _i, _i, _p, _p])
_sig("or_tern_quant_act_n2", _f, [_p, _i, _p, _p])
_sig("or_tern_quant_act_wasm", _f, [_p, _i, _p, _p])
_sig("or_tern_gemv_scalar", None, [_p, _p, _p, _p, _i, _i, _p])
_sig("or_tern_gemv_dequant", None, [_p, _p, _p, _i, _i, _p])
_sig("or_tern_block_dots", None, [_p, _p, _i, _i, _p])
_sig("or_n2_fixture", None, [_i, _i, C.c_uint64, _p, _p, _p, _p, _p, _p])
_sig("or_has_avx2", _i, [])
_sig("or_tern_gemv_avx2", None, [_p, _p, _p, _p, _i, _i, _p])
_sig("or_tern_gemv_avx2_mt", None, [_p, _p, _p, _p, _i, _i, _p, _i])
_sig("or_tern_pool_start", _i, [_i])
_sig("or_tern_pool_stop", None, [])
_sig("or_tern_pool_run", None, [_p, _i])
_sig("or_tern_set_serial", None, [_p, _i])
_sig("or_n2_rmsnorm", None, [_p, _p, _i, _f, _p])
_sig("or_n2_rmsnorm_heads", None, [_p, _p, _i, _i, _f])
_sig("or_n2_rope_table", None, [_i, _i, _f, _p])
_sig("or_n2_rope_with_table", None, [_p, _i, _i, _p])
_sig("or_n2_swiglu", None, [_p, _p, _i, _p])
_sig("or_n2_attention", None, [_p, _p, _p, _i, _i, _i, _i, _p])
_sig("or_n2_argmax", _i, [_p, _i])
_sig("or_requant43", None, [_p, _p, _i, _i, _p, _p])
_sig("or_router", None, [_p, _p, _i, _i, _i, _p, _p])
_sig("or_moe_gemv_q3", None, [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p])
_sig("or_moe_gemm_q3", None, [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p])
_sig("or_moe_combine", None, [_p, _p, _p, _i, _i, _i])


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---- f16 -------------------------------------------------------------------
def f32_to_f16_q3(v):
    return int(_L.or_f32_to_f16_q3(float(np.float32(v))))


def f32_to_f16_eng(v):
    return int(_L.or_f32_to_f16_eng(float(np.float32(v))))


def f16_to_f32(h):
    return float(_L.or_f16_to_f32(int(h)))


def f16_array_to_f64(h):
    """Exact values of an array of f16 bit patterns (numpy's float16 is exact too)."""
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float64)


# ---- int4 group quantizer -----------------------------------------------------
def quant_int4_bf16(w_bf16, N, K):
    w = _c(w_bf16, np.uint16)
    pack = np.zeros(N * K // 8, np.uint32)
    sc = np.zeros(N * K // 32, np.uint16)
    _L.or_quant_int4_bf16(_ptr(w), N, K, _ptr(pack), _ptr(sc))
    return pack, sc


# ---- int8 activation quant, fused RMSNorm + quant -----------------------------
def quant_act_q8(x):
    x = _c(x, np.float32)
    K = x.size
    xq = np.zeros(K // 4, np.uint32)
    xs = np.zeros(K // 32, np.float32)
    xsum = np.zeros(K // 16, np.int32)
    _L.or_quant_act_q8(_ptr(x), K, _ptr(xq), _ptr(xs), _ptr(xsum))
    return xq, xs, xsum


def quant_act_q8_t(x, T, K):
    x = _c(x, np.float32)
    xq = np.zeros(T * K // 4, np.uint32)
    xs = np.zeros(T * K // 32, np.float32)
    _L.or_quant_act_q8_t(_ptr(x), T, K, _ptr(xq), _ptr(xs))
    return xq, xs


def rmsnorm_q8(x, w_f16, eps):
    x = _c(x, np.float32)
    w = _c(w_f16, np.uint16)
    H = x.size
    xq = np.zeros(H // 4, np.uint32)
    xs = np.zeros(H // 32, np.float32)
    xsum = np.zeros(H // 16, np.int32)
    _L.or_rmsnorm_q8(_ptr(x), _ptr(w), H, eps, _ptr(xq), _ptr(xs), _ptr(xsum))
    return xq, xs, xsum


def rmsnorm(x, w_f16, T, H, eps):
    x = _c(x, np.float32)
    w = _c(w_f16, np.uint16)
    y = np.zeros(T * H, np.float32)
    _L.or_rmsnorm(_ptr(x), _ptr(w), T, H, eps, _ptr(y))
    return y


# ---- int4 GEMV / GEMM oracles --------------------------------------------------
def group_dots_q4_q8(xq, pack, N, K):
    d = np.zeros(N * (K // 32), np.int32)
    _L.or_group_dots_q4_q8(_ptr(_c(xq, np.uint32)), _ptr(_c(pack, np.uint32)), N, K, _ptr(d))
    return d


def gemv_q4_q8(xq, xs, pack, sc, N, K):
    y = np.zeros(N, np.float64)
    _L.or_gemv_q4_q8(_ptr(_c(xq, np.uint32)), _ptr(_c(xs, np.float32)), _ptr(_c(pack, np.uint32)),
                     _ptr(_c(sc, np.uint16)), N, K, _ptr(y))
    return y


def quant_tern_bf16(w_bf16, N, K):
    """(pack, scales) of the on-GPU ternary format, or None where the reference returns null."""
    w = _c(w_bf16, np.uint16)
    pack = np.zeros(N * K // 16, np.uint32)
    sc = np.zeros(N * K // 32, np.uint16)
    ok = _L.or_quant_tern_bf16(_ptr(w), N, K, _ptr(pack), _ptr(sc))
    return (pack, sc) if ok else None


def gemv_tern2(xq, xs, pack, sc, N, K):
    y = np.zeros(N, np.float64)
    _L.or_gemv_tern2(_ptr(_c(xq, np.uint32)), _ptr(_c(xs, np.float32)), _ptr(_c(pack, np.uint32)),
                     _ptr(_c(sc, np.uint16)), N, K, _ptr(y))
    return y


def gateup_silu_tern2(xq, xs, gp, gs, up, us, I, H):
    y = np.zeros(I, np.float64)
    _L.or_gateup_silu_tern2(_ptr(_c(xq, np.uint32)), _ptr(_c(xs, np.float32)), _ptr(_c(gp, np.uint32)),
                            _ptr(_c(gs, np.uint16)), _ptr(_c(up, np.uint32)), _ptr(_c(us, np.uint16)), I, H, _ptr(y))
    return y


def gemv_q4_f32(x, pack, sc, N, K):
    y = np.zeros(N, np.float64)
    _L.or_gemv_q4_f32(_ptr(_c(x, np.float32)), _ptr(_c(pack, np.uint32)), _ptr(_c(sc, np.uint16)), N, K, _ptr(y))
    return y


def gateup_silu_q4(xq, xs, gp, gs, up, us, I, H):
    y = np.zeros(I, np.float64)
    _L.or_gateup_silu_q4(_ptr(_c(xq, np.uint32)), _ptr(_c(xs, np.float32)), _ptr(_c(gp, np.uint32)),
                         _ptr(_c(gs, np.uint16)), _ptr(_c(up, np.uint32)), _ptr(_c(us, np.uint16)), I, H, _ptr(y))
    return y


def gemm_q4_q8(xq, xs, pack, sc, T, N, K):
    y = np.zeros(T * N, np.float64)
    _L.or_gemm_q4_q8(_ptr(_c(xq, np.uint32)), _ptr(_c(xs, np.float32)), _ptr(_c(pack, np.uint32)),
                     _ptr(_c(sc, np.uint16)), T, N, K, _ptr(y))
    return y


# ---- KV / attention ----------------------------------------------------------------
def kv_quant(x):
    x = _c(x, np.float32)
    n = x.size
    q = np.zeros(n // 4, np.uint32)
    s = np.zeros(n // 32, np.float32)
    _L.or_kv_quant(_ptr(x), n, _ptr(q), _ptr(s))
    return q, s


def kv_dequant(q, s):
    """Dequantize words/scales (snorm: max(code/127,-1)*scale), f64."""
    codes = np.asarray(q, np.uint32).view(np.int8).astype(np.float64)
    v = np.maximum(codes / 127.0, -1.0)
    return v * np.repeat(np.asarray(s, np.float64), 32)


def attn_prep_q8(q, k, v, qw, kw, nHq, nKv, hd, pos, theta, eps):
    qr = np.zeros(nHq * hd, np.float32)
    kq = np.zeros(nKv * hd // 4, np.uint32)
    ks = np.zeros(nKv * hd // 32, np.float32)
    vq = np.zeros(nKv * hd // 4, np.uint32)
    vs = np.zeros(nKv * hd // 32, np.float32)
    _L.or_attn_prep_q8(_ptr(_c(q, np.float32)), _ptr(_c(k, np.float32)), _ptr(_c(v, np.float32)),
                       _ptr(_c(qw, np.uint16)), _ptr(_c(kw, np.uint16)), nHq, nKv, hd, pos, theta, eps,
                       _ptr(qr), _ptr(kq), _ptr(ks), _ptr(vq), _ptr(vs))
    return qr, kq, ks, vq, vs


def rope_norm_row(x, w_f16, hd, pos, theta, eps, apply_norm):
    out = np.zeros(hd, np.float32)
    w = _c(w_f16 if w_f16 is not None else np.zeros(hd, np.uint16), np.uint16)
    _L.or_rope_norm_row(_ptr(_c(x, np.float32)), _ptr(w), hd, pos, theta, eps, int(apply_norm), _ptr(out))
    return out


def attn_decode_q8(qr, kq, ks, vq, vs, S, nHq, nKv, hd):
    out = np.zeros(nHq * hd, np.float64)
    _L.or_attn_decode_q8(_ptr(_c(qr, np.float32)), _ptr(_c(kq, np.uint32)), _ptr(_c(ks, np.float32)),
                         _ptr(_c(vq, np.uint32)), _ptr(_c(vs, np.float32)), S, nHq, nKv, hd, _ptr(out))
    return out


def attn_causal_q8(qr, kq, ks, vq, vs, T, pos0, nHq, nKv, hd):
    out = np.zeros(T * nHq * hd, np.float64)
    _L.or_attn_causal_q8(_ptr(_c(qr, np.float32)), _ptr(_c(kq, np.uint32)), _ptr(_c(ks, np.float32)),
                         _ptr(_c(vq, np.uint32)), _ptr(_c(vs, np.float32)), T, pos0, nHq, nKv, hd, _ptr(out))
    return out


# ---- parallel forms for full-size checks (ctypes releases the GIL during each call) ----
_POOL = None


def _pool():
    global _POOL
    if _POOL is None:
        import concurrent.futures as cf
        _POOL = cf.ThreadPoolExecutor(max(1, min(16, os.cpu_count() or 1)))
    return _POOL


def _row_chunks(N, parts):
    step = max(32, -(-N // parts))
    return [(r, min(N, r + step)) for r in range(0, N, step)]


def gemv_q4_q8_par(xq, xs, pack, sc, N, K, parts=16):
    """gemv_q4_q8 with its rows split over threads (each row's arithmetic unchanged)."""
    xq, xs, pack, sc = _c(xq, np.uint32), _c(xs, np.float32), _c(pack, np.uint32), _c(sc, np.uint16)
    y = np.zeros(N, np.float64)
    def run(r0, r1):
        _L.or_gemv_q4_q8(_ptr(xq), _ptr(xs), pack.ctypes.data + r0 * K // 2, sc.ctypes.data + r0 * K // 16,
                         r1 - r0, K, y.ctypes.data + r0 * 8)
    list(_pool().map(lambda rr: run(*rr), _row_chunks(N, parts)))
    return y


def gemv_q4_f32_par(x, pack, sc, N, K, parts=16):
    x, pack, sc = _c(x, np.float32), _c(pack, np.uint32), _c(sc, np.uint16)
    y = np.zeros(N, np.float64)
    def run(r0, r1):
        _L.or_gemv_q4_f32(_ptr(x), pack.ctypes.data + r0 * K // 2, sc.ctypes.data + r0 * K // 16, r1 - r0, K,
                          y.ctypes.data + r0 * 8)
    list(_pool().map(lambda rr: run(*rr), _row_chunks(N, parts)))
    return y


def gateup_silu_q4_par(xq, xs, gp, gs, up, us, I, H, parts=16):
    xq, xs = _c(xq, np.uint32), _c(xs, np.float32)
    gp, gs, up, us = _c(gp, np.uint32), _c(gs, np.uint16), _c(up, np.uint32), _c(us, np.uint16)
    y = np.zeros(I, np.float64)
    def run(r0, r1):
        _L.or_gateup_silu_q4(_ptr(xq), _ptr(xs), gp.ctypes.data + r0 * H // 2, gs.ctypes.data + r0 * H // 16,
                             up.ctypes.data + r0 * H // 2, us.ctypes.data + r0 * H // 16, r1 - r0, H,
                             y.ctypes.data + r0 * 8)
    list(_pool().map(lambda rr: run(*rr), _row_chunks(I, parts)))
    return y


def tern_gemv_scalar_par(codes, sc, act, xsum, N, K, parts=16):
    """tern_gemv_scalar with its rows split over threads (each row's arithmetic unchanged)."""
    codes, sc, act, xsum = _c(codes, np.uint8), _c(sc, np.float32), _c(act, np.int8), _c(xsum, np.int32)
    out = np.zeros(N, np.float32)
    def run(r0, r1):
        _L.or_tern_gemv_scalar(codes.ctypes.data + r0 * K // 4, sc.ctypes.data + r0 * (K // 64) * 4, _ptr(act),
                               _ptr(xsum), r1 - r0, K, out.ctypes.data + r0 * 4)
    list(_pool().map(lambda rr: run(*rr), _row_chunks(N, parts)))
    return out


def attn_causal_q8_kvheads(qr, kq, ks, vq, vs, T, pos0, nHq, nKv, hd, hk0, hk1, out=None):
    out = np.zeros(T * nHq * hd, np.float64) if out is None else out
    _L.or_attn_causal_q8_kvheads(_ptr(_c(qr, np.float32)), _ptr(_c(kq, np.uint32)), _ptr(_c(ks, np.float32)),
                                 _ptr(_c(vq, np.uint32)), _ptr(_c(vs, np.float32)), T, pos0, nHq, nKv, hd, hk0, hk1,
                                 _ptr(out))
    return out


def attn_causal_q8_par(qr, kq, ks, vq, vs, T, pos0, nHq, nKv, hd):
    """attn_causal_q8 with one thread per KV head (bit-identical results)."""
    qr, kq, ks, vq, vs = _c(qr, np.float32), _c(kq, np.uint32), _c(ks, np.float32), _c(vq, np.uint32), _c(vs, np.float32)
    out = np.zeros(T * nHq * hd, np.float64)
    list(_pool().map(lambda h: attn_causal_q8_kvheads(qr, kq, ks, vq, vs, T, pos0, nHq, nKv, hd, h, h + 1, out),
                     range(nKv)))
    return out


def embed(ids, emb, T, H):
    y = np.zeros(T * H, np.float32)
    _L.or_embed(_ptr(_c(ids, np.int32)), _ptr(_c(emb, np.uint16)), T, H, _ptr(y))
    return y


def argmax(logits):
    lg = _c(logits, np.float32)
    return int(_L.or_argmax(_ptr(lg), lg.size))


SEED_INIT = 0x9E3779B9    # the reference's initial _rngSeed (models/qwen3.js:2733)


def pcg(v):
    return int(_L.or_pcg(int(v) & 0xFFFFFFFF))


def seed_next(s):
    return int(_L.or_seed_next(int(s) & 0xFFFFFFFF))


def gumbel_noise(logits, seed, temp):
    """logits + temp * Gumbel noise of the step's seed (a new array; f32 as the shader)."""
    lg = np.array(logits, np.float32, copy=True)
    _L.or_gumbel_noise(_ptr(lg), lg.size, int(seed) & 0xFFFFFFFF, float(temp))
    return lg


# ---- ternary ------------------------------------------------------------------------
def tern_pack(w, N, K):
    codes = np.zeros(N * K // 4, np.uint8)
    sc = np.zeros(N * K // 64, np.float32)
    _L.or_tern_pack(_ptr(_c(w, np.float32)), N, K, _ptr(codes), _ptr(sc))
    return codes, sc


def tern_quant_act_n2(x):
    x = _c(x, np.float32)
    K = x.size
    act = np.zeros(K, np.int8)
    xsum = np.zeros(K // 64, np.int32)
    s = _L.or_tern_quant_act_n2(_ptr(x), K, _ptr(act), _ptr(xsum))
    return act, xsum, float(s)


def tern_quant_act_wasm(x):
    x = _c(x, np.float32)
    K = x.size
    act = np.zeros(K, np.int8)
    xsum = np.zeros(K // 64, np.int32)
    s = _L.or_tern_quant_act_wasm(_ptr(x), K, _ptr(act), _ptr(xsum))
    return act, xsum, float(s)


def tern_gemv_scalar(codes, sc, act, xsum, N, K):
    out = np.zeros(N, np.float32)
    _L.or_tern_gemv_scalar(_ptr(_c(codes, np.uint8)), _ptr(_c(sc, np.float32)), _ptr(_c(act, np.int8)),
                           _ptr(_c(xsum, np.int32)), N, K, _ptr(out))
    return out


def tern_gemv_dequant(codes, sc, act, N, K):
    out = np.zeros(N, np.float32)
    _L.or_tern_gemv_dequant(_ptr(_c(codes, np.uint8)), _ptr(_c(sc, np.float32)), _ptr(_c(act, np.int8)), N, K, _ptr(out))
    return out


def tern_block_dots(codes, act, N, K):
    d = np.zeros(N * K // 64, np.int32)
    _L.or_tern_block_dots(_ptr(_c(codes, np.uint8)), _ptr(_c(act, np.int8)), N, K, _ptr(d))
    return d


def n2_fixture(N, K, seed):
    codes = np.zeros(N * K // 4, np.uint8)
    sc = np.zeros(N * K // 64, np.float32)
    act = np.zeros(K, np.int8)
    xsum = np.zeros(K // 64, np.int32)
    w = np.zeros(N * K, np.float32)
    x = np.zeros(K, np.float32)
    _L.or_n2_fixture(N, K, seed, _ptr(codes), _ptr(sc), _ptr(act), _ptr(xsum), _ptr(w), _ptr(x))
    return codes, sc, act, xsum, w, x


def has_avx2():
    return bool(_L.or_has_avx2())


def tern_gemv_avx2(codes, sc, act, xsum, N, K, nthreads=1):
    out = np.zeros(N, np.float32)
    args = (_ptr(_c(codes, np.uint8)), _ptr(_c(sc, np.float32)), _ptr(_c(act, np.int8)), _ptr(_c(xsum, np.int32)), N, K, _ptr(out))
    if nthreads <= 1:
        _L.or_tern_gemv_avx2(*args)
    else:
        _L.or_tern_gemv_avx2_mt(*args, nthreads)
    return out


class _TernMat(C.Structure):
    _fields_ = [("codes", C.c_void_p), ("scales", C.c_void_p), ("act", C.c_void_p), ("xsum", C.c_void_p),
                ("out", C.c_void_p), ("N", C.c_int), ("K", C.c_int)]


class TernPool:
    """The AVX2 ternary GEMV over a whole set of matrices on a persistent thread pool
    (or_tern_pool_*): `run()` is one pass, each matrix row-split over the threads with a
    barrier after it. mats: [(codes u8, scales f32, act i8, xsum i32, out f32, N, K)],
    contiguous arrays kept alive by this object."""

    def __init__(self, mats, nthreads):
        self.keep = mats
        self.arr = (_TernMat * len(mats))(*[_TernMat(c.ctypes.data, s_.ctypes.data, a.ctypes.data, x.ctypes.data,
                                                     o.ctypes.data, N, K) for c, s_, a, x, o, N, K in mats])
        self.n = len(mats)
        self.threads = int(_L.or_tern_pool_start(nthreads))

    def run(self):
        _L.or_tern_pool_run(C.cast(self.arr, C.c_void_p), self.n)

    def run_serial(self):
        """The same pass on the calling thread alone."""
        _L.or_tern_set_serial(C.cast(self.arr, C.c_void_p), self.n)

    def close(self):
        _L.or_tern_pool_stop()


def tern_gemv_avx2_into(codes, sc, act, xsum, N, K, out, nthreads=1):
    """Zero-copy call for timing loops: all arrays must already be contiguous."""
    _L.or_tern_gemv_avx2_mt(_ptr(codes), _ptr(sc), _ptr(act), _ptr(xsum), N, K, _ptr(out), nthreads)


# ---- int3 MoE -----------------------------------------------------------------------
def requant43(pack4, sc4, rows, K):
    gpr = K // 32
    p3 = np.zeros(rows * gpr * 3, np.uint32)
    s3 = np.zeros(rows * gpr, np.uint16)
    _L.or_requant43(_ptr(_c(pack4, np.uint32)), _ptr(_c(sc4, np.uint16)), rows, K, _ptr(p3), _ptr(s3))
    return p3, s3


def router(logits, bias, T, nE, topk):
    idx = np.zeros(T * topk, np.int32)
    wt = np.zeros(T * topk, np.float32)
    _L.or_router(_ptr(_c(logits, np.float32)), _ptr(_c(bias, np.float32)), T, nE, topk, _ptr(idx), _ptr(wt))
    return idx, wt


def moe_gemv_q3(x, p3, s3, idx, pairs, N, K, in_stride, xdiv):
    y = np.zeros(pairs * N, np.float64)
    _L.or_moe_gemv_q3(_ptr(_c(x, np.float32)), _ptr(_c(p3, np.uint32)), _ptr(_c(s3, np.uint16)),
                      _ptr(_c(idx, np.int32)), pairs, N, K, in_stride, xdiv, _ptr(y))
    return y


def moe_gemm_q3(xq, xs, p3, s3, ridx, P, N, K, src_div):
    y = np.zeros(P * N, np.float64)
    _L.or_moe_gemm_q3(_ptr(_c(xq, np.uint32)), _ptr(_c(xs, np.float32)), _ptr(_c(p3, np.uint32)),
                      _ptr(_c(s3, np.uint16)), _ptr(_c(ridx, np.int32)), P, N, K, src_div, _ptr(y))
    return y


def moe_combine(x, o, wt, H, K, T):
    x = np.array(x, dtype=np.float32, copy=True)
    _L.or_moe_combine(_ptr(x), _ptr(_c(o, np.float32)), _ptr(_c(wt, np.float32)), H, K, T)
    return x


# ---- the Bonsai forward's f32 glue (ops.rs, model.rs) ----------------------------------------
def n2_rmsnorm(x, w, eps):
    x, w = _c(x, np.float32), _c(w, np.float32)
    out = np.zeros(x.size, np.float32)
    _L.or_n2_rmsnorm(_ptr(x), _ptr(w), x.size, eps, _ptr(out))
    return out


def n2_rmsnorm_heads(t, w, n_heads, head_dim, eps):
    t = np.array(t, np.float32)
    _L.or_n2_rmsnorm_heads(_ptr(t), _ptr(_c(w, np.float32)), n_heads, head_dim, eps)
    return t


def n2_rope_table(head_dim, pos, theta):
    t = np.zeros(head_dim, np.float32)
    _L.or_n2_rope_table(head_dim, pos, theta, _ptr(t))
    return t


def n2_rope_with_table(t, n_heads, head_dim, table):
    t = np.array(t, np.float32)
    _L.or_n2_rope_with_table(_ptr(t), n_heads, head_dim, _ptr(_c(table, np.float32)))
    return t


def n2_swiglu(gate, up):
    g, u = _c(gate, np.float32), _c(up, np.float32)
    out = np.zeros(g.size, np.float32)
    _L.or_n2_swiglu(_ptr(g), _ptr(u), g.size, _ptr(out))
    return out


def n2_attention(q, kc, vc, S, n_heads, n_kv, head_dim):
    out = np.zeros(n_heads * head_dim, np.float32)
    _L.or_n2_attention(_ptr(_c(q, np.float32)), _ptr(_c(kc, np.float32)), _ptr(_c(vc, np.float32)), S, n_heads, n_kv,
                       head_dim, _ptr(out))
    return out


def n2_argmax(x):
    x = _c(x, np.float32)
    return int(_L.or_n2_argmax(_ptr(x), x.size))
