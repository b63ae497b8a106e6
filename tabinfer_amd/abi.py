"""ctypes binding of libtabinfer.so (include/ti.h).

This is plumbing for Python callers (the test-suite and bench.py); the JS host
uses the N-API addon over the same C ABI. Loading fails loudly when the
library has not been built: there is no fallback implementation.
"""
import ctypes as C
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtabinfer.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "ti.h")

TI_OK, TI_ERR_INVALID, TI_ERR_NO_DEVICE, TI_ERR_HIP, TI_ERR_OOM, TI_ERR_STATE = 0, -1, -2, -3, -4, -5


class TIError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("ti error %d: %s" % (code, msg))
        self.code = code


_p, _i, _f, _sz, _u32 = C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_uint32

# name -> argtypes (all return int unless listed in _RES)
SIGS = {
    "ti_version": [],
    "ti_device_count": [C.POINTER(_i)],
    "ti_init": [_i, C.POINTER(_p)],
    "ti_shutdown": [_p],
    "ti_buf_alloc": [_p, _sz, C.POINTER(_p)],
    "ti_buf_free": [_p, _p],
    "ti_buf_write": [_p, _p, _sz, _p, _sz],
    "ti_buf_read": [_p, _p, _sz, _p, _sz],
    "ti_buf_read_async": [_p, _p, _sz, _p, _sz],
    "ti_host_alloc": [_sz, C.POINTER(_p)],
    "ti_host_free": [_p],
    "ti_buf_copy": [_p, _p, _sz, _p, _sz, _sz],
    "ti_buf_fill_u32": [_p, _p, _u32, _sz],
    "ti_sync": [_p],
    "ti_graph_begin": [_p],
    "ti_graph_end": [_p, C.POINTER(_p)],
    "ti_graph_launch": [_p, _p],
    "ti_graph_destroy": [_p],
    "ti_event_record": [_p, _i],
    "ti_event_elapsed_ms": [_p, _i, _i, C.POINTER(_f)],
    "ti_event_wait": [_p, _i],
    "ti_quant_int4_bf16": [_p, _p, _p, _p, _i, _i],
    "ti_quant_tern_bf16": [_p, _p, _p, _p, _i, _i, _p],
    "ti_gemv_tern2": [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i],
    "ti_gateup_silu_tern2": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i],
    "ti_quant_act_q8": [_p, _p, _p, _p, _p, _i],
    "ti_quant_act_q8_t": [_p, _p, _p, _p, _i, _i],
    "ti_rmsnorm_q8": [_p, _p, _p, _p, _p, _p, _i, _f],
    "ti_rmsnorm": [_p, _p, _p, _p, _i, _i, _f],
    "ti_rmsnorm_q8_t": [_p, _p, _p, _p, _p, _i, _i, _f],
    "ti_gemv_q4_q8": [_p, _p, _p, _p, _p, _p, _i, _i, _i],
    "ti_gemv_q4_f32": [_p, _p, _p, _p, _p, _i, _i, _i],
    "ti_gateup_silu_q4": [_p, _p, _p, _p, _p, _p, _p, _p, _i, _i],
    "ti_linear_q4": [_p, _p, _p, _p, _p, _i, _i, _i, _i],
    "ti_group_dots_q4_q8": [_p, _p, _p, _p, _i, _i],
    "ti_rmsnorm_gemv_q4": [_p, _p, _p, _f, _i, _i, _p, _p, _p, _p, _p, _p],
    "ti_rmsnorm_gateup_silu_q4": [_p, _p, _p, _f, _p, _p, _p, _p, _p, _i, _i, _p, _p],
    "ti_rmsnorm_lm_head_argmax": [_p, _p, _p, _f, _p, _p, _p, _i, _i, _p, _i],
    "ti_argmax": [_p, _p, _i, _p, _i],
    "ti_gumbel_noise": [_p, _p, _i, C.c_uint32, _f],
    "ti_embed": [_p, _p, _p, _p, _i, _i, _i, _i],
    "ti_attn_step_q8": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _f, _f, _i, _p, _p],
    "ti_attn_prep_q8": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _f, _f],
    "ti_attn_decode_q8": [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i],
    "ti_attn_decode_q8_noalloc": [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i],
    "ti_rope_qk": [_p, _p, _p, _p, _i, _i, _i, _i, _f, _f],
    "ti_kv_write_q8": [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i],
    "ti_tern_gemv": [_p, _p, _p, _p, _p, _p, _i, _i],
    "ti_tern_gemm": [_p, _p, C.c_long, _p, _p, _p, _p, _i, _i, _i],
    "ti_tern_gemv_multi": [_p, _p, _p, _i, _i, _p, _p, _p, _p],
    "ti_quant_act_tern": [_p, _p, _p, _p, _p, _i, _i],
    "ti_tern_block_dots": [_p, _p, _p, _p, _i, _i],
    "ti_requant43": [_p, _p, _p, _i, _i, _p, _p],
    "ti_router": [_p, _p, _p, _i, _i, _i, _p, _p],
    "ti_moe_gemv_q3": [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i],
    "ti_moe_gemm_q3": [_p, _p, _i, _p, _p, _p, _p, _i, _i, _i, _i, _i],
    "ti_swiglu": [_p, _p, _p, _p, C.c_long],
    "ti_moe_decode_q3": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i],
    "ti_moe_combine": [_p, _p, _p, _p, _i, _i, _i],
    "ti_moe_prefill_q3": [_p] * 17 + [_i] * 5,
    "ti_qwen3_create": [_p, _p, C.POINTER(_p)],
    "ti_qwen3_destroy": [_p, _p],
    "ti_qwen3_tensor": [_p, C.c_char_p, C.POINTER(_p), C.POINTER(_sz), C.POINTER(_p), C.POINTER(_sz)],
    "ti_qwen3_kv": [_p, _i, C.POINTER(_p), C.POINTER(_p), C.POINTER(_p), C.POINTER(_p)],
    "ti_qwen3_kv_layout": [_p, C.POINTER(_i)],
    "ti_qwen3_kv_write": [_p, _p, _i, _p, _p, _i, _i],
    "ti_qwen3_logits": [_p, C.POINTER(_p)],
    "ti_qwen3_forward": [_p, _p, _p, _i, _i],
    "ti_qwen3_decode": [_p, _p],
    "ti_qwen3_set_pos": [_p, _p, _i],
    "ti_qwen3_decode_splits": [_p, _i, _p],
    "ti_qwen3_sampling": [_p, _p, _f],
    "ti_qwen3_seed": [_p, _p, C.c_uint32],
    "ti_qwen3_get_seed": [_p, _p, C.POINTER(C.c_uint32)],
    "ti_qwen3_trace": [_p, _p, _sz],
    "ti_qwen3_write_tokens": [_p, _p, _i, _i, _p],
    "ti_qwen3_read_tokens": [_p, _p, _i, _i, _p],
    "ti_qwen3_read_tokens_async": [_p, _p, _i, _i, _p],
    "ti_attn_causal_q8": [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i],
}


class Qwen3Config(C.Structure):
    _fields_ = [("layers", _i), ("hidden", _i), ("intermediate", _i), ("n_heads", _i), ("n_kv_heads", _i),
                ("head_dim", _i), ("vocab", _i), ("rope_theta", _f), ("rms_eps", _f), ("max_ctx", _i),
                ("max_tokens", _i)]


class CpuBinTensor(C.Structure):
    """ti_cpubin_tensor_info"""
    _fields_ = [("kind", _i), ("N", C.c_longlong), ("K", C.c_longlong), ("ndim", _i), ("shape", C.c_longlong * 4),
                ("data", _p), ("data_bytes", _sz), ("scales", _p), ("scale_bytes", _sz)]


class BonsaiConfig(C.Structure):
    _fields_ = [("layers", _i), ("hidden", _i), ("intermediate", _i), ("n_heads", _i), ("n_kv_heads", _i),
                ("head_dim", _i), ("vocab", _i), ("rope_theta", _f), ("rms_eps", _f), ("max_ctx", _i)]


SIGS.update({
    "ti_bonsai_create": [_p, C.POINTER(BonsaiConfig), C.POINTER(_p)],
    "ti_bonsai_destroy": [_p, _p],
    "ti_bonsai_load": [_p, _p, _p],
    "ti_bonsai_tensor": [_p, C.c_char_p, C.POINTER(_p), C.POINTER(_sz), C.POINTER(_p), C.POINTER(_sz)],
    "ti_bonsai_kv": [_p, _i, C.POINTER(_p), C.POINTER(_p)],
    "ti_bonsai_logits": [_p, C.POINTER(_p)],
    "ti_bonsai_forward": [_p, _p, _p, _i, _i],
    "ti_bonsai_decode": [_p, _p],
    "ti_bonsai_set_pos": [_p, _p, _i],
    "ti_bonsai_write_tokens": [_p, _p, _i, _i, _p],
    "ti_bonsai_read_tokens": [_p, _p, _i, _i, _p],
    "ti_bonsai_trace": [_p, _p, _sz],
    "ti_cpubin_open": [C.c_char_p, C.POINTER(_p)],
    "ti_cpubin_parse": [_p, _sz, C.POINTER(_p)],
    "ti_cpubin_close": [_p],
    "ti_cpubin_summary": [_p, C.POINTER(_i), C.POINTER(_i), C.POINTER(_sz)],
    "ti_cpubin_name": [_p, _i, C.POINTER(C.c_char_p)],
    "ti_cpubin_tensor": [_p, C.c_char_p, C.POINTER(CpuBinTensor)],
    "ti_cpubin_embed_row": [_p, C.c_char_p, C.c_longlong, _p, _i],
})
_RES = {"ti_last_error": C.c_char_p}


def header_functions(path=HEADER):
    """Names of every function include/ti.h declares."""
    txt = open(path).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(ti_[a-z0-9_]+)\s*\(", txt)))


def load(path=LIB_PATH):
    if not os.path.exists(path):
        raise ImportError("libtabinfer.so is not built (%s); run `python -m tabinfer_amd.build`" % path)
    lib = C.CDLL(path)
    lib.ti_last_error.restype = C.c_char_p
    lib.ti_last_error.argtypes = []
    for name, args in SIGS.items():
        fn = getattr(lib, name)
        fn.restype = C.c_int
        fn.argtypes = args
    return lib


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        _LIB = load()
    return _LIB


def check(rc):
    if rc != 0:
        raise TIError(rc, lib().ti_last_error().decode(errors="replace"))
    return rc


def register(name, argtypes):
    """Declare an additional entry point (used by modules that extend SIGS)."""
    SIGS[name] = argtypes
    if _LIB is not None:
        fn = getattr(_LIB, name)
        fn.restype = C.c_int
        fn.argtypes = argtypes


class DevBuf:
    """A device allocation owned by a Ctx (ptr is the device address)."""

    def __init__(self, ctx, ptr, nbytes):
        self.ctx, self.ptr, self.nbytes = ctx, ptr, nbytes

    def __int__(self):
        return self.ptr

    def free(self):
        if self.ptr:
            check(lib().ti_buf_free(self.ctx.h, self.ptr))
            self.ptr = 0

    def at(self, byte_off):
        """Device address byte_off into this buffer (no ownership)."""
        return self.ptr + byte_off


class Ctx:
    def __init__(self, device=0):
        h = C.c_void_p()
        check(lib().ti_init(device, C.byref(h)))
        self.h = h.value
        self._bufs = []

    # ---- memory ---------------------------------------------------------------
    def alloc(self, nbytes):
        p = C.c_void_p()
        check(lib().ti_buf_alloc(self.h, nbytes, C.byref(p)))
        b = DevBuf(self, p.value, nbytes)
        self._bufs.append(b)
        return b

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        b = self.alloc(max(arr.nbytes, 4))
        if arr.nbytes:
            check(lib().ti_buf_write(self.h, b.ptr, 0, arr.ctypes.data, arr.nbytes))
        return b

    def write(self, buf, arr, off=0):
        arr = np.ascontiguousarray(arr)
        check(lib().ti_buf_write(self.h, int(buf), off, arr.ctypes.data, arr.nbytes))

    def download(self, buf, dtype, count, off=0):
        out = np.empty(count, dtype=dtype)
        if out.nbytes:
            check(lib().ti_buf_read(self.h, int(buf), off, out.ctypes.data, out.nbytes))
        return out

    def zeros(self, nbytes):
        b = self.alloc(nbytes)
        check(lib().ti_buf_fill_u32(self.h, b.ptr, 0, (nbytes + 3) // 4))
        return b

    def fill_u32(self, buf, value, count):
        check(lib().ti_buf_fill_u32(self.h, int(buf), value, count))

    def sync(self):
        check(lib().ti_sync(self.h))

    # ---- generic call ---------------------------------------------------------------
    def call(self, name, *args):
        fn = getattr(lib(), name)
        conv = []
        for a in args:
            if isinstance(a, DevBuf):
                conv.append(a.ptr)
            elif isinstance(a, np.generic):
                conv.append(a.item())
            else:
                conv.append(a)
        return check(fn(self.h, *conv))

    # ---- timing ---------------------------------------------------------------------
    def record(self, slot):
        check(lib().ti_event_record(self.h, slot))

    def elapsed_ms(self, a, b):
        ms = C.c_float()
        check(lib().ti_event_elapsed_ms(self.h, a, b, C.byref(ms)))
        return ms.value

    # ---- graphs -----------------------------------------------------------------------
    def graph_begin(self):
        check(lib().ti_graph_begin(self.h))

    def graph_end(self):
        g = C.c_void_p()
        check(lib().ti_graph_end(self.h, C.byref(g)))
        return g.value

    def graph_launch(self, g):
        check(lib().ti_graph_launch(self.h, g))

    def graph_destroy(self, g):
        check(lib().ti_graph_destroy(g))

    def close(self):
        if self.h:
            for b in self._bufs:
                if b.ptr:
                    lib().ti_buf_free(self.h, b.ptr)
                    b.ptr = 0
            check(lib().ti_shutdown(self.h))
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Qwen3:
    """The native Qwen3 decoder (ti_qwen3_*) on a Ctx."""

    def __init__(self, ctx, **cfg):
        self.ctx = ctx
        self.cfg = Qwen3Config(**cfg)
        h = C.c_void_p()
        check(lib().ti_qwen3_create(ctx.h, C.byref(self.cfg), C.byref(h)))
        self.h = h.value

    def tensor(self, name):
        d, s = C.c_void_p(), C.c_void_p()
        nd, ns = C.c_size_t(), C.c_size_t()
        check(lib().ti_qwen3_tensor(self.h, name.encode(), C.byref(d), C.byref(nd), C.byref(s), C.byref(ns)))
        return d.value, nd.value, s.value, ns.value

    def kv(self, layer):
        ptrs = [C.c_void_p() for _ in range(4)]
        check(lib().ti_qwen3_kv(self.h, layer, *[C.byref(p) for p in ptrs]))
        return [p.value for p in ptrs]

    def kv_slots(self):
        """Code slots per cached position (>= n_kv_heads; the scale rows are n_kv_heads wide)."""
        n = C.c_int()
        check(lib().ti_qwen3_kv_layout(self.h, C.byref(n)))
        return n.value

    def kv_write(self, layer, kr, v, T, pos):
        """kvQuantWrite of T rows (device f32 [T][n_kv*head_dim] K (roped) and V) at pos."""
        check(lib().ti_qwen3_kv_write(self.ctx.h, self.h, layer, int(kr), int(v), T, pos))

    def logits_ptr(self):
        p = C.c_void_p()
        check(lib().ti_qwen3_logits(self.h, C.byref(p)))
        return p.value

    def forward(self, ids, pos, T=None):
        """forward(ids, pos); ids None runs the T tokens already in the history."""
        if ids is None:
            check(lib().ti_qwen3_forward(self.ctx.h, self.h, None, T, pos))
            return
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        check(lib().ti_qwen3_forward(self.ctx.h, self.h, ids.ctypes.data, ids.size, pos))

    def decode(self):
        check(lib().ti_qwen3_decode(self.ctx.h, self.h))

    def set_pos(self, pos):
        check(lib().ti_qwen3_set_pos(self.ctx.h, self.h, pos))

    def decode_splits(self, pos):
        """Attention splits per KV head of a decode step captured at pos (ti_qwen3_decode_splits)."""
        n = C.c_int(0)
        check(lib().ti_qwen3_decode_splits(self.h, pos, C.byref(n)))
        return n.value

    def sampling(self, temperature):
        """Temperature of the following steps (ti_qwen3_sampling); 0 is greedy."""
        check(lib().ti_qwen3_sampling(self.ctx.h, self.h, float(temperature)))

    def seed(self, state):
        check(lib().ti_qwen3_seed(self.ctx.h, self.h, int(state) & 0xFFFFFFFF))

    def get_seed(self):
        v = C.c_uint32()
        check(lib().ti_qwen3_get_seed(self.ctx.h, self.h, C.byref(v)))
        return v.value

    def trace(self, buf):
        """Route the parity trace (ti_qwen3_trace) into the DevBuf `buf`; None stops it."""
        check(lib().ti_qwen3_trace(self.h, int(buf) if buf is not None else None, buf.nbytes if buf is not None else 0))

    def write_tokens(self, start, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        check(lib().ti_qwen3_write_tokens(self.ctx.h, self.h, start, ids.size, ids.ctypes.data))

    def read_tokens(self, start, count):
        out = np.zeros(count, np.int32)
        check(lib().ti_qwen3_read_tokens(self.ctx.h, self.h, start, count, out.ctypes.data))
        return out

    def close(self):
        if self.h:
            check(lib().ti_qwen3_destroy(self.ctx.h, self.h))
            self.h = None


class Bonsai:
    """The native Bonsai ternary decoder (ti_bonsai_*) on a Ctx."""

    def __init__(self, ctx, **cfg):
        self.ctx = ctx
        self.cfg = BonsaiConfig(**cfg)
        h = C.c_void_p()
        check(lib().ti_bonsai_create(ctx.h, C.byref(self.cfg), C.byref(h)))
        self.h = h.value

    def tensor(self, name):
        d, s = C.c_void_p(), C.c_void_p()
        nd, ns = C.c_size_t(), C.c_size_t()
        check(lib().ti_bonsai_tensor(self.h, name.encode(), C.byref(d), C.byref(nd), C.byref(s), C.byref(ns)))
        return d.value, nd.value, s.value, ns.value

    def load(self, cpubin):
        check(lib().ti_bonsai_load(self.ctx.h, self.h, cpubin.h))

    def kv(self, layer):
        k, v = C.c_void_p(), C.c_void_p()
        check(lib().ti_bonsai_kv(self.h, layer, C.byref(k), C.byref(v)))
        return k.value, v.value

    def logits_ptr(self):
        p = C.c_void_p()
        check(lib().ti_bonsai_logits(self.h, C.byref(p)))
        return p.value

    def forward(self, ids, pos, T=None):
        if ids is None:
            check(lib().ti_bonsai_forward(self.ctx.h, self.h, None, T, pos))
            return
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        check(lib().ti_bonsai_forward(self.ctx.h, self.h, ids.ctypes.data, ids.size, pos))

    def decode(self):
        check(lib().ti_bonsai_decode(self.ctx.h, self.h))

    def set_pos(self, pos):
        check(lib().ti_bonsai_set_pos(self.ctx.h, self.h, pos))

    def write_tokens(self, start, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        check(lib().ti_bonsai_write_tokens(self.ctx.h, self.h, start, ids.size, ids.ctypes.data))

    def read_tokens(self, start, count):
        out = np.zeros(count, np.int32)
        check(lib().ti_bonsai_read_tokens(self.ctx.h, self.h, start, count, out.ctypes.data))
        return out

    def trace(self, buf):
        check(lib().ti_bonsai_trace(self.h, int(buf) if buf is not None else None, buf.nbytes if buf is not None else 0))

    def close(self):
        if self.h:
            check(lib().ti_bonsai_destroy(self.ctx.h, self.h))
            self.h = None


class CpuBin:
    """A `.cpu.bin` container read by the library (ti_cpubin_*, host only)."""

    TERN, EMBED_F16, F32 = 1, 2, 3

    def __init__(self, path=None, data=None):
        h = C.c_void_p()
        if path is not None:
            check(lib().ti_cpubin_open(path.encode(), C.byref(h)))
        else:
            buf = bytes(data)
            check(lib().ti_cpubin_parse(C.c_char_p(buf), len(buf), C.byref(h)))
        self.h = h.value

    def summary(self):
        g, n, b = C.c_int(), C.c_int(), C.c_size_t()
        check(lib().ti_cpubin_summary(self.h, C.byref(g), C.byref(n), C.byref(b)))
        return g.value, n.value, b.value

    def names(self):
        out = []
        for i in range(self.summary()[1]):
            p = C.c_char_p()
            check(lib().ti_cpubin_name(self.h, i, C.byref(p)))
            out.append(p.value.decode())
        return out

    def tensor(self, name):
        """(kind, info, data bytes, scale bytes) with numpy copies of the blob ranges."""
        t = CpuBinTensor()
        check(lib().ti_cpubin_tensor(self.h, name.encode(), C.byref(t)))
        data = np.ctypeslib.as_array((C.c_uint8 * t.data_bytes).from_address(t.data)).copy() if t.data_bytes else np.zeros(0, np.uint8)
        sc = (np.ctypeslib.as_array((C.c_uint8 * t.scale_bytes).from_address(t.scales)).copy()
              if t.scale_bytes else np.zeros(0, np.uint8))
        return t, data, sc

    def embed_row(self, name, row, dim):
        out = np.zeros(dim, np.float32)
        check(lib().ti_cpubin_embed_row(self.h, name.encode(), row, out.ctypes.data, dim))
        return out

    def close(self):
        if self.h:
            lib().ti_cpubin_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def device_count():
    n = C.c_int()
    check(lib().ti_device_count(C.byref(n)))
    return n.value
