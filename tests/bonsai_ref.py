"""Test helpers for the Bonsai ternary decoder (test infrastructure): synthetic checkpoints,
a `.cpu.bin` writer in the packer's layout, the decoder's parity trace, and the oracle's
forward (native/crates/n2-core/src/model.rs:349-501 restated with the oracle's n2 ops).

Teacher forcing: at every int8 quantization point the oracle is fed the GPU's own f32
input, so the codes must agree bit for bit, the ternary GEMVs (exact block dots, the
reference's f32 order) and every scale/residual step after them too; only the reductions
the GPU runs as trees (norm sums, attention, expf) are held to a tolerance.
"""
import json
import struct

import numpy as np

TOL = 1e-3
SHAPES = {"self_attn.q_proj.weight": ("nq", "H"), "self_attn.k_proj.weight": ("nkv", "H"),
          "self_attn.v_proj.weight": ("nkv", "H"), "self_attn.o_proj.weight": ("H", "nq"),
          "mlp.gate_proj.weight": ("I", "H"), "mlp.up_proj.weight": ("I", "H"), "mlp.down_proj.weight": ("H", "I")}
NORMS = ("input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_norm.weight", "self_attn.k_norm.weight")


def dims(cfg):
    hd = cfg["head_dim"]
    return dict(H=cfg["hidden"], I=cfg["intermediate"], nq=cfg["n_heads"] * hd, nkv=cfg["n_kv_heads"] * hd, hd=hd)


def tern_codes(rng, nbytes):
    """Packed code bytes whose four 2-bit codes are uniform on {0, 1, 2}."""
    lut = np.array([(v % 3) | ((v // 3 % 3) << 2) | ((v // 9 % 3) << 4) | ((v // 27 % 3) << 6) for v in range(81)], np.uint8)
    u = rng.bit_generator.random_raw((nbytes + 3) // 4).view(np.uint16)[:nbytes].astype(np.uint32)
    return lut[(u * 81) >> 16]


def make_weights(cfg, seed, emb_ids=None):
    """Ternary projections and lm_head (codes uniform on {0,1,2}, scales U(0.01, 0.05)
    rounded to f16, stored f32), f32 norms 1 + 0.1 N(0,1), f16 embeddings N(0, 0.5): all
    rows, or only those of emb_ids (the others are never read)."""
    rng = np.random.default_rng(seed)
    d = dims(cfg)
    W = {}
    tern = lambda N, K: (tern_codes(rng, N * K // 4), rng.uniform(0.01, 0.05, N * (K // 64)).astype(np.float16).astype(np.float32))
    for l in range(cfg["layers"]):
        p = "model.layers.%d." % l
        for name, (n, k) in SHAPES.items():
            W[p + name] = tern(d[n], d[k])
        for name in NORMS:
            W[p + name] = (1 + 0.1 * rng.standard_normal(d["hd"] if "_norm" in name and "attn" in name else d["H"])).astype(np.float32)
    W["model.norm.weight"] = (1 + 0.1 * rng.standard_normal(d["H"])).astype(np.float32)
    W["lm_head.weight"] = tern(cfg["vocab"], d["H"])
    if emb_ids is None:
        W["model.embed_tokens.weight"] = (rng.standard_normal(cfg["vocab"] * d["H"]) * 0.5).astype(np.float16).view(np.uint16)
    else:
        W["emb_rows"] = {int(t): (rng.standard_normal(d["H"]) * 0.5).astype(np.float16).view(np.uint16)
                         for t in sorted(set(int(i) for i in emb_ids))}
    return W


def emb_row(W, tok, H):
    if "emb_rows" in W:
        return W["emb_rows"][int(tok)]
    return W["model.embed_tokens.weight"][int(tok) * H:(int(tok) + 1) * H]


def write_cpubin(path, cfg, W, shapes=None):
    """A `.cpu.bin` container (native/docs/FORMAT.md) as native/tools/pack_bin.py lays it
    out: u32 header length, JSON header with blob-relative offsets, every entry 16-aligned.
    shapes: {name: (N, K)} recorded in place of a ternary tensor's own (a mislabelled file)."""
    d = dims(cfg)
    blob, tensors = bytearray(), {}

    def put(b):
        off = len(blob)
        blob.extend(b)
        blob.extend(bytes((-len(blob)) % 16))
        return off

    for name, val in W.items():
        if isinstance(val, tuple):
            codes, sc = val
            K = d["I"] if name.endswith("down_proj.weight") else (d["nq"] if name.endswith("o_proj.weight") else d["H"])
            N = codes.size * 4 // K
            if shapes and name in shapes:
                N, K = shapes[name]
            co = put(codes.tobytes())
            so = put(sc.tobytes())
            tensors[name] = {"kind": "tern", "N": N, "K": K, "codesOff": co, "codesLen": codes.size, "scalesOff": so,
                             "scalesLen": sc.nbytes}
        elif name == "model.embed_tokens.weight":
            tensors[name] = {"kind": "embed_f16", "shape": [cfg["vocab"], d["H"]], "off": put(val.tobytes()), "len": val.nbytes}
        elif name != "emb_rows":
            tensors[name] = {"kind": "f32", "shape": [val.size], "off": put(val.tobytes()), "len": val.nbytes}
    hdr = json.dumps({"G": 64, "tensors": tensors}).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<I", len(hdr)) + hdr + bytes(blob))


def load_into(ctx, model, W, H):
    for name, val in W.items():
        if name == "emb_rows":
            dp, _, _, _ = model.tensor("model.embed_tokens.weight")
            for t, row in val.items():
                ctx.write(dp, row, t * H * 2)
            continue
        dp, nd, sp, ns = model.tensor(name)
        if isinstance(val, tuple):
            assert val[0].nbytes == nd and val[1].nbytes == ns, name
            ctx.write(dp, val[0])
            ctx.write(sp, val[1])
        else:
            assert val.nbytes == nd, name
            ctx.write(dp, val)


FIELDS = [("x_in", "H", np.float32), ("xn", "H", np.float32), ("a_act", "H/4", np.int8), ("a_scale", "1", np.float32),
          ("q", "nq", np.float32), ("k", "nkv", np.float32), ("v", "nkv", np.float32), ("attn", "nq", np.float32),
          ("b_act", "nq/4", np.int8), ("b_scale", "1", np.float32), ("x_mid", "H", np.float32), ("xn2", "H", np.float32),
          ("c_act", "H/4", np.int8), ("c_scale", "1", np.float32), ("g", "I", np.float32), ("u", "I", np.float32),
          ("swi", "I", np.float32), ("d_act", "I/4", np.int8), ("d_scale", "1", np.float32), ("d", "H", np.float32)]


def _words(d, spec):
    if spec == "1":
        return 1
    n, _, div = spec.partition("/")
    return d[n] // (int(div) if div else 1)


def trace_bytes(cfg):
    d = dims(cfg)
    return 4 * (sum(_words(d, s) for _, s, _ in FIELDS) * cfg["layers"] + 2 * d["H"] + d["H"] // 4 + 1)


def parse_trace(raw, cfg):
    d = dims(cfg)
    off, layers = 0, []
    for _ in range(cfg["layers"]):
        rec = {}
        for name, spec, dt in FIELDS:
            n = _words(d, spec)
            rec[name] = raw[off:off + n].view(dt)
            off += n
        layers.append(rec)
    H = d["H"]
    fin = {"x": raw[off:off + H].view(np.float32), "xn": raw[off + H:off + 2 * H].view(np.float32),
           "act": raw[off + 2 * H:off + 2 * H + H // 4].view(np.int8), "scale": raw[off + 2 * H + H // 4:off + 2 * H + H // 4 + 1].view(np.float32)}
    return layers, fin


def rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def inv_of(scale):
    return np.float32(1.0) / np.float32(scale)


class Report:
    def __init__(self):
        self.err, self.exact = {}, {}

    def e(self, k, v):
        self.err[k] = max(self.err.get(k, 0.0), v)

    def x(self, k, ok):
        self.exact[k] = self.exact.get(k, 0) + (0 if ok else 1)

    def __str__(self):
        return "errors: %s | exact mismatches: %s" % (" ".join("%s=%.2e" % kv for kv in sorted(self.err.items())),
                                                      " ".join("%s=%d" % kv for kv in sorted(self.exact.items())))

    def check(self):
        for k, v in self.err.items():
            assert v < TOL, (k, v, str(self))
        assert all(v == 0 for v in self.exact.values()), str(self)


def quant_eq(orc, R, key, x, act, scale):
    a, xs, s = orc.tern_quant_act_n2(x)
    R.x(key, np.array_equal(a, act) and np.float32(s) == np.float32(scale))
    return a, xs


def teacher_forced(orc, cfg, W, trace, fin, kc_rows, vc_rows, kc_new, vc_new, pos, logits):
    """One traced decode step at position `pos`. kc_rows/vc_rows: the GPU's f32 cache rows
    [0, pos] of every layer (teacher forcing: the attention reads what the GPU wrote);
    kc_new/vc_new: the same rows at `pos` (compared with the oracle's). logits: the GPU's."""
    d = dims(cfg)
    H, I, nq, nkv, hd = d["H"], d["I"], d["nq"], d["nkv"], d["hd"]
    nHq, nKv, eps = cfg["n_heads"], cfg["n_kv_heads"], np.float32(cfg["rms_eps"])
    table = orc.n2_rope_table(hd, pos, np.float32(cfg["rope_theta"]))
    R = Report()
    for l in range(cfg["layers"]):
        p = "model.layers.%d." % l
        t = trace[l]
        nxt = trace[l + 1]["x_in"] if l + 1 < cfg["layers"] else fin["x"]
        R.e("rmsnorm", rel(t["xn"], orc.n2_rmsnorm(t["x_in"], W[p + "input_layernorm.weight"], eps)))
        a, xs = quant_eq(orc, R, "quantize_act", t["xn"], t["a_act"], t["a_scale"][0])
        for name, key, n in (("q", "self_attn.q_proj.weight", nq), ("k", "self_attn.k_proj.weight", nkv),
                             ("v", "self_attn.v_proj.weight", nkv)):
            R.x("ternary GEMV", np.array_equal(t[name], orc.tern_gemv_scalar_par(*W[p + key], a, xs, n, H)))
        inv = inv_of(t["a_scale"][0])
        q = orc.n2_rope_with_table(orc.n2_rmsnorm_heads(t["q"] * inv, W[p + "self_attn.q_norm.weight"], nHq, hd, eps), nHq, hd, table)
        k = orc.n2_rope_with_table(orc.n2_rmsnorm_heads(t["k"] * inv, W[p + "self_attn.k_norm.weight"], nKv, hd, eps), nKv, hd, table)
        R.e("k row", rel(kc_new[l], k))
        R.x("v row", np.array_equal(vc_new[l], t["v"] * inv))
        att = orc.n2_attention(q, kc_rows[l], vc_rows[l], pos + 1, nHq, nKv, hd)
        R.e("attention", rel(t["attn"], att))
        a, xs = quant_eq(orc, R, "quantize_act", t["attn"], t["b_act"], t["b_scale"][0])
        o = orc.tern_gemv_scalar_par(*W[p + "self_attn.o_proj.weight"], a, xs, H, nq)
        R.x("residual", np.array_equal(t["x_mid"], t["x_in"] + o * inv_of(t["b_scale"][0])))
        R.e("rmsnorm", rel(t["xn2"], orc.n2_rmsnorm(t["x_mid"], W[p + "post_attention_layernorm.weight"], eps)))
        a, xs = quant_eq(orc, R, "quantize_act", t["xn2"], t["c_act"], t["c_scale"][0])
        R.x("ternary GEMV", np.array_equal(t["g"], orc.tern_gemv_scalar_par(*W[p + "mlp.gate_proj.weight"], a, xs, I, H)))
        R.x("ternary GEMV", np.array_equal(t["u"], orc.tern_gemv_scalar_par(*W[p + "mlp.up_proj.weight"], a, xs, I, H)))
        ic = inv_of(t["c_scale"][0])
        R.e("swiglu", rel(t["swi"], orc.n2_swiglu(t["g"] * ic, t["u"] * ic)))
        a, xs = quant_eq(orc, R, "quantize_act", t["swi"], t["d_act"], t["d_scale"][0])
        R.x("ternary GEMV", np.array_equal(t["d"], orc.tern_gemv_scalar_par(*W[p + "mlp.down_proj.weight"], a, xs, H, I)))
        R.x("residual", np.array_equal(nxt, t["x_mid"] + t["d"] * inv_of(t["d_scale"][0])))
    R.e("rmsnorm", rel(fin["xn"], orc.n2_rmsnorm(fin["x"], W["model.norm.weight"], eps)))
    a, xs = quant_eq(orc, R, "quantize_act", fin["xn"], fin["act"], fin["scale"][0])
    lm = orc.tern_gemv_scalar_par(*W["lm_head.weight"], a, xs, cfg["vocab"], H)
    R.x("logits", np.array_equal(logits, lm * inv_of(fin["scale"][0])))
    return R


def oracle_step(orc, cfg, W, kc, vc, tok, pos):
    """model.rs forward of one token at `pos` on the oracle alone; kc/vc: per-layer f32
    caches [capacity][nkv] that receive row `pos`. Returns the logits."""
    d = dims(cfg)
    H, I, nq, nkv, hd = d["H"], d["I"], d["nq"], d["nkv"], d["hd"]
    nHq, nKv, eps = cfg["n_heads"], cfg["n_kv_heads"], np.float32(cfg["rms_eps"])
    table = orc.n2_rope_table(hd, pos, np.float32(cfg["rope_theta"]))
    x = orc.f16_array_to_f64(emb_row(W, tok, H)).astype(np.float32)

    def linear(key, v, N, K):
        a, xs, s = orc.tern_quant_act_n2(v)
        return orc.tern_gemv_scalar_par(*W[key], a, xs, N, K) * inv_of(s)

    for l in range(cfg["layers"]):
        p = "model.layers.%d." % l
        xn = orc.n2_rmsnorm(x, W[p + "input_layernorm.weight"], eps)
        q = linear(p + "self_attn.q_proj.weight", xn, nq, H)
        k = linear(p + "self_attn.k_proj.weight", xn, nkv, H)
        v = linear(p + "self_attn.v_proj.weight", xn, nkv, H)
        q = orc.n2_rope_with_table(orc.n2_rmsnorm_heads(q, W[p + "self_attn.q_norm.weight"], nHq, hd, eps), nHq, hd, table)
        k = orc.n2_rope_with_table(orc.n2_rmsnorm_heads(k, W[p + "self_attn.k_norm.weight"], nKv, hd, eps), nKv, hd, table)
        kc[l][pos], vc[l][pos] = k, v
        att = orc.n2_attention(q, kc[l][:pos + 1].ravel(), vc[l][:pos + 1].ravel(), pos + 1, nHq, nKv, hd)
        x = x + linear(p + "self_attn.o_proj.weight", att, H, nq)
        xn = orc.n2_rmsnorm(x, W[p + "post_attention_layernorm.weight"], eps)
        g = linear(p + "mlp.gate_proj.weight", xn, I, H)
        u = linear(p + "mlp.up_proj.weight", xn, I, H)
        x = x + linear(p + "mlp.down_proj.weight", orc.n2_swiglu(g, u), H, I)
    xn = orc.n2_rmsnorm(x, W["model.norm.weight"], eps)
    return linear("lm_head.weight", xn, cfg["vocab"], H)
