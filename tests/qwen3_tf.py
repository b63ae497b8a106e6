"""Teacher-forced, per-layer parity of the native Qwen3 decoder against the oracle
(test infrastructure).

The decoder's parity trace (ti_qwen3_trace) records, for every layer, the values the
reference's forward (models/qwen3.js:3959-4049) passes between launchers: the residual,
the rmsnormQ codes, q/k/v, the attention output and its quantQ8 codes, the residual after
o_proj, swi and its codes. At every re-quantization point the oracle is fed the GPU's own
int8 codes, so each float output of a layer is compared with the oracle's f64 value of
the same quantized operands and held to the reference's 1e-3 (normwise, models/qwen3.js:
3104), however many layers precede it. Where the GPU's codes differ from the codes the
oracle would have produced itself (a value on a rounding boundary: the GPU's f32 sums vs
the oracle's f64), the flips are counted and bounded instead.

Weights are synthetic int4: nibble = a + b + 1 with a, b uniform on 0..7 (q in [-7, 7],
symmetric) and f16 scales U(0.004, 0.008), the range the int4 quantizer gives bf16
N(0, 0.02) rows (its own bit-exactness is tested separately); norms f16(1 + 0.1 N(0,1)).
The prefix KV cache is seeded with int8 codes uniform on [-127, 127] and scales U(1, 3)
(the snorm range of N(0,1) rows)."""
import numpy as np

TOL = 1e-3
SHAPES = {"self_attn.q_proj.weight": ("nq", "H"), "self_attn.k_proj.weight": ("nkv", "H"),
          "self_attn.v_proj.weight": ("nkv", "H"), "self_attn.o_proj.weight": ("H", "nq"),
          "mlp.gate_proj.weight": ("I", "H"), "mlp.up_proj.weight": ("I", "H"), "mlp.down_proj.weight": ("H", "I")}


def dims(cfg):
    hd = cfg["head_dim"]
    return dict(H=cfg["hidden"], I=cfg["intermediate"], nq=cfg["n_heads"] * hd, nkv=cfg["n_kv_heads"] * hd, hd=hd)


def rand_words(rng, n):
    """n uniform random uint32 words (the generator's raw 64-bit output, split in two)."""
    return rng.bit_generator.random_raw((n + 1) // 2).view(np.uint32)[:n]


def rand_int4(rng, N, K):
    n = N * K // 8
    a = rand_words(rng, n) & np.uint32(0x77777777)
    b = rand_words(rng, n) & np.uint32(0x77777777)
    pack = a + b + np.uint32(0x11111111)               # per nibble a + b + 1 <= 15: no carries
    sc = rng.uniform(0.004, 0.008, N * K // 32).astype(np.float16).view(np.uint16)
    return pack, sc


def make_weights(cfg, seed, emb_ids):
    """Synthetic int4 checkpoint; embedding rows only for the token ids in emb_ids."""
    rng = np.random.default_rng(seed)
    d = dims(cfg)
    W = {}
    norm = lambda n: (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float16).view(np.uint16)
    for l in range(cfg["layers"]):
        p = "model.layers.%d." % l
        for name, (n, k) in SHAPES.items():
            W[p + name] = rand_int4(rng, d[n], d[k])
        for name, n in (("input_layernorm.weight", d["H"]), ("post_attention_layernorm.weight", d["H"]),
                        ("self_attn.q_norm.weight", d["hd"]), ("self_attn.k_norm.weight", d["hd"])):
            W[p + name] = norm(n)
    W["model.norm.weight"] = norm(d["H"])
    W["lm_head.weight"] = rand_int4(rng, cfg["vocab"], d["H"])
    W["emb_rows"] = {int(t): (rng.standard_normal(d["H"]) * 0.5).astype(np.float16).view(np.uint16)
                     for t in sorted(set(int(i) for i in emb_ids))}
    return W


def load_into(ctx, model, W, H):
    for name, val in W.items():
        if name == "emb_rows":
            d, _, _, _ = model.tensor("model.embed_tokens.weight")
            for t, row in val.items():
                ctx.write(d, row, t * H * 2)
            continue
        dp, nd, sp, ns = model.tensor(name)
        if isinstance(val, tuple):
            assert val[0].nbytes == nd and val[1].nbytes == ns, name
            ctx.write(dp, val[0])
            ctx.write(sp, val[1])
        else:
            assert val.nbytes == nd, name
            ctx.write(dp, val)


def write_kv_codes(ctx, model, dst, codes, P, cfg):
    """Dense int8 code rows [P][nkv] (as uint32 words) into the decoder's code buffer, whose
    rows carry model.kv_slots() head slots (the spare slots stay zero)."""
    nkv, hd = dims(cfg)["nkv"], cfg["head_dim"]
    slots = model.kv_slots()
    rows = np.zeros((P, slots * hd // 4), np.uint32)
    rows[:, :nkv // 4] = np.asarray(codes, np.uint32).reshape(P, nkv // 4)
    ctx.write(dst, rows)


def read_kv_codes(ctx, model, src, P, T, cfg):
    """Code rows [P, P+T) of the decoder's code buffer as dense uint32 words [T][nkv/4]."""
    nkv, hd = dims(cfg)["nkv"], cfg["head_dim"]
    row_w = model.kv_slots() * hd // 4
    return ctx.download(src, np.uint32, T * row_w, off=P * row_w * 4).reshape(T, row_w)[:, :nkv // 4].copy()


def seed_prefix(ctx, model, cfg, P, cap, seed):
    """Seeded prefix KV of P positions in every layer, written to the model; returns the
    host copies with room for cap positions: [(kq, ks, vq, vs)] per layer."""
    rng = np.random.default_rng(seed)
    nkv = dims(cfg)["nkv"]
    host = []
    for l in range(cfg["layers"]):
        arrs = []
        for _ in range(2):
            q = np.zeros(cap * nkv, np.int8)
            q[:P * nkv] = rand_words(rng, P * nkv // 4).view(np.int8)
            np.maximum(q, -127, out=q)                 # snorm codes span [-127, 127]
            s = np.zeros(cap * nkv // 32, np.float32)
            s[:P * nkv // 32] = rng.uniform(1.0, 3.0, P * nkv // 32).astype(np.float32)
            arrs += [q.view(np.uint32), s]
        dk = model.kv(l)
        for i, (dst, src, n) in enumerate(zip(dk, arrs, (P * nkv // 4, P * nkv // 32) * 2)):
            if i % 2 == 0:
                write_kv_codes(ctx, model, dst, src[:n], P, cfg)
            else:
                ctx.write(dst, src[:n])
        host.append(arrs)
    return host


FIELDS = [("x_in", "H", np.float32), ("xn_q", "H/4", np.uint32), ("xn_s", "H/32", np.float32),
          ("q", "nq", np.float32), ("k", "nkv", np.float32), ("v", "nkv", np.float32), ("attn", "nq", np.float32),
          ("a_q", "nq/4", np.uint32), ("a_s", "nq/32", np.float32), ("x_mid", "H", np.float32),
          ("swi", "I", np.float32), ("s_q", "I/4", np.uint32), ("s_s", "I/32", np.float32)]


def _words(d, spec):
    n, _, div = spec.partition("/")
    return d[n] // (int(div) if div else 1)


def trace_bytes(cfg):
    d, Tm = dims(cfg), cfg["max_tokens"]
    per_layer = sum(_words(d, s) for _, s, _ in FIELDS) * Tm
    return 4 * (per_layer * cfg["layers"] + d["H"] * Tm)


def parse_trace(raw, cfg):
    """raw u32 words -> [per layer {field: array [max_tokens, words]}], x_final [max_tokens, H]."""
    d, Tm = dims(cfg), cfg["max_tokens"]
    off, layers = 0, []
    for _ in range(cfg["layers"]):
        rec = {}
        for name, spec, dt in FIELDS:
            n = _words(d, spec) * Tm
            rec[name] = raw[off:off + n].view(dt).reshape(Tm, -1)
            off += n
        layers.append(rec)
    return layers, raw[off:off + d["H"] * Tm].view(np.float32).reshape(Tm, -1)


def rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def code_diff(a, b):
    """|difference| of two packed int8 code arrays, elementwise."""
    return np.abs(np.asarray(a, np.uint32).view(np.int8).astype(int) - np.asarray(b, np.uint32).view(np.int8).astype(int))


class Report:
    def __init__(self):
        self.err = {}        # float output -> max rel error over layers and tokens
        self.flips = {}      # code point -> [flipped codes, total codes, max |delta|]
        self.exact = {}      # integer output expected bit-exact -> mismatches

    def e(self, key, v):
        self.err[key] = max(self.err.get(key, 0.0), v)

    def f(self, key, d):
        s = self.flips.setdefault(key, [0, 0, 0])
        s[0] += int(np.count_nonzero(d))
        s[1] += int(d.size)
        s[2] = max(s[2], int(d.max()) if d.size else 0)

    def x(self, key, ok):
        self.exact[key] = self.exact.get(key, 0) + (0 if ok else 1)

    def __str__(self):
        e = " ".join("%s=%.2e" % kv for kv in sorted(self.err.items()))
        f = " ".join("%s=%d/%d(max %d)" % (k, *v) for k, v in sorted(self.flips.items()))
        x = " ".join("%s=%d" % kv for kv in sorted(self.exact.items()))
        return "errors: %s | flips: %s | exact mismatches: %s" % (e, f, x)


def teacher_forced(orc, cfg, W, kv_host, trace, x_final, gpu_rows, P, T):
    """Per-layer comparison of the traced GPU forward of T tokens at positions P..P+T-1.
    kv_host: host prefix KV per layer (capacity >= P+T); gpu_rows[l] = the GPU's new KV rows
    (kq, ks, vq, vs) for positions P..P+T-1. Returns a Report."""
    d = dims(cfg)
    H, I, nq, nkv, hd = d["H"], d["I"], d["nq"], d["nkv"], d["hd"]
    nHq, nKv = cfg["n_heads"], cfg["n_kv_heads"]
    eps, theta = np.float32(cfg["rms_eps"]), np.float32(cfg["rope_theta"])
    R = Report()
    for l in range(cfg["layers"]):
        p = "model.layers.%d." % l
        tr = trace[l]
        nxt = trace[l + 1]["x_in"] if l + 1 < cfg["layers"] else x_final
        kq, ks, vq, vs = [a.reshape(-1) for a in kv_host[l]]      # views: row writes land in kv_host
        gk, gks, gv, gvs = gpu_rows[l]
        qr_all = np.zeros((T, nq), np.float32)
        has_xn = T == 1 or T > 4
        has_f32 = T == 1
        for t in range(T):
            x_in = tr["x_in"][t]
            oq, os_, _ = orc.rmsnorm_q8(x_in, W[p + "input_layernorm.weight"], eps)
            if has_xn:
                R.x("rmsnormQ codes", np.array_equal(tr["xn_q"][t], oq) and np.array_equal(tr["xn_s"][t], os_))
                oq, os_ = tr["xn_q"][t], tr["xn_s"][t]
            for name, key, n in (("q", "self_attn.q_proj.weight", nq), ("k", "self_attn.k_proj.weight", nkv),
                                 ("v", "self_attn.v_proj.weight", nkv)):
                R.e(name, rel(tr[name][t], orc.gemv_q4_q8_par(oq, os_, *W[p + key], n, H)))
            qr, krow, ksr, vrow, vsr = orc.attn_prep_q8(tr["q"][t], tr["k"][t], tr["v"][t], W[p + "self_attn.q_norm.weight"],
                                                        W[p + "self_attn.k_norm.weight"], nHq, nKv, hd, P + t, theta, eps)
            qr_all[t] = qr
            R.f("kv codes", np.concatenate([code_diff(gk[t], krow), code_diff(gv[t], vrow)]))
            R.e("kv scales", max(rel(gks[t], ksr), rel(gvs[t], vsr)))
            # the GPU's own rows enter the cache the attention reads (teacher forcing)
            kq.reshape(-1, nkv // 4)[P + t], ks.reshape(-1, nkv // 32)[P + t] = gk[t], gks[t]
            vq.reshape(-1, nkv // 4)[P + t], vs.reshape(-1, nkv // 32)[P + t] = gv[t], gvs[t]
        S = P + T
        att = orc.attn_causal_q8_par(qr_all, kq[:S * nkv // 4], ks[:S * nkv // 32], vq[:S * nkv // 4], vs[:S * nkv // 32],
                                     T, P, nHq, nKv, hd).reshape(T, nq)
        for t in range(T):
            if has_f32:
                R.e("attn", rel(tr["attn"][t], att[t]))
                aq, as_, _ = orc.quant_act_q8(tr["attn"][t])
                R.x("attn quantQ8", np.array_equal(aq, tr["a_q"][t]) and np.array_equal(as_, tr["a_s"][t]))
            aq, _, _ = orc.quant_act_q8(att[t].astype(np.float32))
            R.f("attn codes", code_diff(tr["a_q"][t], aq))
            x_in, x_mid = tr["x_in"][t].astype(np.float64), tr["x_mid"][t].astype(np.float64)
            R.e("o_proj", rel(x_mid - x_in, orc.gemv_q4_q8_par(tr["a_q"][t], tr["a_s"][t], *W[p + "self_attn.o_proj.weight"],
                                                                H, nq)))
            pq, ps, _ = orc.rmsnorm_q8(tr["x_mid"][t], W[p + "post_attention_layernorm.weight"], eps)
            swi = orc.gateup_silu_q4_par(pq, ps, *W[p + "mlp.gate_proj.weight"], *W[p + "mlp.up_proj.weight"], I, H)
            if has_f32:
                R.e("swi", rel(tr["swi"][t], swi))
                sq, ss, _ = orc.quant_act_q8(tr["swi"][t])
                R.x("swi quantQ8", np.array_equal(sq, tr["s_q"][t]) and np.array_equal(ss, tr["s_s"][t]))
            sq, _, _ = orc.quant_act_q8(swi.astype(np.float32))
            R.f("swi codes", code_diff(tr["s_q"][t], sq))
            R.e("down", rel(nxt[t].astype(np.float64) - x_mid,
                            orc.gemv_q4_q8_par(tr["s_q"][t], tr["s_s"][t], *W[p + "mlp.down_proj.weight"], H, I)))
    return R


def check(R):
    """The bars of a teacher-forced report: float outputs within TOL (KV scales, a max over
    32 values of identical f32 inputs, within 1e-5), quantizers of identical inputs exact,
    code flips at most one step and rare (at most 1 in 500, or 4)."""
    for key, err in R.err.items():
        assert err < (1e-5 if key == "kv scales" else TOL), (key, err, str(R))
    assert all(v == 0 for v in R.exact.values()), str(R)
    for key, (n, total, mx) in R.flips.items():
        assert mx <= 1 and n <= max(4, total // 500), (key, n, total, mx)


def new_kv_rows(ctx, model, cfg, P, T):
    """The decoder's KV rows for positions P..P+T-1 of every layer: [(kq, ks, vq, vs)]."""
    nkv = dims(cfg)["nkv"]
    rows = []
    for l in range(cfg["layers"]):
        kq, ks, vq, vs = model.kv(l)
        rows.append((read_kv_codes(ctx, model, kq, P, T, cfg),
                     ctx.download(ks, np.float32, T * nkv // 32, off=P * nkv // 8).reshape(T, -1),
                     read_kv_codes(ctx, model, vq, P, T, cfg),
                     ctx.download(vs, np.float32, T * nkv // 32, off=P * nkv // 8).reshape(T, -1)))
    return rows


def traced(ctx, model, cfg, run):
    """Run `run()` with the model's parity trace on; returns (layers, x_final)."""
    tb = trace_bytes(cfg)
    buf = ctx.alloc(tb)
    try:
        ctx.call("ti_buf_fill_u32", buf, 0x7FC00000, tb // 4)
        model.trace(buf)
        run()
        ctx.sync()
        model.trace(None)
        return parse_trace(ctx.download(buf, np.uint32, tb // 4), cfg)
    finally:
        buf.free()


def final_logits(orc, cfg, W, x_last):
    H = cfg["hidden"]
    normed = orc.rmsnorm(x_last, W["model.norm.weight"], 1, H, np.float32(cfg["rms_eps"]))
    return orc.gemv_q4_f32_par(normed, *W["lm_head.weight"], cfg["vocab"], H)


def oracle_decode(orc, cfg, W, kv_host, tokens, P):
    """The oracle alone (no teacher forcing), token after token from position P, in the
    reference's T = 1 order (models/qwen3.js:3959-4055); its KV rows are written into
    kv_host. Returns the last logits."""
    d = dims(cfg)
    H, I, nq, nkv, hd = d["H"], d["I"], d["nq"], d["nkv"], d["hd"]
    nHq, nKv = cfg["n_heads"], cfg["n_kv_heads"]
    eps, theta = np.float32(cfg["rms_eps"]), np.float32(cfg["rope_theta"])
    for i, tok in enumerate(tokens):
        pos = P + i
        x = orc.f16_array_to_f64(W["emb_rows"][int(tok)]).astype(np.float32)
        for l in range(cfg["layers"]):
            p = "model.layers.%d." % l
            kq, ks, vq, vs = [a.reshape(-1) for a in kv_host[l]]
            xq, xs, _ = orc.rmsnorm_q8(x, W[p + "input_layernorm.weight"], eps)
            q = orc.gemv_q4_q8_par(xq, xs, *W[p + "self_attn.q_proj.weight"], nq, H).astype(np.float32)
            k = orc.gemv_q4_q8_par(xq, xs, *W[p + "self_attn.k_proj.weight"], nkv, H).astype(np.float32)
            v = orc.gemv_q4_q8_par(xq, xs, *W[p + "self_attn.v_proj.weight"], nkv, H).astype(np.float32)
            qr, krow, ksr, vrow, vsr = orc.attn_prep_q8(q, k, v, W[p + "self_attn.q_norm.weight"],
                                                        W[p + "self_attn.k_norm.weight"], nHq, nKv, hd, pos, theta, eps)
            kq.reshape(-1, nkv // 4)[pos], ks.reshape(-1, nkv // 32)[pos] = krow, ksr
            vq.reshape(-1, nkv // 4)[pos], vs.reshape(-1, nkv // 32)[pos] = vrow, vsr
            S = pos + 1
            att = orc.attn_causal_q8_par(qr, kq[:S * nkv // 4], ks[:S * nkv // 32], vq[:S * nkv // 4], vs[:S * nkv // 32],
                                         1, pos, nHq, nKv, hd)
            aq, as_, _ = orc.quant_act_q8(att.astype(np.float32))
            x = (x + orc.gemv_q4_q8_par(aq, as_, *W[p + "self_attn.o_proj.weight"], H, nq).astype(np.float32)).astype(np.float32)
            pq, ps, _ = orc.rmsnorm_q8(x, W[p + "post_attention_layernorm.weight"], eps)
            swi = orc.gateup_silu_q4_par(pq, ps, *W[p + "mlp.gate_proj.weight"], *W[p + "mlp.up_proj.weight"], I, H)
            sq, ss, _ = orc.quant_act_q8(swi.astype(np.float32))
            x = (x + orc.gemv_q4_q8_par(sq, ss, *W[p + "mlp.down_proj.weight"], H, I).astype(np.float32)).astype(np.float32)
    return final_logits(orc, cfg, W, x)
