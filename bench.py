#!/usr/bin/env python3
"""Benchmark of the quantized decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only gemv|moe|decode|all]

Headline workload (`value`): the int4 GEMV set of one Qwen3-0.6B batch-1 decode
step (hidden 1024, intermediate 3072, 16/8 heads of dim 128, 28 layers, vocab
151936), launched the way the decode step launches it (models/qwen3.js:
3981-4049, fused here): per layer [rmsnormQ + q/k/v GEMVs] [o_proj GEMV on the
int8 attention output + residual] [rmsnormQ + gate/up + SiLU + quantQ8 of swi]
[down_proj GEMV + residual], then [final rmsnorm + lm_head 151936x1024 + argmax]. Weights are seeded bf16
N(0, 0.02) quantized on the GPU by the int4 quantizer; activations are seeded
N(0,1) rounded to f16. Two independent weight sets (2 x 337 MB) alternate
between steps, so every step streams its weights from HBM, not from the 256 MB
Infinity Cache. Each step is one captured HIP graph; `value` = algorithmic
bytes of the step / wall time of the timed steps (launch gaps included).

Beside it, each bounded to a few seconds (not `value`):
  kernels       per kernel family, its average launch duration (the family's launches of
                one step back to back in one graph, after a cache flush); the family
                with the most bytes per step sets `roofline`; in_chain_us: one more launch of the
                family in a chain (graph over both weight sets minus graph over one)
  gemv_set_1p7b the same GEMV set at the Qwen3-1.7B shapes (967.75 MB of int4 weights)
  gemv_sustained_1p7b  the projection GEMV kernel at the 1.7B reduction sizes over 198 MB
                of stacked rows per launch: its streaming rate with the launch amortised
  launch_floor  chains of 113 stream-ordered launches that do (almost) nothing
  decode_1p7b   full Qwen3-1.7B int4/int8-KV decode step (the native decoder, one
                graph per token, device-side token chaining) at 8k and 32k prefix
                contexts: tokens/s and whole-step GB/s; and one T = 8 forward (8
                consecutive tokens of one sequence, the batch configuration)
  attention     fused split-KV attention per layer at 4k and 32k (GB/s, cold)
  ternary_bonsai_step  the Bonsai-1.7B ternary GEMV set of one decode step on the GPU
                (28 layers + lm_head, 537.6 MB)
  moe           LFM2.5-8B-A1B int3 MoE block (router, 32 experts top-4, hidden 2048,
                expert intermediate 1792) at batch 1 and 16: us per block, GB/s of
                the distinct experts' weights
  cpu_baseline  the reference's native CPU path, n2 avx2::gemv_tern (restated in C), over
                the same 537.6 MB Bonsai-1.7B ternary set on the host cores, 1 thread and
                N threads, with the reference's timing discipline (control, alternation,
                min of 31)
"""
import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# the decode step's q/k/v GEMV runs inside its attention launch unless this is set (the
# library reads it when a context is created)
QKV_SEPARATE = os.environ.get("TI_DECODE_QKV_SEPARATE", "0") not in ("", "0")
METRIC = "int4 GEMV HBM GB/s (% of peak) + Qwen3-1.7B bs1 decode tok/s at 32k ctx"

QWEN3_06B = dict(layers=28, hidden=1024, inter=3072, n_heads=16, n_kv=8, head_dim=128, vocab=151936)
QWEN3_17B = dict(layers=28, hidden=2048, inter=6144, n_heads=16, n_kv=8, head_dim=128, vocab=151936)


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


# ---- algorithmic bytes (each operand counted once per launch) ------------------------
def int4_bytes(N, K):
    return N * K // 2 + (N * K // 32) * 2


def qkv_bytes(Ns, K):          # f32 x + f16 norm weight in, weights, f32 outputs
    return K * 4 + K * 2 + sum(int4_bytes(N, K) + N * 4 for N in Ns)


def q8_linear_bytes(N, K):     # int8 activation (codes + scales) in, weights, residual read + write
    return K + (K // 32) * 4 + int4_bytes(N, K) + 2 * N * 4


def gateup_bytes(I, H):        # f32 x + norm weight in, gate/up weights, swi out as int8 codes + scales
    return H * 4 + H * 2 + 2 * int4_bytes(I, H) + I + (I // 32) * 4


def lmhead_bytes(N, K):        # f32 x + norm weight in, weights, logits out
    return K * 4 + K * 2 + int4_bytes(N, K) + N * 4


def kv_bytes(S, nKv, hd):      # int8 K and V + their f32 scales, positions [0, S)
    return S * 2 * (nKv * hd + (nKv * hd // 32) * 4)


class Pool:
    """A device pool of seeded bf16 N(0, 0.02) values from which weights are quantized."""

    def __init__(self, ctx, n, seed):
        rng = np.random.default_rng(seed)
        w = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.02))
        self.buf = ctx.upload((w.view(np.uint32) >> 16).astype(np.uint16))
        self.n = n
        self.ctx = ctx

    def quantize_into(self, pack, sc, N, K, rng):
        rows_per = max(1, min(N, self.n // K))
        r = 0
        while r < N:
            nr = min(rows_per, N - r)
            off = int(rng.integers(0, (self.n - nr * K) // 32 + 1)) * 32
            self.ctx.call("ti_quant_int4_bf16", self.buf.at(off * 2), int(pack) + r * K // 2,
                          int(sc) + r * K // 32 * 2, nr, K)
            r += nr

    def quantized(self, N, K, rng):
        pack = self.ctx.alloc(N * K // 2)
        sc = self.ctx.alloc(N * K // 32 * 2)
        self.quantize_into(pack, sc, N, K, rng)
        return pack, sc


# ---- the headline GEMV set ------------------------------------------------------------
class GemvSet:
    """Device-resident int4 weights of one decode step's GEMVs."""

    def __init__(self, ctx, cfg, seed, pool):
        H, I = cfg["hidden"], cfg["inter"]
        nq = cfg["n_heads"] * cfg["head_dim"]
        nkv = cfg["n_kv"] * cfg["head_dim"]
        rng = np.random.default_rng(seed)
        self.shapes = {"q": (nq, H), "k": (nkv, H), "v": (nkv, H), "o": (H, nq),
                       "gate": (I, H), "up": (I, H), "down": (H, I)}
        self.layers = [{n: pool.quantized(N, K, rng) for n, (N, K) in self.shapes.items()} for _ in range(cfg["layers"])]
        self.lm = pool.quantized(cfg["vocab"], H, rng)


def c_ptrs(vals):
    import ctypes as C
    arr = (C.c_void_p * len(vals))()
    for i, v in enumerate(vals):
        arr[i] = int(v)
    return arr


def c_ints(vals):
    import ctypes as C
    arr = (C.c_int * len(vals))()
    for i, v in enumerate(vals):
        arr[i] = v
    return arr


class Step:
    """The launch sequence of one decode step's GEMV set, and its byte count."""

    FAMILIES = ("qkv", "o_proj", "gateup", "down", "lm_head")

    def __init__(self, ctx, cfg):
        self.ctx, self.cfg = ctx, cfg
        H, I = cfg["hidden"], cfg["inter"]
        self.nq = cfg["n_heads"] * cfg["head_dim"]
        self.nkv = cfg["n_kv"] * cfg["head_dim"]
        rng = np.random.default_rng(7)
        f16 = lambda n: rng.standard_normal(n).astype(np.float16).astype(np.float32)
        self.x = ctx.upload(f16(H))                       # residual stream
        # the attention output as the fused attention leaves it: quantized per 32 (quantQ8)
        self.attn_q, self.attn_s = ctx.zeros(self.nq), ctx.zeros(self.nq // 8)
        ctx.call("ti_quant_act_q8", ctx.upload(f16(self.nq)), self.attn_q, self.attn_s, None, self.nq)
        self.swq, self.sws = ctx.zeros(I), ctx.zeros(I // 8)    # swi, quantized by the gate/up kernel
        self.norm = ctx.upload(np.full(H, 0x3C00, np.uint16))   # RMSNorm weights 1.0
        self.q, self.k, self.v = ctx.zeros(self.nq * 4), ctx.zeros(self.nkv * 4), ctx.zeros(self.nkv * 4)
        self.logits = ctx.zeros(cfg["vocab"] * 4)
        self.hist = ctx.zeros(64)
        self.fam_bytes = {
            "qkv": qkv_bytes((self.nq, self.nkv, self.nkv), H),
            "o_proj": q8_linear_bytes(H, self.nq),
            "gateup": gateup_bytes(I, H),
            "down": q8_linear_bytes(H, I),
            "lm_head": lmhead_bytes(cfg["vocab"], H),
        }
        L = cfg["layers"]
        self.fam_launches = {"qkv": L, "o_proj": L, "gateup": L, "down": L, "lm_head": 1}
        self.bytes = sum(self.fam_bytes[f] * self.fam_launches[f] for f in self.FAMILIES)
        self.launches = sum(self.fam_launches.values())

    def issue(self, ws, families=FAMILIES, mark=None):
        """Launch the step's kernels of `families`; mark(fam, when) (when = 0 before, 1
        after a launch) lets a caller place event records around one family's launches."""
        c, cfg = self.ctx, self.cfg
        H, I = cfg["hidden"], cfg["inter"]
        eps = np.float32(1e-6)
        m = mark or (lambda fam, when: None)
        for Lw in ws.layers:
            if "qkv" in families:
                m("qkv", 0)
                c.call("ti_rmsnorm_gemv_q4", self.x, self.norm, eps, H, 3,
                       c_ptrs([Lw["q"][0], Lw["k"][0], Lw["v"][0]]), c_ptrs([Lw["q"][1], Lw["k"][1], Lw["v"][1]]),
                       c_ptrs([self.q, self.k, self.v]), c_ints([self.nq, self.nkv, self.nkv]), None, None)
                m("qkv", 1)
            if "o_proj" in families:
                m("o_proj", 0)
                c.call("ti_gemv_q4_q8", self.attn_q, self.attn_s, *Lw["o"], self.x, H, self.nq, 1)
                m("o_proj", 1)
            if "gateup" in families:
                m("gateup", 0)
                c.call("ti_rmsnorm_gateup_silu_q4", self.x, self.norm, eps, *Lw["gate"], *Lw["up"], None, I, H,
                       self.swq, self.sws)
                m("gateup", 1)
            if "down" in families:
                m("down", 0)
                c.call("ti_gemv_q4_q8", self.swq, self.sws, *Lw["down"], self.x, H, I, 1)
                m("down", 1)
        if "lm_head" in families:
            m("lm_head", 0)
            c.call("ti_rmsnorm_lm_head_argmax", self.x, self.norm, eps, *ws.lm, self.logits, cfg["vocab"], H,
                   self.hist, 1)
            m("lm_head", 1)


def graph_of(ctx, issue):
    ctx.graph_begin()
    try:
        issue()
    except Exception:
        try:
            ctx.graph_destroy(ctx.graph_end())      # close the capture so the stream stays usable
        except Exception:
            pass
        raise
    return ctx.graph_end()


def time_graphs(ctx, graphs, reps):
    """Average ms of one graph launch over `reps` launches cycling through `graphs`."""
    ctx.sync()
    ctx.record(20)
    for i in range(reps):
        ctx.graph_launch(graphs[i % len(graphs)])
    ctx.record(21)
    ctx.sync()
    return ctx.elapsed_ms(20, 21) / reps


class Flush:
    """Evicts the 256 MB Infinity Cache (and L2) between timed graph launches: a
    512 MB device-to-device copy, outside the timed interval."""

    def __init__(self, ctx, nbytes=512 << 20):
        self.ctx = ctx
        self.buf = ctx.alloc(2 * nbytes)
        self.n = nbytes

    def __call__(self):
        self.ctx.call("ti_buf_copy", self.buf, self.n, self.buf, 0, self.n)


def cold_ms(ctx, graphs, reps, flush):
    """Average ms of one graph launch, each launch timed alone (HIP events on the
    context stream) after a cache flush, cycling through `graphs`."""
    total = 0.0
    for i in range(reps):
        flush()
        ctx.record(30)
        ctx.graph_launch(graphs[i % len(graphs)])
        ctx.record(31)
        ctx.sync()
        total += ctx.elapsed_ms(30, 31)
    return total / reps


def family_profile(ctx, step, sets, flush, reps=12, keep=None, chain=True):
    """Per kernel family: its launches of one step (real shapes, all layers' weights)
    captured into one graph and timed with HIP events after a cache flush; the
    average per launch includes the back-to-back dispatch gaps inside the graph, and the
    graph's own launch. With two weight sets, also `in_chain_us`: the cost of one more
    launch in a chain, from a graph of the family's launches over both sets minus the
    graph over one (both cold), which leaves the graph launch and the first launch's
    start-up out, as inside the step."""
    out = {}
    out_keep = keep
    keep = []      # destroyed together at the end: under rocprofv3's kernel trace, launching a
    #                graph instantiated after another was destroyed has crashed the profiler
    for fam in Step.FAMILIES:
        gs = [graph_of(ctx, lambda ws=ws: step.issue(ws, (fam,))) for ws in sets]
        keep += gs
        time_graphs(ctx, gs, 2)
        ms = cold_ms(ctx, gs, reps, flush)
        n = step.fam_launches[fam]
        us = ms * 1e3 / n
        out[fam] = {"launches_per_step": n, "avg_us": round(us, 3), "bytes_per_launch": step.fam_bytes[fam],
                    "GB_s": round(step.fam_bytes[fam] / (us * 1e-6) / 1e9, 1)}
        if chain and len(sets) >= 2:
            g2 = [graph_of(ctx, lambda a=a, b=b: (step.issue(a, (fam,)), step.issue(b, (fam,))))
                  for a, b in ((sets[0], sets[1]), (sets[1], sets[0]))]
            keep += g2
            time_graphs(ctx, g2, 2)
            ms2 = cold_ms(ctx, g2, reps, flush)
            out[fam]["in_chain_us"] = round((ms2 - ms) * 1e3 / n, 3)
    ctx.sync()
    if out_keep is not None:
        out_keep += keep
    else:
        for g in keep:
            ctx.graph_destroy(g)
    return out


def sha256_file(path):
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def traffic_record(fam):
    """The HBM bytes per dispatch of family `fam`'s kernel from profiles/traffic.json (two
    rocprofv3 --pmc runs of this command, summarised by `python -m tabinfer_amd.rocprof_summary
    traffic`), its source line, the commit it was measured at, and whether it is stale: the
    file stamps the sha256 of each kernel source it was measured on, and any of them that
    differs from the file here now makes the figure stale (None when there is no stamp)."""
    tp = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(tp):
        return None, None, None, None
    with open(tp) as f:
        tj = json.load(f)
    stamp = tj.get("_stamp") or {}
    srcs = stamp.get("sources")
    stale = None
    if srcs:
        stale = any(not os.path.exists(os.path.join(ROOT, p)) or sha256_file(os.path.join(ROOT, p)) != h
                    for p, h in srcs.items())
    fams = tj.get("families", tj)
    return fams.get(fam), tj.get("_source"), stamp.get("commit"), stale


# ---- the launch boundary ----------------------------------------------------------------------
def launch_floor(ctx, n, reps=20, keep=None):
    """The cost of a kernel boundary when nothing else is done: chains of n stream-ordered
    launches captured in one HIP graph and launched like a decode step, (a) 4 KB copies
    of one workgroup, each reading what the previous one wrote, (b) 256 KB fills of 256
    workgroups (a full grid, as the step's kernels have). Returns us per launch of each."""
    buf = ctx.alloc(8192)
    big = ctx.alloc(2 << 20)
    ctx.call("ti_buf_fill_u32", buf, 1, 2048)

    def copies():
        for i in range(n):
            src, dst = (0, 4096) if i % 2 == 0 else (4096, 0)
            ctx.call("ti_buf_copy", buf, dst, buf, src, 4096)

    def fills():
        for i in range(n):
            ctx.call("ti_buf_fill_u32", big.at((i % 8) << 18), i, 1 << 16)
    out = []
    gs = []
    for issue in (copies, fills):
        g = graph_of(ctx, issue)
        gs.append(g)
        time_graphs(ctx, [g], 3)
        out.append(time_graphs(ctx, [g], reps) * 1e3 / n)
    ctx.sync()
    if keep is not None:       # the caller destroys them (see family_profile)
        keep += gs
    else:
        for g in gs:
            ctx.graph_destroy(g)
    buf.free()
    big.free()
    return out


# ---- the projection kernel's sustained rate at the Qwen3-1.7B K's ----------------------------
def gemv_sustained(ctx, pool, reps=12):
    """The batch-1 projection GEMV (int8 activation codes x int4 weights, ti_gemv_q4_q8) over
    many rows at the Qwen3-1.7B reduction sizes: the 28 layers' gate matrices stacked
    (172032 x 2048, 198 MB) and their down matrices stacked (57344 x 6144, 198 MB), six
    launches back to back in one graph cycling over three weight sets (a 594 MB live set,
    more than twice the 256 MB Infinity Cache, so each launch streams from HBM). The
    kernel's streaming rate once its launch and first round trip are amortised, which the
    decode step's 1-14 MB GEMVs never reach (see launch_floor)."""
    rng = np.random.default_rng(77)
    out = {}
    for name, N, K in (("gate_x28_2048", 172032, 2048), ("down_x28_6144", 57344, 6144)):
        sets = [pool.quantized(N, K, rng) for _ in range(3)]
        x = ctx.upload(rng.standard_normal(K).astype(np.float32))
        xq, xs, xsum = ctx.zeros(K), ctx.zeros(K // 8), ctx.zeros(K)
        ctx.call("ti_quant_act_q8", x, xq, xs, xsum, K)
        y = ctx.zeros(N * 4)

        def issue():
            for i in range(6):
                p, sc = sets[i % 3]
                ctx.call("ti_gemv_q4_q8", xq, xs, p, sc, y, N, K, 0)
        g = graph_of(ctx, issue)
        time_graphs(ctx, [g], 2)
        us = time_graphs(ctx, [g], reps) * 1e3 / 6
        ctx.graph_destroy(g)
        nb = int4_bytes(N, K) + K + (K // 32) * 4 + N * 4
        out[name] = {"N": N, "K": K, "us_per_launch": round(us, 2), "bytes_per_launch": nb,
                     "live_set_bytes": 3 * int4_bytes(N, K),
                     "GB_s": round(nb / (us * 1e-6) / 1e9, 1), "pct_of_hbm_peak": round(100 * nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 1)}
        for b in (x, xq, xs, xsum, y):
            b.free()
        for p, sc in sets:
            p.free()
            sc.free()
    return out


# ---- the Qwen3-1.7B int4 GEMV set (the north-star shapes), weights only ------------------------
def gemv_set_1p7b(ctx, pool, flush, steps=20):
    """The int4 GEMV set of one Qwen3-1.7B batch-1 decode step, launched as the decode step
    launches it (fused q/k/v, o_proj + residual, gate/up + SiLU + quantQ8, down + residual,
    28 layers, then rmsnorm + lm_head 151936 x 2048 + argmax): 967.75 MB of int4 weights,
    past the 256 MB Infinity Cache, so every step streams them from HBM. One HIP graph."""
    cfg = QWEN3_17B
    step = Step(ctx, cfg)
    ws = GemvSet(ctx, cfg, 300, pool)
    ctx.sync()
    g = graph_of(ctx, lambda: step.issue(ws))
    time_graphs(ctx, [g], 3)
    ms = time_graphs(ctx, [g], steps)
    ctx.graph_destroy(g)
    gbs = step.bytes / (ms * 1e-3) / 1e9
    res = {"ms_per_step": round(ms, 4), "bytes_per_step": step.bytes, "GB_s": round(gbs, 1),
           "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2), "launches_per_step": step.launches,
           "kernels_cold": family_profile(ctx, step, [ws], flush, reps=6)}
    for L in ws.layers:
        for p_, s_ in L.values():
            p_.free()
            s_.free()
    ws.lm[0].free()
    ws.lm[1].free()
    return res


# ---- full Qwen3-1.7B decode ----------------------------------------------------------------
def decode_1p7b(ctx, pool, contexts=(8192, 32768), steps=64, batch8=True, batch1=True):
    from tabinfer_amd import abi
    cfg = QWEN3_17B
    H, I, hd = cfg["hidden"], cfg["inter"], cfg["head_dim"]
    nq, nkv = cfg["n_heads"] * hd, cfg["n_kv"] * hd
    cap = max(contexts) + steps + 8
    m = abi.Qwen3(ctx, layers=cfg["layers"], hidden=H, intermediate=I, n_heads=cfg["n_heads"], n_kv_heads=cfg["n_kv"],
                  head_dim=hd, vocab=cfg["vocab"], rope_theta=1e6, rms_eps=1e-6, max_ctx=cap, max_tokens=8)
    rng = np.random.default_rng(17)
    shapes = {"self_attn.q_proj.weight": (nq, H), "self_attn.k_proj.weight": (nkv, H),
              "self_attn.v_proj.weight": (nkv, H), "self_attn.o_proj.weight": (H, nq),
              "mlp.gate_proj.weight": (I, H), "mlp.up_proj.weight": (I, H), "mlp.down_proj.weight": (H, I)}
    wbytes = 0
    for l in range(cfg["layers"]):
        for name, (N, K) in shapes.items():
            d, nd, s, ns = m.tensor("model.layers.%d.%s" % (l, name))
            pool.quantize_into(d, s, N, K, rng)
            wbytes += nd + ns
        for name in ("input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_norm.weight",
                     "self_attn.k_norm.weight"):
            d, nd, _, _ = m.tensor("model.layers.%d.%s" % (l, name))
            ctx.fill_u32(d, 0x3C003C00, nd // 4)      # norm weights 1.0
    d, nd, s, ns = m.tensor("lm_head.weight")
    pool.quantize_into(d, s, cfg["vocab"], H, rng)
    wbytes += nd + ns
    d, nd, _, _ = m.tensor("model.norm.weight")
    ctx.fill_u32(d, 0x3C003C00, nd // 4)
    d, nd, _, _ = m.tensor("model.embed_tokens.weight")   # f16 embeddings: N(0,0.02) bf16 pool bits as f16
    done = 0
    while done < nd:
        n = min(nd - done, pool.n * 2)
        ctx.call("ti_buf_copy", d, done, pool.buf, 0, n)
        done += n
    # seeded random prefix KV, written through the KV quantizer (kvQuantWrite)
    chunk = 2048
    kx = ctx.upload(rng.standard_normal(chunk * nkv).astype(np.float16).astype(np.float32))
    vx = ctx.upload(rng.standard_normal(chunk * nkv).astype(np.float16).astype(np.float32))
    for l in range(cfg["layers"]):
        for p0 in range(0, max(contexts), chunk):
            m.kv_write(l, kx, vx, chunk, p0)
    m.write_tokens(0, rng.integers(0, cfg["vocab"], cap + 1).astype(np.int32))
    ctx.sync()
    res = {}
    for S in contexts:
        res["ctx_%d" % S] = {}
        if batch1:
            m.set_pos(S)
            ctx.graph_begin()
            m.decode()
            g = ctx.graph_end()
            for _ in range(3):
                ctx.graph_launch(g)
            m.set_pos(S)
            ctx.sync()
            ctx.record(22)
            for _ in range(steps):
                ctx.graph_launch(g)
            ctx.record(23)
            ctx.sync()
            ms = ctx.elapsed_ms(22, 23) / steps
            ctx.graph_destroy(g)
            step_bytes = wbytes + cfg["layers"] * kv_bytes(S + steps // 2, cfg["n_kv"], hd)
            res["ctx_%d" % S].update({"tok_s": round(1e3 / ms, 1), "ms_per_token": round(ms, 4),
                                      "step_GB_s": round(step_bytes / (ms * 1e-3) / 1e9, 1),
                                      "pct_of_hbm_peak": round(100 * step_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                                      "bytes_per_step": step_bytes,
                                      "launches_per_step": 2 + (5 if QKV_SEPARATE else 4) * cfg["layers"]})
            log("decode 1.7B at %d: %.1f tok/s" % (S, 1e3 / ms))
        if not batch8:
            continue
        # batch 8 (a T = 8 forward of one sequence at positions S..S+7: the MFMA GEMM path)
        ctx.graph_begin()
        m.forward(None, S, T=8)
        g8 = ctx.graph_end()
        for _ in range(2):
            ctx.graph_launch(g8)
        ctx.sync()
        ctx.record(22)
        reps = 10
        for _ in range(reps):
            ctx.graph_launch(g8)
        ctx.record(23)
        ctx.sync()
        ms8 = ctx.elapsed_ms(22, 23) / reps
        ctx.graph_destroy(g8)
        res["ctx_%d" % S]["t8_forward_tok_s"] = round(8e3 / ms8, 1)
        res["ctx_%d" % S]["t8_forward_ms"] = round(ms8, 4)
        log("T=8 forward 1.7B at %d: %.1f tok/s" % (S, 8e3 / ms8))
    m.close()
    res["weights_bytes"] = wbytes
    if batch8:
        res["t8_forward"] = ("one forward of 8 consecutive tokens of one sequence at positions S..S+7 (the batch "
                             "configuration: the reference has no multi-sequence batching): every weight and the "
                             "KV cache read once for the 8 tokens, the lm_head once for the last token")
    return res


# ---- attention (one layer, fused step) --------------------------------------------------------
def attention(ctx, flush, contexts=(4096, 32768), reps=6):
    nHq, nKv, hd = 16, 8, 128
    rng = np.random.default_rng(23)
    cap = max(contexts) + 1
    row_w, row_g = nKv * hd // 4, nKv * hd // 32
    layers = 8       # distinct layer caches, cycled (8 x 75 MB at 32k: past the Infinity Cache)
    caches = []
    kx = ctx.upload(rng.standard_normal(2048 * nKv * hd).astype(np.float16).astype(np.float32))
    for _ in range(layers):
        c4 = [ctx.alloc(cap * row_w * 4), ctx.alloc(cap * row_g * 4), ctx.alloc(cap * row_w * 4), ctx.alloc(cap * row_g * 4)]
        for p0 in range(0, cap - 2048, 2048):
            ctx.call("ti_kv_write_q8", kx, kx, *c4, 2048, nKv, hd, p0)
        caches.append(c4)
    q = ctx.upload(rng.standard_normal(nHq * hd).astype(np.float32))
    k = ctx.upload(rng.standard_normal(nKv * hd).astype(np.float32))
    v = ctx.upload(rng.standard_normal(nKv * hd).astype(np.float32))
    w = ctx.upload(np.full(hd, 0x3C00, np.uint16))
    out = ctx.zeros(nHq * hd * 4)
    oq, os_ = ctx.zeros(nHq * hd), ctx.zeros(nHq * hd // 8)
    res = {}
    for S in contexts:
        def issue():
            for c4 in caches:
                ctx.call("ti_attn_step_q8", q, k, v, w, w, *c4, out, nHq, nKv, hd, S - 1, cap, np.float32(1e6),
                         np.float32(1e-6), 0, oq, os_)
        g = graph_of(ctx, issue)
        time_graphs(ctx, [g], 2)
        ms = cold_ms(ctx, [g], reps, flush)
        ctx.graph_destroy(g)
        us = ms * 1e3 / layers
        nb = kv_bytes(S, nKv, hd) + 2 * nHq * hd * 4
        res["S_%d" % S] = {"avg_us": round(us, 3), "bytes_per_launch": nb, "GB_s": round(nb / (us * 1e-6) / 1e9, 1)}
    for c4 in caches:
        for b in c4:
            b.free()
    return res


# ---- LFM2.5-8B-A1B int3 MoE experts ------------------------------------------------------------
def int3_bytes(N, K):
    return N * K // 32 * 14          # three u32 bitplanes + one f16 scale per 32 weights


def moe(ctx, flush, reps=4, layers=28):
    """One MoE block (router -> w1/w3 -> swiglu -> w2 -> combine, models/lfm25.js:2145-2166)
    at batch 1 (the fused decode launches) and batch 16 (ti_moe_prefill_q3: expert-grouped GEMMs, 5 launches), over
    `layers` independent expert sets (copies of one seeded set at distinct addresses) in
    one graph, so the weights stream from HBM the way consecutive decode layers do: at batch
    1 the 4 routed experts of 28 sets are 28 x 19.3 MB = 540 MB, more than twice the 256 MB
    Infinity Cache; us per block = graph time / layers."""
    H, I, nE, K = 2048, 1792, 32, 4
    rng = np.random.default_rng(5)
    base = []
    for N, Kc in ((I, H), (I, H), (H, I)):
        ng = nE * N * Kc // 32
        base.append((ctx.upload(rng.integers(0, 2 ** 32, ng * 3, dtype=np.uint64).astype(np.uint32)),
                     ctx.upload(rng.uniform(0.005, 0.02, ng).astype(np.float16).view(np.uint16)), ng))
    wsets = []
    for _ in range(layers):
        lw = []
        for p3, s3, ng in base:
            dp, ds = ctx.alloc(ng * 12), ctx.alloc(ng * 2)
            ctx.call("ti_buf_copy", dp, 0, p3, 0, ng * 12)
            ctx.call("ti_buf_copy", ds, 0, s3, 0, ng * 2)
            lw.append((dp, ds))
        wsets.append(lw)
    out = {}
    for T in (1, 16):
        P = T * K
        logits = rng.standard_normal(T * nE).astype(np.float32)
        idx = np.zeros(P, np.int32)
        # distinct experts this routing touches (the bytes a launch must read)
        s = 1.0 / (1.0 + np.exp(-logits.reshape(T, nE)))
        for t in range(T):
            idx[t * K:(t + 1) * K] = np.argsort(-s[t], kind="stable")[:K]
        ne = len(set(idx.tolist()))
        b = dict(normed=ctx.upload(rng.standard_normal(T * H).astype(np.float32)), logits=ctx.upload(logits),
                 bias=ctx.upload(np.zeros(nE, np.float32)), x=ctx.upload(rng.standard_normal(T * H).astype(np.float32)),
                 idx=ctx.zeros(P * 4), wt=ctx.zeros(P * 4), gate=ctx.zeros(P * I * 4), up=ctx.zeros(P * I * 4),
                 act=ctx.zeros(P * I * 4), out=ctx.zeros(P * H * 4))

        def issue(T=T, P=P, b=b):
            for lw in wsets:
                (p1, s1), (p3_, s3_), (p2, s2) = lw
                if T == 1:     # the fused decode block: [router + w1/w3 + swiglu], [w2 + combine]
                    ctx.call("ti_moe_decode_q3", b["x"], b["normed"], b["logits"], b["bias"], p1, s1, p3_, s3_, p2, s2,
                             b["idx"], b["wt"], b["act"], H, I, nE, K)
                    continue
                # the prefill block: [router + quant], [w1 + w3], [swiglu + quant], w2, combine
                ctx.call("ti_moe_prefill_q3", b["x"], b["normed"], b["logits"], b["bias"], p1, s1, p3_, s3_, p2, s2,
                         b["idx"], b["wt"], b["gate"], b["up"], b["act"], b["out"], T, H, I, nE, K)

        g = graph_of(ctx, issue)
        time_graphs(ctx, [g], 1)
        us = time_graphs(ctx, [g], reps) * 1e3 / layers
        ctx.graph_destroy(g)
        wbytes = ne * (2 * int3_bytes(I, H) + int3_bytes(H, I))
        out["batch%d" % T] = {"block_us": round(us, 2), "distinct_experts": ne, "weight_bytes": wbytes,
                              "live_set_bytes": layers * wbytes,
                              "GB_s": round(wbytes / (us * 1e-6) / 1e9, 1),
                              "pct_of_hbm_peak": round(100 * wbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 2),
                              "launches": 2 if T == 1 else 5}
        for v in b.values():
            v.free()
    for lw in wsets:
        for p3, s3 in lw:
            p3.free()
            s3.free()
    for p3, s3, _ in base:
        p3.free()
        s3.free()
    return out


# ---- Bonsai-1.7B ternary set (config 1): shapes, bytes, seeded codes ---------------------------
BONSAI_SHAPES = [(2048, 2048), (1024, 2048), (1024, 2048), (2048, 2048), (6144, 2048), (6144, 2048), (2048, 6144)]
BONSAI_LAYERS, BONSAI_VOCAB, BONSAI_H = 28, 151936, 2048


def tern_mat_bytes(N, K):      # codes + f32 scales (.cpu.bin layout) + int8 act + xsum + f32 out
    return N * K // 4 + (N * K // 64) * 4 + K + (K // 64) * 4 + N * 4


def tern_codes_fast(rng, nbytes):
    """Packed Q2_0_g64 code bytes whose four 2-bit codes are uniform on {0, 1, 2}: a
    byte-sized draw v in [0, 81) (16-bit uniforms scaled by 81) read as four base-3 digits."""
    lut = np.array([(v % 3) | ((v // 3 % 3) << 2) | ((v // 9 % 3) << 4) | ((v // 27 % 3) << 6) for v in range(81)],
                   np.uint8)
    u = rng.bit_generator.random_raw((nbytes + 3) // 4).view(np.uint16)[:nbytes].astype(np.uint32)
    return lut[(u * 81) >> 16]


def bonsai_set_bytes():
    layer = sum(tern_mat_bytes(N, K) for N, K in BONSAI_SHAPES)
    return BONSAI_LAYERS * layer + tern_mat_bytes(BONSAI_VOCAB, BONSAI_H), layer


def ternary_step(ctx, reps=10):
    """The Bonsai-1.7B ternary GEMV set of one decode step on the GPU: 28 layers (q/k/v in
    one launch, o, gate/up in one launch, down) + the 151936 x 2048 ternary lm_head, 28
    distinct layers' weights (537.6 MB: every step streams them from HBM), one graph."""
    import ctypes as C
    rng = np.random.default_rng(3)
    layer_host = [(tern_codes_fast(rng, N * K // 4), rng.uniform(0.01, 0.05, N * K // 64).astype(np.float16).astype(np.float32))
                  for N, K in BONSAI_SHAPES]
    layer_dev = [(ctx.upload(c), ctx.upload(sc)) for c, sc in layer_host]
    layers = []
    for l in range(BONSAI_LAYERS):
        mats = []
        for (N, K), (dc, ds) in zip(BONSAI_SHAPES, layer_dev):
            c2, s2 = ctx.alloc(N * K // 4), ctx.alloc(N * K // 64 * 4)
            ctx.call("ti_buf_copy", c2, 0, dc, 0, N * K // 4)
            ctx.call("ti_buf_copy", s2, 0, ds, 0, N * K // 64 * 4)
            mats.append((c2, s2))
        layers.append(mats)
    lm = (ctx.upload(tern_codes_fast(rng, BONSAI_VOCAB * BONSAI_H // 4)),
          ctx.upload(rng.uniform(0.01, 0.05, BONSAI_VOCAB * BONSAI_H // 64).astype(np.float16).astype(np.float32)))
    acts = {K: (ctx.upload(rng.integers(-127, 128, K, dtype=np.int8)), ctx.upload(np.zeros(K // 64, np.int32)))
            for K in (2048, 6144)}
    o3 = [ctx.zeros(N * 4) for N in (2048, 1024, 1024)]
    og = [ctx.zeros(6144 * 4) for _ in range(2)]
    o2, olm = ctx.zeros(2048 * 4), ctx.zeros(BONSAI_VOCAB * 4)
    arr = lambda vals, t=C.c_void_p: (t * len(vals))(*vals)

    def issue():
        a, x = acts[2048]
        for (q, k, v, o, g, u, d) in layers:
            ctx.call("ti_tern_gemv_multi", a, x, 2048, 3, arr([q[0].ptr, k[0].ptr, v[0].ptr]), arr([q[1].ptr, k[1].ptr, v[1].ptr]),
                     arr([b.ptr for b in o3]), arr([2048, 1024, 1024], C.c_int))
            ctx.call("ti_tern_gemv", o2, o[0], o[1], a, x, 2048, 2048)
            ctx.call("ti_tern_gemv_multi", a, x, 2048, 2, arr([g[0].ptr, u[0].ptr]), arr([g[1].ptr, u[1].ptr]),
                     arr([b.ptr for b in og]), arr([6144, 6144], C.c_int))
            ctx.call("ti_tern_gemv", o2, d[0], d[1], acts[6144][0], acts[6144][1], 2048, 6144)
        ctx.call("ti_tern_gemv", olm, lm[0], lm[1], a, x, BONSAI_VOCAB, BONSAI_H)

    g = graph_of(ctx, issue)
    time_graphs(ctx, [g], 2)
    ms = time_graphs(ctx, [g], reps)
    ctx.graph_destroy(g)
    nb, layer_b = bonsai_set_bytes()
    for mats in layers:
        for c2, s2 in mats:
            c2.free()
            s2.free()
    return {"step_us": round(ms * 1e3, 1), "bytes_per_step": nb, "GB_s": round(nb / (ms * 1e-3) / 1e9, 1),
            "pct_of_hbm_peak": round(100 * nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
            "GMAC_s": round((BONSAI_LAYERS * sum(N * K for N, K in BONSAI_SHAPES) + BONSAI_VOCAB * BONSAI_H) / (ms * 1e-3) / 1e9, 1),
            "launches_per_step": 4 * BONSAI_LAYERS + 1,
            "what": "28 layers (q/k/v in one launch, o, gate/up in one launch, down) + lm_head 151936x2048, distinct weights"}


def tern2_step(ctx, reps=10):
    """The Bonsai-1.7B GEMV set of one decode step in the reference's on-GPU ternary format
    (quantizeTernaryBf16's codes, f16 scales per 32; gemvTern2 / gateupTern2): 28 distinct
    layers of q, k, v, o (ti_gemv_tern2 each), gate/up + SiLU (ti_gateup_silu_tern2), down,
    then the 151936 x 2048 lm_head, one graph; int8 activations with their sums."""
    rng = np.random.default_rng(4)
    def mat(N, K):
        return (ctx.upload(tern_codes_fast(rng, N * K // 4)),
                ctx.upload(rng.uniform(0.01, 0.05, N * K // 32).astype(np.float16).view(np.uint16)))
    src = {shape: mat(*shape) for shape in set(BONSAI_SHAPES)}
    layers = []
    for l in range(BONSAI_LAYERS):
        mats = []
        for N, K in BONSAI_SHAPES:
            c0, s0 = src[(N, K)]
            c2, s2 = ctx.alloc(N * K // 4), ctx.alloc(N * K // 16)
            ctx.call("ti_buf_copy", c2, 0, c0, 0, N * K // 4)
            ctx.call("ti_buf_copy", s2, 0, s0, 0, N * K // 16)
            mats.append((c2, s2))
        layers.append(mats)
    lm = mat(BONSAI_VOCAB, BONSAI_H)
    acts = {}
    for K in (2048, 6144):
        acts[K] = (ctx.upload(rng.integers(0, 2 ** 32, K // 4, dtype=np.uint64).astype(np.uint32)),
                   ctx.upload(rng.uniform(0.01, 0.02, K // 32).astype(np.float32)),
                   ctx.upload(rng.integers(-500, 500, K // 16).astype(np.int32)))
    outs = {N: ctx.zeros(N * 4) for N in (1024, 2048, 6144, BONSAI_VOCAB)}

    def issue():
        a = acts[2048]
        for (q, k, v, o, g, u, d) in layers:
            for (cm, sm), N in ((q, 2048), (k, 1024), (v, 1024), (o, 2048)):
                ctx.call("ti_gemv_tern2", *a, cm, sm, outs[N], N, 2048, 0)
            ctx.call("ti_gateup_silu_tern2", *a, g[0], g[1], u[0], u[1], outs[6144], 6144, 2048)
            ctx.call("ti_gemv_tern2", *acts[6144], d[0], d[1], outs[2048], 2048, 6144, 0)
        ctx.call("ti_gemv_tern2", *a, lm[0], lm[1], outs[BONSAI_VOCAB], BONSAI_VOCAB, BONSAI_H, 0)

    g = graph_of(ctx, issue)
    time_graphs(ctx, [g], 2)
    ms = time_graphs(ctx, [g], reps)
    ctx.graph_destroy(g)
    for mats in layers:
        for c2, s2 in mats:
            c2.free()
            s2.free()
    nb = BONSAI_LAYERS * sum(N * K * 5 // 16 for N, K in BONSAI_SHAPES) + BONSAI_VOCAB * BONSAI_H * 5 // 16
    return {"step_us": round(ms * 1e3, 1), "bytes_per_step": nb, "GB_s": round(nb / (ms * 1e-3) / 1e9, 1),
            "pct_of_hbm_peak": round(100 * nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2), "launches_per_step": 6 * BONSAI_LAYERS + 1,
            "what": "28 layers (q, k, v, o, gate/up + SiLU, down) + lm_head 151936x2048 in the reference's on-GPU "
                    "ternary format (2-bit codes, f16 scale per 32), distinct weights"}


def bonsai_decode(ctx, contexts=(1024, 8192), steps=64, eager=False):
    """The Bonsai-1.7B ternary decoder (ti_bonsai_*, model.rs's forward) at batch 1: one
    captured decode step (6 launches per layer) replayed token after token over an f32 KV
    prefix of S positions; every layer's distinct ternary weights (541 MB with the lm_head)
    and the f32 KV cache (S x 8 KV heads x 128 x 2 x 4 B per layer) stream from HBM."""
    from tabinfer_amd import abi
    rng = np.random.default_rng(5)
    H, I, nq, nkv = BONSAI_H, 6144, 2048, 1024
    shapes = {"self_attn.q_proj.weight": (nq, H), "self_attn.k_proj.weight": (nkv, H), "self_attn.v_proj.weight": (nkv, H),
              "self_attn.o_proj.weight": (H, nq), "mlp.gate_proj.weight": (I, H), "mlp.up_proj.weight": (I, H),
              "mlp.down_proj.weight": (H, I)}
    src = {}
    for name, (N, K) in shapes.items():
        if (N, K) not in src:
            src[(N, K)] = (ctx.upload(tern_codes_fast(rng, N * K // 4)),
                           ctx.upload(rng.uniform(0.01, 0.05, N * K // 64).astype(np.float16).astype(np.float32)))
    out = {}
    for S in contexts:
        m = abi.Bonsai(ctx, layers=BONSAI_LAYERS, hidden=H, intermediate=I, n_heads=16, n_kv_heads=8, head_dim=128,
                       vocab=BONSAI_VOCAB, rope_theta=1e6, rms_eps=1e-6, max_ctx=S + steps + 8)
        try:
            for l in range(BONSAI_LAYERS):
                pre = "model.layers.%d." % l
                for name, (N, K) in shapes.items():
                    dp, nd, sp, ns = m.tensor(pre + name)
                    c0, s0 = src[(N, K)]
                    ctx.call("ti_buf_copy", dp, 0, c0, 0, nd)
                    ctx.call("ti_buf_copy", sp, 0, s0, 0, ns)
                for name in ("input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_norm.weight",
                             "self_attn.k_norm.weight"):
                    dp, nd, _, _ = m.tensor(pre + name)
                    ctx.call("ti_buf_fill_u32", dp, 0x3F800000, nd // 4)            # 1.0f
                k, v = m.kv(l)
                n = (S + steps + 8) * nkv
                ctx.call("ti_buf_fill_u32", k, 0x3C23D70A, n)                        # 0.01f
                ctx.call("ti_buf_fill_u32", v, 0x3C23D70A, n)
            dp, nd, _, _ = m.tensor("model.norm.weight")
            ctx.call("ti_buf_fill_u32", dp, 0x3F800000, nd // 4)
            dp, nd, sp, ns = m.tensor("lm_head.weight")
            ctx.write(dp, tern_codes_fast(rng, nd))
            ctx.write(sp, rng.uniform(0.01, 0.05, ns // 4).astype(np.float16).astype(np.float32))
            dp, nd, _, _ = m.tensor("model.embed_tokens.weight")
            ctx.call("ti_buf_fill_u32", dp, 0x2E663266, nd // 4)                  # f16 pairs ~0.1 / ~0.2
            m.write_tokens(S, np.array([17], np.int32))
            m.set_pos(S)
            ctx.sync()
            if eager:                       # launched directly (kernel traces without graphs)
                for _ in range(4):
                    m.decode()
                m.set_pos(S)
                ctx.sync()
                ctx.record(30)
                for _ in range(steps):
                    m.decode()
                ctx.record(31)
                ctx.sync()
                ms = ctx.elapsed_ms(30, 31) / steps
            else:
                g = graph_of(ctx, m.decode)
                try:
                    for _ in range(4):
                        ctx.graph_launch(g)
                    ctx.sync()
                    m.set_pos(S)
                    ctx.sync()
                    ctx.record(30)
                    for _ in range(steps):
                        ctx.graph_launch(g)
                    ctx.record(31)
                    ctx.sync()
                    ms = ctx.elapsed_ms(30, 31) / steps
                finally:
                    ctx.graph_destroy(g)
        finally:
            m.close()
        wb, _ = bonsai_set_bytes()
        kvb = BONSAI_LAYERS * S * nkv * 2 * 4
        out["ctx_%d" % S] = {"tok_s": round(1e3 / ms, 1), "ms_per_token": round(ms, 4),
                             "step_GB_s": round((wb + kvb) / (ms * 1e-3) / 1e9, 1),
                             "pct_of_hbm_peak": round(100 * (wb + kvb) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                             "bytes_per_step": wb + kvb}
    return out


# ---- the CPU baseline: the reference's native CPU path on config 1 --------------------------------
def cpu_features():
    """CPU model, logical CPUs, usable CPUs and the SIMD features that set the ternary
    kernel's ceiling (native/crates/n2-kernels/src/cpu.rs:16-80)."""
    model, flags = "unknown", set()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            elif line.startswith("flags") and not flags:
                flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    want = ("avx2", "fma", "avx_vnni", "avx512f", "avx512_vnni", "bmi2")
    return {"model": model, "nproc": os.cpu_count(), "usable": len(os.sched_getaffinity(0)),
            "features": {f: f in flags for f in want}}


def _once(f):
    t0 = time.perf_counter()
    f()
    return time.perf_counter() - t0


def ab_min(a, b, reps, warmup):
    """Alternating-order, warmed-up, min-of-reps A/B (native/crates/n2-kernels/src/timing.rs:65-98)."""
    for _ in range(warmup):
        _once(a)
        _once(b)
    ta = tb = float("inf")
    for i in range(reps):
        if i % 2 == 0:
            ta = min(ta, _once(a))
            tb = min(tb, _once(b))
        else:
            tb = min(tb, _once(b))
            ta = min(ta, _once(a))
    return ta, tb


CPU_REPS = 241


def cpu_baseline(threads=16):
    """The reference's native CPU path, n2 avx2::gemv_tern (restated in C,
    oracle/tern_avx2.c), over the whole Bonsai-1.7B ternary GEMV set of one decode step
    28 distinct layers + the 151936 x 2048 lm_head, 537.6 MB of codes
    and f32 scales (DRAM-streaming), activations quantized by n2's quantize_act. Timed with
    the reference's discipline (timing.rs): a base-vs-base control that must read
    1.00 +- 0.15 (retried up to 3 times, else the figures are withheld), then 1 thread
    (the reference's configuration) against N threads on a persistent pool (a barrier after
    each GEMV, as a forward pass needs), alternating order, 3 warm-ups, min of CPU_REPS (at
    least the reference's 31; 241 passes of each make a ~10 s sample)."""
    from oracle import oracle as orc
    if not orc.has_avx2():
        return None
    rng = np.random.default_rng(3)
    layer = [(tern_codes_fast(rng, N * K // 4), rng.uniform(0.01, 0.05, N * K // 64).astype(np.float16).astype(np.float32))
             for N, K in BONSAI_SHAPES]
    acts = {K: orc.tern_quant_act_n2(rng.standard_normal(K).astype(np.float32)) for K in (2048, 6144)}
    mats = []
    for l in range(BONSAI_LAYERS):
        for (N, K), (c, sc) in zip(BONSAI_SHAPES, layer):
            a, xs, _ = acts[K]
            mats.append((c.copy(), sc.copy(), a, xs, np.zeros(N, np.float32), N, K))   # distinct addresses
    a, xs, _ = acts[BONSAI_H]
    mats.append((tern_codes_fast(rng, BONSAI_VOCAB * BONSAI_H // 4),
                 rng.uniform(0.01, 0.05, BONSAI_VOCAB * BONSAI_H // 64).astype(np.float16).astype(np.float32), a, xs,
                 np.zeros(BONSAI_VOCAB, np.float32), BONSAI_VOCAB, BONSAI_H))
    # correctness first, as the reference checks its kernel (native/crates/n2-cli/src/main.rs:
    # 132-138): within 1e-5 of the dequant oracle on the first layer's matrices
    for c, sc, a_, x_, _, N, K in mats[:len(BONSAI_SHAPES)]:
        got = orc.tern_gemv_avx2(c, sc, a_, x_, N, K)
        ref = orc.tern_gemv_dequant(c, sc, a_, N, K)
        assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    nthreads = max(1, min(threads, len(os.sched_getaffinity(0))))
    pool = orc.TernPool(mats, nthreads)
    nb, _ = bonsai_set_bytes()
    macs = BONSAI_LAYERS * sum(N * K for N, K in BONSAI_SHAPES) + BONSAI_VOCAB * BONSAI_H
    t0 = time.perf_counter()
    try:
        control = None
        for attempt in range(3):
            c1, c2 = ab_min(pool.run_serial, pool.run_serial, 9, 2)
            control = c1 / c2
            if abs(control - 1.0) <= 0.15:
                break
        clean = abs(control - 1.0) <= 0.15
        t1, tn = ab_min(pool.run_serial, pool.run, CPU_REPS, 3)
    finally:
        pool.close()
    dt = time.perf_counter() - t0
    f = cpu_features()
    res = {"value": round(nb / t1 / 1e9, 2) if clean else None, "unit": "GB/s", "cores": 1, "kind": "port",
           "sample": "n2 avx2::gemv_tern restated in C (oracle/tern_avx2.c), the reference's native CPU path (it "
                     "has no CPU int4 path): the Bonsai-1.7B ternary GEMV set of one decode step, 28 layers + "
                     "lm_head 151936x2048, %.1f MB; min of %d alternating 1-thread/%d-thread passes after 3 "
                     "warm-ups; %.1f s" % (nb / 1e6, CPU_REPS, pool.threads, dt),
           "ms_per_step_1t": round(t1 * 1e3, 2), "GMAC_s_1t": round(macs / t1 / 1e9, 2),
           "threads_n": {"threads": pool.threads, "GB_s": round(nb / tn / 1e9, 2) if clean else None,
                         "GMAC_s": round(macs / tn / 1e9, 2) if clean else None, "ms_per_step": round(tn * 1e3, 2)},
           "control": round(control, 3), "control_clean": clean, "cpu": f}
    if not clean:
        res["withheld"] = "the base-vs-base control read %.3f, outside 1.00 +- 0.15" % control
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--only", choices=("gemv", "all", "moe", "decode", "decode8", "tern", "tern2", "bonsai"),
                    default="all",
                    help="gemv: the headline workload only; moe: headline + the int3 MoE leg; "
                         "decode: the Qwen3-1.7B batch-1 decode leg alone, --steps tokens (no headline line); "
                         "decode8: its batch-8 (T = 8 forward) leg alone; tern: the ternary GEMV step alone; tern2: "
                         "the same step in the on-GPU ternary format; "
                         "bonsai: the Bonsai decoder alone at --ctx (default 1024) (no headline line)")
    ap.add_argument("--eager", action="store_true", help="--only bonsai: launch the steps directly, without a graph")
    ap.add_argument("--no-chain", action="store_true",
                    help="skip kernels[].in_chain_us (its two-set graphs crash rocprofv3's kernel trace; profiling "
                         "runs pass this)")
    ap.add_argument("--ctx", type=int, nargs="*", default=None,
                    help="context lengths of the decode leg (default 8192 32768)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one MI355X: this build runs on a single GPU (the multi-GPU sharding is a "
              "design only); --gpus %d is not supported" % args.gpus, file=sys.stderr)
        sys.exit(2)

    from tabinfer_amd import abi
    ctx = abi.Ctx(0)
    contexts = tuple(args.ctx) if args.ctx else (8192, 32768)
    if args.only in ("decode", "decode8"):   # one Qwen3-1.7B decode leg alone (profiling runs)
        pool = Pool(ctx, 48 << 20, 1234)
        log("decode 1.7B")
        res = decode_1p7b(ctx, pool, contexts=contexts, steps=args.steps, batch8=args.only == "decode8",
                          batch1=args.only == "decode")
        ctx.close()
        print(json.dumps({"decode_1p7b": res}))
        return
    if args.only in ("tern", "tern2", "bonsai"):   # one ternary leg alone, one graph per process (profiling runs)
        if args.only == "tern":
            log("ternary step")
            res = {"ternary_bonsai_step": ternary_step(ctx)}
        elif args.only == "tern2":
            log("ternary step, on-GPU format")
            res = {"ternary_gpu_format_step": tern2_step(ctx)}
        else:
            log("bonsai decode")
            res = {"bonsai_decode": bonsai_decode(ctx, contexts=tuple(args.ctx) if args.ctx else (1024,),
                                                  eager=args.eager)}
        ctx.close()
        print(json.dumps(res))
        return
    cfg = QWEN3_06B
    step = Step(ctx, cfg)
    log("building weights (2 sets x %.0f MB)" % (step.bytes / 1e6))
    pool = Pool(ctx, 48 << 20, 1234)
    sets = [GemvSet(ctx, cfg, 100 + i, pool) for i in range(2)]
    ctx.sync()
    graphs = [graph_of(ctx, lambda ws=ws: step.issue(ws)) for ws in sets]
    for i in range(args.warmup):
        ctx.graph_launch(graphs[i % 2])
    ctx.sync()
    log("timing %d steps" % args.steps)
    ctx.record(10)
    for i in range(args.steps):
        ctx.graph_launch(graphs[i % 2])
    ctx.record(11)
    ctx.sync()
    ms_per_step = ctx.elapsed_ms(10, 11) / args.steps
    value = step.bytes / (ms_per_step * 1e-3) / 1e9

    log("launch floor")
    held = list(graphs)        # every graph of this leg is destroyed after the last launch
    floor_copy_us, floor_us = launch_floor(ctx, step.launches, keep=held)
    log("kernel families")
    flush = Flush(ctx)
    kern = family_profile(ctx, step, sets, flush, keep=held, chain=not args.no_chain)
    # the family that carries the most of the step's HBM bytes (gate/up: 99 of 337 MB); by
    # time per step gate/up and q/k/v are within 1% of each other and trade places between
    # runs, while the byte count is fixed by the shapes
    ctx.sync()
    for g in held:
        ctx.graph_destroy(g)
    dom_name = max(kern, key=lambda k: kern[k]["bytes_per_launch"] * kern[k]["launches_per_step"])
    dom = kern[dom_name]
    achieved = dom["bytes_per_launch"] / (dom["avg_us"] * 1e-6) / 1e9
    timing = ("cold, in the graph: the family's launches of one step (every layer's weights) back to back in one "
              "graph, timed with HIP events around the graph on the context stream after a 512 MiB flush, divided "
              "by the launches (gaps included); the rocprofv3 kernel trace of this command "
              "(profiles/gemv06_set_kernel_trace.md) records each dispatch about 0.5 us longer, its own "
              "per-dispatch timestamps included")
    traffic, traffic_src, traffic_stamp, traffic_stale = traffic_record(dom_name)
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int4xint8",
        "data": "synthetic (seeded bf16 N(0,0.02) weights, GPU-quantized; N(0,1) f16 activations)",
        "config": {"workload": "Qwen3-0.6B int4 GEMV set of one batch-1 decode step: 28 x [rmsnorm+q/k/v 1024->2048/1024/1024] "
                               "[o 2048->1024 +res] [rmsnorm+gate/up 1024->3072 +SiLU+quant] [down 3072->1024 +res] + "
                               "rmsnorm+lm_head 1024->151936+argmax; fused launches, one HIP graph per step",
                   "bytes_per_step": step.bytes, "launches_per_step": step.launches, "weight_sets": 2,
                   "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2)},
        "roofline": {"bound": "hbm", "kernel": dom_name, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "avg_us": dom["avg_us"], "bytes_per_launch": dom["bytes_per_launch"],
                     "timing": timing, "traffic_source": traffic_src,
                     "traffic_measured_at": traffic_stamp, "traffic_stale": traffic_stale},
        "kernels": kern,
        "kernels_in_chain_ms_per_step": (round(sum(k["in_chain_us"] * k["launches_per_step"] for k in kern.values()) * 1e-3, 4)
                                         if all("in_chain_us" in k for k in kern.values()) else None),
        "launch_floor": {
            "us_per_launch": round(floor_us, 3), "us_per_launch_1wg_copy": round(floor_copy_us, 3),
            "launches": step.launches, "floor_ms_per_step": round(floor_us * step.launches * 1e-3, 4),
            "step_over_floor": round(ms_per_step / (floor_us * step.launches * 1e-3), 3),
            "what": "chains of %d stream-ordered launches in one HIP graph doing (almost) nothing: 256 KB fills "
                    "of 256 workgroups (us_per_launch), 4 KB copies of one workgroup each reading the previous "
                    "one's output (us_per_launch_1wg_copy); the step's kernel boundaries alone cost "
                    "floor_ms_per_step; step_over_floor = ms_per_step / floor_ms_per_step" % step.launches},
    }
    if args.only == "moe":
        log("int3 MoE")
        out["moe_lfm25_block"] = moe(ctx, flush)
    if args.only == "all":
        log("Qwen3-1.7B int4 GEMV set")
        out["gemv_set_1p7b"] = gemv_set_1p7b(ctx, pool, flush)
        log("projection GEMV, sustained")
        out["gemv_sustained_1p7b"] = gemv_sustained(ctx, pool)
        log("ternary step")
        out["ternary_bonsai_step"] = ternary_step(ctx)
        log("ternary step, on-GPU format")
        out["ternary_gpu_format_step"] = tern2_step(ctx)
        log("int3 MoE")
        out["moe_lfm25_block"] = moe(ctx, flush)
        log("attention")
        out["attention_layer"] = attention(ctx, flush)
        log("decode 1.7B")
        out["decode_1p7b"] = decode_1p7b(ctx, pool, contexts=contexts)
        log("bonsai decode")
        out["bonsai_decode"] = bonsai_decode(ctx)
        # the same boundary floor under each batch-1 step of its launch count
        for leg in (out["gemv_set_1p7b"], out["ternary_bonsai_step"], out["ternary_gpu_format_step"],
                    *(v for k, v in out["decode_1p7b"].items() if k.startswith("ctx_"))):
            if isinstance(leg, dict) and "launches_per_step" in leg:
                leg["launch_floor_ms"] = round(floor_us * leg["launches_per_step"] * 1e-3, 4)
    if not args.no_cpu:
        log("cpu baseline")
        cb = cpu_baseline()
        if cb:
            out["cpu_baseline"] = cb
    ctx.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
