#!/usr/bin/env python3
"""Benchmark of the quantized decode hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Workload (one "step"): the int4 GEMV set of one Qwen3-0.6B decode step at batch
1, launched exactly as the reference's decode issues it (models/qwen3.js:
3981-4049): per layer q/k/v GEMVs on the RMSNorm'd int8 activation (projGemv),
o_proj through linearQ (int8 quantize + GEMV, fused residual), fused
gate+up+SiLU, down_proj through linearQ; then the lm_head through linearQ's
f32-activation GEMV (N = 151936 >= 16384). 28 layers, hidden 1024,
intermediate 3072, 16/8 heads of dim 128. Weights are seeded bf16 N(0, 0.02)
quantized on the GPU by the int4 quantizer (the reference's quantizeInt4Bf16);
activations are seeded N(0,1) rounded to f16. Two independent weight sets
(2 x 335 MB) alternate between steps so every step streams its weights from HBM,
not from the 256 MB Infinity Cache. Each step is one captured HIP graph.

Prints one JSON line: value = algorithmic GB/s of the whole step (weights +
activations + outputs, counted once per launch) over the timed steps.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0

QWEN3_06B = dict(layers=28, hidden=1024, inter=3072, n_heads=16, n_kv=8, head_dim=128, vocab=151936)


def int4_bytes(N, K):
    return N * K // 2 + (N * K // 32) * 2


def gemv_q8_bytes(N, K):       # weights + int8 act (codes + scales) + f32 out
    return int4_bytes(N, K) + K + (K // 32) * 4 + N * 4


def linear_q8_bytes(N, K):     # f32 act in, quantized inside linearQ
    return int4_bytes(N, K) + K * 4 + N * 4


def gemv_f32_bytes(N, K):
    return int4_bytes(N, K) + K * 4 + N * 4


def gateup_bytes(I, H):
    return 2 * int4_bytes(I, H) + H + (H // 32) * 4 + I * 4


class GemvSet:
    """Device-resident weights and activations of one 0.6B decode step."""

    def __init__(self, ctx, cfg, seed, pool):
        from tabinfer_amd import abi
        self.ctx, self.cfg = ctx, cfg
        H, I = cfg["hidden"], cfg["inter"]
        nq = cfg["n_heads"] * cfg["head_dim"]
        nkv = cfg["n_kv"] * cfg["head_dim"]
        rng = np.random.default_rng(seed)
        self.shapes = {"q": (nq, H), "k": (nkv, H), "v": (nkv, H), "o": (H, nq),
                       "gate": (I, H), "up": (I, H), "down": (H, I)}
        self.layers = []
        for _ in range(cfg["layers"]):
            L = {}
            for name, (N, K) in self.shapes.items():
                L[name] = self._quantized(N, K, rng, pool)
            self.layers.append(L)
        self.lm = self._quantized(cfg["vocab"], H, rng, pool)

    def _quantized(self, N, K, rng, pool):
        """int4-quantize N x K bf16 weights drawn from the device pool, on the GPU."""
        ctx = self.ctx
        pack = ctx.alloc(N * K // 2)
        sc = ctx.alloc(N * K // 32 * 2)
        pool_buf, pool_n = pool
        rows_per = max(1, min(N, pool_n // K))
        r = 0
        while r < N:
            nr = min(rows_per, N - r)
            span = nr * K
            off = int(rng.integers(0, (pool_n - span) // 32 + 1)) * 32
            ctx.call("ti_quant_int4_bf16", pool_buf.at(off * 2), pack.at(r * K // 2), sc.at(r * K // 32 * 2), nr, K)
            r += nr
        return pack, sc


def make_pool(ctx, n, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.02))
    bf = (w.view(np.uint32) >> 16).astype(np.uint16)
    return ctx.upload(bf), n


class Step:
    """The launch sequence of one decode step's GEMV set (and its byte count)."""

    def __init__(self, ctx, cfg, act):
        self.ctx, self.cfg, self.act = ctx, cfg, act
        H, I = cfg["hidden"], cfg["inter"]
        nq = cfg["n_heads"] * cfg["head_dim"]
        nkv = cfg["n_kv"] * cfg["head_dim"]
        per_layer = (gemv_q8_bytes(nq, H) + 2 * gemv_q8_bytes(nkv, H) + linear_q8_bytes(H, nq)
                     + gateup_bytes(I, H) + linear_q8_bytes(H, I))
        self.bytes = cfg["layers"] * per_layer + gemv_f32_bytes(cfg["vocab"], H)
        self.launches = cfg["layers"] * 8 + 1   # 3 gemv + 2x(quant+gemv) + gateup, + lm_head

    def issue(self, ws):
        c, a, cfg = self.ctx, self.act, self.cfg
        H, I = cfg["hidden"], cfg["inter"]
        nq = cfg["n_heads"] * cfg["head_dim"]
        nkv = cfg["n_kv"] * cfg["head_dim"]
        for L in ws.layers:
            c.call("ti_gemv_q4_q8", a["xq"], a["xs"], *L["q"], a["q"], nq, H, 0)
            c.call("ti_gemv_q4_q8", a["xq"], a["xs"], *L["k"], a["k"], nkv, H, 0)
            c.call("ti_gemv_q4_q8", a["xq"], a["xs"], *L["v"], a["v"], nkv, H, 0)
            c.call("ti_linear_q4", a["attn"], *L["o"], a["x"], 1, H, nq, 1)
            c.call("ti_gateup_silu_q4", a["xq"], a["xs"], *L["gate"], *L["up"], a["swi"], I, H)
            c.call("ti_linear_q4", a["swi"], *L["down"], a["x"], 1, H, I, 1)
        c.call("ti_linear_q4", a["last"], *ws.lm, a["logits"], 1, cfg["vocab"], H, 0)


def make_acts(ctx, cfg, seed):
    rng = np.random.default_rng(seed)
    H, I = cfg["hidden"], cfg["inter"]
    nq = cfg["n_heads"] * cfg["head_dim"]
    f16 = lambda n: rng.standard_normal(n).astype(np.float16).astype(np.float32)
    x_norm = f16(H)
    a = {}
    # q/k/v and gate/up read the RMSNorm'd int8 activation (quantized on the GPU)
    dx = ctx.upload(x_norm)
    a["xq"], a["xs"], a["xsum"] = ctx.zeros(H), ctx.zeros(H // 8), ctx.zeros(H // 4)
    ctx.call("ti_quant_act_q8", dx, a["xq"], a["xs"], a["xsum"], H)
    a["attn"] = ctx.upload(f16(nq))
    a["last"] = ctx.upload(f16(H))
    a["x"] = ctx.upload(f16(H))
    for name, n in (("q", nq), ("k", cfg["n_kv"] * cfg["head_dim"]), ("v", cfg["n_kv"] * cfg["head_dim"]),
                    ("swi", I), ("logits", cfg["vocab"])):
        a[name] = ctx.zeros(n * 4)
    return a


def kernel_profile(ctx, step, ws, lm_copies):
    """Average duration of each kernel family over its launches in one step: the
    family's launches (real shapes, all 28 layers' weights) are captured into one
    graph and timed with HIP events on the context stream, so the average includes
    the back-to-back dispatch gaps (a lower bound on the kernel's bandwidth)."""
    cfg, a = step.cfg, step.act
    H, I = cfg["hidden"], cfg["inter"]
    nq = cfg["n_heads"] * cfg["head_dim"]
    nkv = cfg["n_kv"] * cfg["head_dim"]
    fams = {}

    def timed(name, issue, n, nbytes):
        ctx.graph_begin()
        issue()
        g = ctx.graph_end()
        ctx.sync()
        ctx.record(0)
        ctx.graph_launch(g)
        ctx.record(1)
        ms = ctx.elapsed_ms(0, 1)
        ctx.graph_destroy(g)
        fams[name] = {"launches": n, "avg_us": ms * 1e3 / n, "bytes_per_launch": nbytes / n}

    def qkv():
        for l in ws.layers:
            for nm, N in (("q", nq), ("k", nkv), ("v", nkv)):
                ctx.call("ti_gemv_q4_q8", a["xq"], a["xs"], *l[nm], a[nm], N, H, 0)
    timed("gemv_q4_q8", qkv, 3 * len(ws.layers),
          len(ws.layers) * (gemv_q8_bytes(nq, H) + 2 * gemv_q8_bytes(nkv, H)))

    def gu():
        for l in ws.layers:
            ctx.call("ti_gateup_silu_q4", a["xq"], a["xs"], *l["gate"], *l["up"], a["swi"], I, H)
    timed("gateup_q4_q8", gu, len(ws.layers), gateup_bytes(I, H) * len(ws.layers))

    def lm():
        for w in lm_copies:
            ctx.call("ti_gemv_q4_f32", a["last"], *w, a["logits"], cfg["vocab"], H, 0)
    timed("gemv_q4_f32", lm, len(lm_copies), gemv_f32_bytes(cfg["vocab"], H) * len(lm_copies))
    return fams


def cpu_baseline(cfg, budget_s=12.0):
    """The oracle's int4 GEMV (a C port of the reference arithmetic, 1 thread) on a
    bounded sample of the same GEMV set: layer-shaped GEMVs then the lm_head."""
    from oracle import oracle as orc
    rng = np.random.default_rng(5)
    H, I = cfg["hidden"], cfg["inter"]
    nq = cfg["n_heads"] * cfg["head_dim"]
    nkv = cfg["n_kv"] * cfg["head_dim"]
    shapes = [(nq, H), (nkv, H), (nkv, H), (H, nq), (I, H), (I, H), (H, I)]
    mats = [(rng.integers(0, 2 ** 32, N * K // 8, dtype=np.uint64).astype(np.uint32),
             rng.uniform(1e-3, 1e-2, N * K // 32).astype(np.float16).view(np.uint16), N, K) for N, K in shapes]
    x = rng.standard_normal(max(H, I, nq)).astype(np.float32)
    nbytes, t0, layers = 0, time.perf_counter(), 0
    while time.perf_counter() - t0 < budget_s * 0.5:
        for pack, sc, N, K in mats:
            xq, xs, _ = orc.quant_act_q8(x[:K])
            orc.gemv_q4_q8(xq, xs, pack, sc, N, K)
            nbytes += gemv_q8_bytes(N, K)
        layers += 1
    # lm_head rows, f32 activation path
    N = 16384
    pack = rng.integers(0, 2 ** 32, N * H // 8, dtype=np.uint64).astype(np.uint32)
    sc = rng.uniform(1e-3, 1e-2, N * H // 32).astype(np.float16).view(np.uint16)
    lm_rows = 0
    while time.perf_counter() - t0 < budget_s:
        orc.gemv_q4_f32(x[:H], pack, sc, N, H)
        nbytes += gemv_f32_bytes(N, H)
        lm_rows += N
    dt = time.perf_counter() - t0
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": "oracle int4 GEMV (C, 1 thread): %d Qwen3-0.6B layer GEMV sets + %d lm_head rows (K=1024), %.1f s"
                      % (layers, lm_rows, dt)}


def tern_avx2_baseline(budget_s=6.0):
    """The reference's native CPU path, n2 avx2::gemv_tern (restated in C), on the
    Bonsai-1.7B ternary GEMV shapes of one layer (q, k, v, o, gate, up, down),
    min over repetitions; 1 thread (the reference's configuration) and N threads."""
    from oracle import oracle as orc
    if not orc.has_avx2():
        return None
    shapes = [(2048, 2048), (1024, 2048), (1024, 2048), (2048, 2048), (6144, 2048), (6144, 2048), (2048, 6144)]
    rng = np.random.default_rng(3)
    per_layer = sum(N * K // 4 + (N * K // 64) * 4 + K + (K // 64) * 4 + N * 4 for N, K in shapes)
    mats = [(rng.integers(0, 3, N * K // 4, dtype=np.uint8) * np.uint8(0x55),
             rng.uniform(0.01, 0.05, N * K // 64).astype(np.float16).astype(np.float32), N, K) for N, K in shapes]
    acts = {K: orc.tern_quant_act_n2(rng.standard_normal(K).astype(np.float32)) for K in (2048, 6144)}
    outs = {N: np.zeros(N, np.float32) for N in (1024, 2048, 6144)}
    res = {}
    ncpu = len(os.sched_getaffinity(0))
    for threads in sorted({1, max(1, min(16, ncpu))}):
        best = None
        t_end = time.perf_counter() + budget_s / 2
        while time.perf_counter() < t_end:
            t0 = time.perf_counter()
            for c_, s_, N, K in mats:
                a_, xs_, _ = acts[K]
                orc.tern_gemv_avx2_into(c_, s_, a_, xs_, N, K, outs[N], threads)
            dt = time.perf_counter() - t0
            best = dt if best is None or dt < best else best
        macs = sum(N * K for N, K in shapes)
        res["threads_%d" % threads] = {"GB_s": round(per_layer / best / 1e9, 2), "GMAC_s": round(macs / best / 1e9, 2)}
    return {"kind": "port", "what": "n2 avx2::gemv_tern restated in C (oracle/tern_avx2.c), Bonsai-1.7B layer GEMV shapes, min over reps",
            **res}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py runs on one GPU only: this build measures one MI355X's share of the work "
              "(see DESIGN.md for how the path would shard); --gpus %d is not supported" % args.gpus, file=sys.stderr)
        sys.exit(2)

    from tabinfer_amd import abi
    ctx = abi.Ctx(0)
    cfg = QWEN3_06B
    print("[bench] building weights (2 sets x %.0f MB)" % ((Step(ctx, cfg, None).bytes) / 1e6), file=sys.stderr, flush=True)
    pool = make_pool(ctx, 48 << 20, 1234)
    sets = [GemvSet(ctx, cfg, 100 + i, pool) for i in range(2)]
    act = make_acts(ctx, cfg, 7)
    step = Step(ctx, cfg, act)
    ctx.sync()
    graphs = []
    for ws in sets:
        ctx.graph_begin()
        step.issue(ws)
        graphs.append(ctx.graph_end())
    for i in range(args.warmup):
        ctx.graph_launch(graphs[i % 2])
    ctx.sync()
    print("[bench] timing %d steps" % args.steps, file=sys.stderr, flush=True)
    ctx.record(10)
    for i in range(args.steps):
        ctx.graph_launch(graphs[i % 2])
    ctx.record(11)
    ctx.sync()
    ms = ctx.elapsed_ms(10, 11)
    ms_per_step = ms / args.steps
    value = step.bytes / (ms_per_step * 1e-3) / 1e9

    lm_extra = [sets[0]._quantized(cfg["vocab"], cfg["hidden"], np.random.default_rng(77 + i), pool) for i in range(2)]
    last = (args.steps - 1) % 2
    fams = kernel_profile(ctx, step, sets[1 - last], [sets[0].lm, sets[1].lm] + lm_extra)
    dom_name = max(fams, key=lambda k: fams[k]["avg_us"] * fams[k]["launches"])
    dom = fams[dom_name]
    achieved = dom["bytes_per_launch"] / (dom["avg_us"] * 1e-6) / 1e9
    traffic = None
    tp = os.path.join(ROOT, "profiles", "traffic_%s.json" % dom_name)
    if os.path.exists(tp):
        traffic = json.load(open(tp)).get("hbm_bytes_per_launch")
    out = {
        "metric": "int4 GEMV HBM GB/s (% of peak) + Qwen3-1.7B bs1 decode tok/s at 32k ctx",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int4xint8", "data": "synthetic (seeded bf16 N(0,0.02) weights, GPU-quantized; N(0,1) f16 activations)",
        "config": {"workload": "Qwen3-0.6B int4 GEMV set of one batch-1 decode step (28 layers q/k/v/o/gate+up/down + lm_head 151936x1024), graph-launched",
                   "bytes_per_step": step.bytes, "launches_per_step": step.launches, "weight_sets": 2,
                   "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2)},
        "roofline": {"bound": "hbm", "kernel": dom_name, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic},
        "kernels": {k: {kk: round(vv, 3) for kk, vv in v.items()} for k, v in fams.items()},
    }
    if not args.no_cpu:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(cfg)
        tb = tern_avx2_baseline()
        if tb:
            out["cpu_tern_avx2"] = tb
    for g in graphs:
        ctx.graph_destroy(g)
    ctx.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
