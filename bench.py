"""Benchmark of the EXL3 quantized matmul path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S]

Workload (the configuration its metric "EXL3 GEMV
HBM GB/s at bs=1" is quoted on): a decode pass at batch 1 over the linears of
a 36-layer Qwen3-8B-shaped decoder (per layer q/o 4096->4096, k/v
4096->1024, gate/up 4096->12288, down 12288->4096), EXL3 K=4 mul1 weights,
uniform-random trellis words, suh +-1, svh f16(+-U[0.5,1.5]*0.02), f16
N(0,1) activations.  One step = every linear once (one kernel per launch: prepare + decode GEMV +
finish), the linears that read the same rows in one launch as a decoder layer
issues them (q+k+v, o, gate+up, down: exl3_matmul_shared; --per-linear: one
launch each), 252 linears, 3.47 GB of distinct packed weights (beyond the
256 MB Infinity Cache, so every step reads HBM).  The step is captured once into a
HIP graph and replayed.

`value` = packed-weight bytes per step * steps / timed seconds (GB/s).
`roofline` = the dominant kernel (the K=4 decode GEMV, which is the whole
matmul: prepare, GEMV and finish in one launch): algorithmic bytes per launch
(in*out*K/8 summed over the launch's linears) / average launch duration, the
duration from HIP events around the timed region's graph replays (the
launches run back to back) divided by the launches, against the 8 TB/s HBM
peak; the rocprof kernel trace of the same command agrees
(profiles/gemv_k4_qwen3_8b_decode.md).  `cpu_baseline` = the CPU oracle's projection
(prepare + decode + f32 dot + finish, the reference's CPU path restated in
C, oracle/exl3_oracle.c) on the host cores over a bounded sample of the same
linears.  `extra` carries the prefill GEMM (M=2048, K=4) TFLOP/s.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "EXL3 GEMV HBM GB/s (% of peak) at bs=1; prefill GEMM TFLOPS; decode tok/s"
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
LAYERS = 36
SHAPES = [("q", 4096, 4096), ("k", 4096, 1024), ("v", 4096, 1024), ("o", 4096, 4096),
          ("gate", 4096, 12288), ("up", 4096, 12288), ("down", 12288, 4096)]
K_BITS = 4


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_model(torch, X, layers: int, seed: int, k_bits: int = K_BITS):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    lins = []
    n = 16 * k_bits
    for _ in range(layers):
        for name, i, o in SHAPES:
            t = torch.randint(-32768, 32768, (i // 16, o // 16, n), dtype=torch.int32, device="cuda",
                              generator=g).to(torch.int16)
            suh = (torch.randint(0, 2, (i,), device="cuda", generator=g) * 2 - 1).to(torch.float16)
            sgn = torch.randint(0, 2, (o,), device="cuda", generator=g) * 2 - 1
            mag = torch.rand(o, device="cuda", generator=g) + 0.5
            svh = (sgn * mag * 0.02).to(torch.float16)
            lins.append((name, i, o, X.Linear(t, suh, svh)))
    return lins


def packed_bytes(i: int, o: int) -> int:
    return i * o * K_BITS // 8


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_ms(torch, fn, reps: int = 20) -> float:
    """Median over `reps` runs of fn, each between two HIP events.  The runs
    are queued behind a ~3 ms spin kernel, so they run back to back on the
    GPU as a serving loop issues them, and the host's launch time (ctypes,
    three launches per prefill call) does not enter the GPU's timeline."""
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    torch.cuda.synchronize()
    torch.cuda._sleep(int(7e6))
    evs[0].record()
    for i in range(reps):
        fn()
        evs[i + 1].record()
    torch.cuda.synchronize()
    ts = sorted(evs[i].elapsed_time(evs[i + 1]) for i in range(reps))
    return ts[len(ts) // 2]


# Distinct bytes a rotating working set should reach, so that each pass reads
# HBM rather than the 256 MB Infinity Cache (MALL).
ROTATE_BYTES = 512 << 20


def cpu_baseline(seconds: float):
    from oracle import oracle as O
    rng = np.random.default_rng(7)
    n = 16 * K_BITS
    todo = []
    for name, i, o in SHAPES:
        t = rng.integers(0, 65536, (i // 16, o // 16, n), dtype=np.uint16)
        suh = np.where(rng.random(i) < 0.5, -1.0, 1.0).astype(np.float16).view(np.uint16)
        svh = (np.where(rng.random(o) < 0.5, -1.0, 1.0) * rng.uniform(0.5, 1.5, o) * 0.02
               ).astype(np.float16).view(np.uint16)
        x = rng.standard_normal((1, i)).astype(np.float32)
        todo.append((i, o, t, suh, svh, x))
    done_bytes = 0
    linears = 0
    t0 = time.perf_counter()
    while True:
        for i, o, t, suh, svh, x in todo:
            O.project(x, t, suh, svh, i, o, n)
            done_bytes += packed_bytes(i, o)
            linears += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(done_bytes / el / 1e9, 3), "unit": "GB/s", "cores": O.threads(),
            "cpu_model": _cpu_model(), "kind": "port",
            "sample": f"{linears} batch-1 K=4 projections cycling one Qwen3-8B layer's 7 linears "
                      f"(q,k,v,o,gate,up,down; {sum(packed_bytes(i, o) for _, i, o in SHAPES) / 1e6:.1f} MB "
                      f"packed), {el:.1f} s, oracle/exl3_oracle.c exl3o_project"}


def gemm_tflops(torch, iters: int = 10):
    """Prefill GEMM M=2048 at K=4 on the gate/up shape (4096 -> 12288)."""
    from plugins_amd import exl3 as X
    rows, i, o = 2048, 4096, 12288
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    lins = []
    copies = -(-ROTATE_BYTES // packed_bytes(i, o))  # rotate >= 512 MB of weights
    for _ in range(copies):
        t = torch.randint(-32768, 32768, (i // 16, o // 16, 64), dtype=torch.int32, device="cuda",
                          generator=g).to(torch.int16)
        suh = torch.ones(i, dtype=torch.float16, device="cuda")
        svh = torch.full((o,), 0.02, dtype=torch.float16, device="cuda")
        lins.append(X.Linear(t, suh, svh))
    x = torch.randn(rows, i, device="cuda", generator=g).to(torch.float16)
    y = torch.empty(rows, o, dtype=torch.float16, device="cuda")
    for lin in lins:
        lin(x, out=y)
    torch.cuda.synchronize()
    turn = [0]

    def one():
        lins[turn[0] % copies](x, out=y)
        turn[0] += 1
    ms = _median_ms(torch, one, max(20, iters))
    tf = 2.0 * rows * i * o / (ms * 1e-3) / 1e12
    # context: a dense f16 GEMM of the same shape through torch (hipBLASLt),
    # the library's rate on unquantized weights (6 x 100 MB rotated)
    del lins
    ws = [torch.randn(i, o, device="cuda", generator=g).to(torch.float16) for _ in range(6)]
    for w in ws:
        torch.matmul(x, w, out=y)
    torch.cuda.synchronize()
    turn[0] = 0

    def dense():
        torch.matmul(x, ws[turn[0] % len(ws)], out=y)
        turn[0] += 1
    dms = _median_ms(torch, dense, max(20, iters))
    dtf = 2.0 * rows * i * o / (dms * 1e-3) / 1e12
    return {"prefill_gemm_m2048_gate_up_k4": {"tflops": round(tf, 2), "ms": round(ms, 4),
                                              "timing": f"median of 20 back-to-back launches, {copies} weight copies "
                                                        f"({copies * packed_bytes(i, o) >> 20} MiB) rotated",
                                              "frac_of_fp16_peak": round(tf / FP16_PEAK_TFLOPS, 4),
                                              "includes": "prepare + LDS-decode MFMA GEMM + finish",
                                              "dense_f16_torch_same_shape_tflops": round(dtf, 1)}}


def _graph_ms(torch, fn, reps: int = 20) -> float:
    """Captures fn (after two eager calls on the capture stream) into a HIP
    graph and returns the median replay time in ms over max(reps, 20)
    replays, each between its own HIP events."""
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        fn()
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap, capture_error_mode="thread_local"):
        fn()
    g.replay()
    torch.cuda.synchronize()
    return _median_ms(torch, g.replay, max(reps, 20))


def gemv_cache_resident(torch, X, distinct: int = 2):
    """The headline pass (36 layers of launches, batch 1, K=4) with the
    weights of `distinct` layers reused (layer l uses layer l % distinct):
    at 2 layers 193 MB, inside the 256 MB Infinity Cache, so the pass reads
    no weights from HBM after the first replay.  Set beside the streamed
    pass it shows how much of the launch time HBM bandwidth accounts for."""
    lins_d = build_model(torch, X, distinct, seed=1234)
    per = len(SHAPES)
    lins = [lins_d[(l % distinct) * per + j] for l in range(LAYERS) for j in range(per)]
    nbytes = sum(packed_bytes(i, o) for _, i, o, _ in lins)
    xs = {i: torch.randn(1, i, device="cuda").to(torch.float16) for i in (4096, 12288)}
    ys = [torch.empty(1, o, dtype=torch.float16, device="cuda") for _, _, o, _ in lins]
    groups = []
    for l0 in range(0, len(lins), per):
        groups += [[l0, l0 + 1, l0 + 2], [l0 + 3], [l0 + 4, l0 + 5], [l0 + 6]]

    def step():
        for g in groups:
            i = lins[g[0]][1]
            X.matmul_shared([lins[j][3].weight for j in g], xs[i], outs=[ys[j] for j in g])
    ms = _graph_ms(torch, step, 20)
    return {"gemv_pass_cache_resident": {
        "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1), "ms_per_step": round(ms, 4),
        "us_per_launch": round(ms * 1e3 / len(groups), 3),
        "distinct_mb": round(sum(packed_bytes(i, o) for _, i, o, _ in lins_d) / 1e6, 1),
        "timing": "median of 20 graph replays"}}


def gemv_sweep(torch, X, ks=(2, 3, 4, 5, 6, 8), batches=(1, 2, 4, 8), reps=20):
    """the decode GEMV over the Qwen3-8B-shaped linears at
    each rate K and batch (as many layers as make >= 512 MB of weights at
    that rate, launches grouped as a decoder issues them, HIP graph, median
    of 20 replays): packed GB/s."""
    out = {}
    per_layer = sum(i * o for _, i, o in SHAPES)
    for k in ks:
        layers = -(-ROTATE_BYTES // (per_layer * k // 8))
        lins = build_model(torch, X, layers, seed=100 + k, k_bits=k)
        nbytes = sum(i * o * k // 8 for _, i, o, _ in lins)
        per = len(SHAPES)
        groups = []
        for l0 in range(0, len(lins), per):
            groups += [[l0, l0 + 1, l0 + 2], [l0 + 3], [l0 + 4, l0 + 5], [l0 + 6]]
        res = {}
        for B in batches:
            xs = {i: torch.randn(B, i, device="cuda").to(torch.float16) for i in (4096, 12288)}
            ys = [torch.empty(B, o, dtype=torch.float16, device="cuda") for _, _, o, _ in lins]

            def step():
                for g in groups:
                    i = lins[g[0]][1]
                    X.matmul_shared([lins[j][3].weight for j in g], xs[i], outs=[ys[j] for j in g])
            ms = _graph_ms(torch, step, reps)
            res[f"batch{B}"] = {"gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                "us_per_launch": round(ms * 1e3 / len(groups), 2)}
        res["layers"] = layers
        res["distinct_mb"] = round(nbytes / 1e6, 1)
        out[f"K{k}"] = res
        del lins
        torch.cuda.empty_cache()
    return {"gemv_sweep": {"packed_bytes": "in*out*K/8", "timing": "median of 20 graph replays",
                           **out}}


def gemm_sweep(torch, X, ms=(128, 512, 2048, 4096), iters=8):
    """the prefill GEMM at K=4 on each Qwen3-8B layer shape
    and M (prepare + GEMM + finish; 3 weight copies rotated): TFLOP/s."""
    g = torch.Generator(device="cuda")
    g.manual_seed(12)
    shapes = [("q/o", 4096, 4096), ("k/v", 4096, 1024), ("gate/up", 4096, 12288),
              ("down", 12288, 4096)]
    out = {}
    for name, i, o in shapes:
        lins = []
        copies = -(-ROTATE_BYTES // packed_bytes(i, o))
        for _ in range(copies):
            t = torch.randint(-32768, 32768, (i // 16, o // 16, 64), dtype=torch.int32,
                              device="cuda", generator=g).to(torch.int16)
            lins.append(X.Linear(t, torch.ones(i, dtype=torch.float16, device="cuda"),
                                 torch.full((o,), 0.02, dtype=torch.float16, device="cuda")))
        res = {}
        for M in ms:
            x = torch.randn(M, i, device="cuda", generator=g).to(torch.float16)
            y = torch.empty(M, o, dtype=torch.float16, device="cuda")
            for lin in lins:
                lin(x, out=y)
            torch.cuda.synchronize()
            turn = [0]

            def one():
                lins[turn[0] % copies](x, out=y)
                turn[0] += 1
            t_ms = _median_ms(torch, one, max(20, iters))
            res[f"M{M}"] = {"tflops": round(2.0 * M * i * o / (t_ms * 1e-3) / 1e12, 1),
                            "us": round(t_ms * 1e3, 1)}
        res["weight_copies"] = copies
        out[name] = res
        del lins
        torch.cuda.empty_cache()
    return {"gemm_sweep_k4": {"timing": "median of 20 back-to-back launches, >= 512 MB of weights rotated", **out}}


def moe_bench(torch, X, batches=(1, 16, 64), routings=8, reps=20):
    """a DeepSeek-V3-style routed MoE layer at K=3 (hidden
    7168, expert intermediate 2048, 256 routed experts top-8 from the softmax
    of N(0,1) logits, renormalized, plus one shared expert).  One graph
    replay runs the layer `routings` times, each call with its own routing,
    so a replay reads the union of their experts (at batch 1 about 8 x 8
    experts, ~1.1 GB, beyond the 256 MB MALL): the routed swiglu and the
    shared expert's dense swiglu per call.  Packed bytes per replay = (the
    union of the routed experts the replay's calls read + 1 shared) * 3 *
    7168 * 2048 * 3/8 (distinct bytes, each counted once; `gbs_per_call_sum`
    counts each call's own distinct experts + the shared one, the bytes the
    calls ask for, some of which an earlier call left in L2/MALL); median of
    20 replays.  `swiglu_shared`: the same calls with the shared expert gated
    (sigmoid(logit)) inside the routed launches (QuantTable.swiglu_shared)."""
    E, H, I, K, topk = 256, 7168, 2048, 3, 8
    n = 16 * K
    g = torch.Generator(device="cuda")
    g.manual_seed(13)

    def bank(e, i, o):
        t = torch.randint(-32768, 32768, (e, i // 16, o // 16, n), dtype=torch.int32, device="cuda",
                          generator=g).to(torch.int16)
        suh = (torch.randint(0, 2, (e, i), device="cuda", generator=g) * 2 - 1).to(torch.float16)
        svh = ((torch.randint(0, 2, (e, o), device="cuda", generator=g) * 2 - 1) *
               (torch.rand(e, o, device="cuda", generator=g) + 0.5) * 0.02).to(torch.float16)
        return t, suh, svh

    gb, ub, db = bank(E, H, I), bank(E, H, I), bank(E, I, H)
    G, U, D = X.wrap(*gb), X.wrap(*ub), X.wrap(*db)
    sg, su, sd = (X.Linear(*[a[0] for a in bank(1, H, I)]), X.Linear(*[a[0] for a in bank(1, H, I)]),
                  X.Linear(*[a[0] for a in bank(1, I, H)]))
    per_expert = 3 * H * I * K // 8
    out = {}
    for B in batches:
        x = torch.randn(B, 1, H, device="cuda", generator=g).to(torch.float16)
        calls, union, per_call = [], set(), 0
        for _ in range(routings):
            probs = torch.softmax(torch.randn(B, E, device="cuda", generator=g), -1)
            top = probs.topk(topk, -1)
            scores = (top.values / top.values.sum(-1, keepdim=True)).reshape(B, 1, topk)
            inds = top.indices.to(torch.int32).reshape(B, 1, topk)
            distinct = torch.unique(inds).tolist()
            union.update(distinct)
            per_call += (len(distinct) + 1) * per_expert
            calls.append((inds, scores))
        y = torch.empty_like(x)
        ys = torch.empty_like(x)
        logit = torch.randn(B, device="cuda", generator=g).to(torch.float16)

        def layer():
            for inds, scores in calls:
                X.swiglu(G, U, D, x, inds, scores, out=y)
                X.swiglu(sg.weight, su.weight, sd.weight, x, out=ys)

        def layer_shared():
            for inds, scores in calls:
                X.swiglu_shared(G, U, D, x, [sg.weight, su.weight, sd.weight], inds=inds,
                                scores=scores, logit=logit, out=y)
        nbytes = (len(union) + 1) * per_expert
        ms = _graph_ms(torch, layer, reps)
        res = {"gbs": round(nbytes / (ms * 1e-3) / 1e9, 1), "us_per_call": round(ms * 1e3 / routings, 1),
               "gbs_per_call_sum": round(per_call / (ms * 1e-3) / 1e9, 1),
               "distinct_experts_per_replay": len(union), "distinct_mb": round(nbytes / 1e6, 1)}
        try:
            ms2 = _graph_ms(torch, layer_shared, reps)
            res["swiglu_shared"] = {"gbs": round(nbytes / (ms2 * 1e-3) / 1e9, 1),
                                    "gbs_per_call_sum": round(per_call / (ms2 * 1e-3) / 1e9, 1),
                                    "us_per_call": round(ms2 * 1e3 / routings, 1)}
        except Exception as ex:  # reported, not hidden (e.g. refused at prefill sizes)
            res["swiglu_shared"] = {"refused": str(ex)}
        out[f"batch{B}"] = res
    for w in (G, U, D):
        X.release(w)
    return {"moe_k3_deepseek_v3_layer": {"routings_per_replay": routings,
                                         "timing": "median of 20 graph replays", **out}}


def decode_tok_s(torch, batches=(1, 16), ctx=2048, steps=8):
    """a 36-layer Qwen3-8B-shaped decoder decode step (EXL3
    K=4 linears incl. lm_head, f16 attention over a random KV cache at context
    `ctx`), captured in a HIP graph; tokens per second per batch size."""
    from plugins_amd import qwen3 as Q
    res = {}
    for B in batches:
        m = Q.Qwen3Decoder(Q.Qwen3Config(), B, ctx, seed=21)
        cap = torch.cuda.Stream()
        cap.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(cap):
            m.step(stream=cap)
            m.step(stream=cap)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap, capture_error_mode="thread_local"):
            m.step(stream=cap)
        g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            g.replay()
        torch.cuda.synchronize()
        el = (time.perf_counter() - t0) / steps
        wb, kvb = m.weight_bytes(), m.kv_bytes()
        res[f"batch{B}"] = {"tok_s": round(B / el, 1), "ms_per_step": round(el * 1e3, 3),
                            "weight_bytes": wb, "kv_bytes": kvb,
                            "gbs": round((wb + kvb) / el / 1e9, 1)}
        del g, m
        torch.cuda.empty_cache()
    res["config"] = ("36 layers, hidden 4096, 32/8 heads x 128, SwiGLU 12288, vocab 151936, EXL3 K=4 "
                     f"mul1 (lm_head too), f16 KV cache at context {ctx}, HIP graph per step")
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="skip the decoder tok/s leg")
    ap.add_argument("--no-sweep", action="store_true",
                    help="skip the config 1-3 legs (GEMV K x batch sweep, GEMM M sweep, MoE layer)")
    ap.add_argument("--only", choices=["gemv", "gemm", "decode", "sweep", "moe"], default=None,
                    help="run one leg (gemv: the decode GEMV pass and its roofline leg only)")
    ap.add_argument("--per-linear", action="store_true",
                    help="one launch per linear instead of one per shared-input group")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="only copy a buffer of this many MiB 5 times (calibrates HBM byte counters)")
    args = ap.parse_args()
    if args.copy_mib:
        import torch
        src = torch.ones(args.copy_mib << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_mib": args.copy_mib, "copies": 5}))
        return 0
    if args.only in ("gemm", "decode", "sweep", "moe"):
        # one leg alone (for counter runs of its kernels); prints that leg's numbers
        import torch
        from plugins_amd import exl3 as X
        torch.cuda.set_device(0)
        if args.only == "gemm":
            res = gemm_tflops(torch)
        elif args.only == "decode":
            res = decode_tok_s(torch)
        elif args.only == "moe":
            res = moe_bench(torch, X)
        else:
            res = {**gemv_sweep(torch, X), **gemm_sweep(torch, X), **moe_bench(torch, X)}
        print(json.dumps({"only": args.only, **res}), flush=True)
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the EXL3 path has no multi-GPU leg); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import torch
    from plugins_amd import exl3 as X
    torch.cuda.set_device(0)
    log("building model:", args.layers, "layers")
    lins = build_model(torch, X, args.layers, seed=1234)
    step_bytes = sum(packed_bytes(i, o) for _, i, o, _ in lins)
    xs = {i: torch.randn(1, i, device="cuda").to(torch.float16) for i in (4096, 12288)}
    ys = [torch.empty(1, o, dtype=torch.float16, device="cuda") for _, _, o, _ in lins]
    # launches of one step: the linears that read the same rows go together
    # (q,k,v and gate,up), as a decoder layer issues them
    groups = []
    if args.per_linear:
        groups = [[j] for j in range(len(lins))]
    else:
        per = len(SHAPES)
        for l0 in range(0, len(lins), per):
            groups += [[l0, l0 + 1, l0 + 2], [l0 + 3], [l0 + 4, l0 + 5], [l0 + 6]]

    def launch(g):
        if len(g) == 1:
            name, i, o, lin = lins[g[0]]
            lin(xs[i], out=ys[g[0]])
        else:
            i = lins[g[0]][1]
            X.matmul_shared([lins[j][3].weight for j in g], xs[i], outs=[ys[j] for j in g])

    def step():
        for g in groups:
            launch(g)

    # Warm up on the stream the graph is captured on: the library keeps its
    # scratch per stream and sizes it at the first call, outside the capture.
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        for _ in range(args.warmup):
            step()
    torch.cuda.synchronize()
    run = step
    graph = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=cap, capture_error_mode="thread_local"):
            step()
        for _ in range(2):
            graph.replay()
        torch.cuda.synchronize()
        run = graph.replay
    log("timing", args.steps, "steps")
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        run()
    ev1.record()
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    ms_per_step = el * 1e3 / args.steps
    value = step_bytes * args.steps / el / 1e9
    # GPU time of the timed region (HIP events on the stream the graph is
    # launched on): the launches run back to back, so a launch's average
    # duration is the region's time over the launches it holds
    gpu_ms_per_step = ev0.elapsed_time(ev1) / args.steps

    # per-shape diagnostic: the matmul of each linear is one kernel launch
    # (prepare, decode GEMV and finish fused); HIP event pairs around each
    # launch, every linear of the model once per pass, 3 passes (the pairs
    # add their own ~2 us per launch; the roofline uses the timed region).  A
    # sleep kernel first lets the host queue every launch ahead of the GPU.
    log("per-shape leg")
    step()  # the library sizes its scratch for this stream on first use
    torch.cuda.synchronize()
    pairs = []
    torch.cuda._sleep(int(2.4e9 * 0.1))
    for _ in range(3):
        for g in groups:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            launch(g)
            b.record()
            name = "+".join(lins[j][0] for j in g)
            pairs.append((name, sum(packed_bytes(lins[j][1], lins[j][2]) for j in g), a, b))
    torch.cuda.synchronize()
    launches = len(groups)
    avg_launch_ms = gpu_ms_per_step / launches
    achieved = step_bytes / launches / (avg_launch_ms * 1e-3) / 1e9
    per_shape = {}
    for name, nb, a, b in pairs:
        d = per_shape.setdefault(name, [0, 0.0, 0])
        d[0] += nb
        d[1] += a.elapsed_time(b)
        d[2] += 1
    shapes = {k: {"gbs": round(v[0] / (v[1] * 1e-3) / 1e9, 1), "us": round(v[1] * 1e3 / v[2], 2)}
              for k, v in per_shape.items()}

    extra = {}
    if args.only != "gemv":
        try:
            extra.update(gemm_tflops(torch))
        except Exception as ex:  # reported, not hidden
            extra["prefill_gemm_error"] = repr(ex)
    extra["gemv_gbs_per_shape"] = shapes
    try:
        log("cache-resident pass")
        extra.update(gemv_cache_resident(torch, X))
    except Exception as ex:  # reported, not hidden
        extra["gemv_cache_resident_error"] = repr(ex)
    if not args.no_decode and args.only != "gemv":
        try:
            log("decode step")
            extra["decode_tok_s"] = decode_tok_s(torch)
        except Exception as ex:  # reported, not hidden
            extra["decode_error"] = repr(ex)
    if not args.no_sweep and args.only != "gemv":
        for name, leg in (("gemv sweep", gemv_sweep), ("gemm sweep", gemm_sweep), ("moe", moe_bench)):
            try:
                log(name)
                extra.update(leg(torch, X))
            except Exception as ex:  # reported, not hidden
                extra[name.replace(" ", "_") + "_error"] = repr(ex)
    extra["graph"] = graph is not None

    cpu = None
    if not args.no_cpu and args.only != "gemv":
        log("cpu baseline")
        cpu = cpu_baseline(args.cpu_seconds)

    # the median of 20 single-step replays (each between its own HIP events)
    median_launch_us = None
    if graph is not None:
        median_launch_us = round(_median_ms(torch, graph.replay, 20) * 1e3 / launches, 3)

    # HBM traffic per launch of this workload, measured by the FETCH_SIZE /
    # WRITE_SIZE counter runs of profiles/gemv_k4_qwen3_8b_decode.md (each
    # scaled by its plain-copy calibration); null when that file is absent.
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "gemv_k4_qwen3_8b_decode.json")
    valu_ceiling = None
    if args.layers == LAYERS and not args.per_linear and os.path.exists(tpath):
        prof = json.load(open(tpath))
        traffic = prof.get("traffic_bytes_per_launch")
        # The VALU ceiling: the GB/s at which the pass's measured VALU
        # instructions (SQ_INSTS_VALU of the counter run, decode and every
        # fixed part included) would keep every SIMD's VALU busy: 1024 SIMDs
        # at the held shader clock, VALU_CYCLES per wave-instruction, plus
        # the measured extra cycles of the decode's one v_mul_lo_u32 per
        # weight (timed against v_xor_b32 in the same dependent-chain loop by
        # a standalone probe; SQ_INSTS_VALU counts it as one).
        vi = prof.get("valu_wave_insts_per_step")
        if vi:
            muls = step_bytes * 8 / K_BITS / 64
            cycles = vi * prof["valu_cycles_per_inst"] + muls * prof.get("mul_lo_extra_cycles", 0.0)
            secs = cycles / (256 * 4 * prof["shader_clock_hz"])
            valu_ceiling = {"gbs": round(step_bytes / secs / 1e9, 1),
                            "frac_of_hbm_peak": round(step_bytes / secs / 1e9 / HBM_PEAK_GBS, 3),
                            "valu_insts_per_weight": round(vi * 64 / (step_bytes * 8 / K_BITS), 2),
                            "basis": "SQ_INSTS_VALU per step (profiles/gemv_k4_qwen3_8b_decode.md) at "
                                     f"{prof['valu_cycles_per_inst']} cycles per wave-instruction, "
                                     f"+{prof.get('mul_lo_extra_cycles', 0.0)} cycles per v_mul_lo_u32 "
                                     "(one per weight, timed by a standalone instruction-rate probe), "
                                     f"{prof['shader_clock_hz'] / 1e9:.2f} GHz, 1024 SIMDs"}

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": f"decode GEMV pass, batch 1, EXL3 K={K_BITS} mul1, "
                               f"{args.layers}-layer Qwen3-8B-shaped linears (q,k,v,o,gate,up,down)",
                   "layers": args.layers, "batch": 1, "K": K_BITS, "packed_bytes_per_step": step_bytes,
                   "linears_per_step": len(lins), "launches_per_step": len(groups),
                   "launch_groups": "per linear" if args.per_linear else "q+k+v, o, gate+up, down"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_unit": "bytes per launch (profiles/gemv_k4_qwen3_8b_decode.md)",
                     "algorithmic_bytes_per_launch": round(step_bytes / launches),
                     "kernel": "exl3::gemv_kernel<4,0,false,0,0> (mul1, K=4, window 16, one prepare batch, plain input)",
                     "median_launch_us": median_launch_us,
                     "valu_ceiling": valu_ceiling,
                     "launches": launches * args.steps,
                     "avg_launch_us": round(avg_launch_ms * 1e3, 3),
                     "timing": "HIP events around the timed region's graph replays / launches"},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
