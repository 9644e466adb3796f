"""Phase timeline of the decode GEMV launches (a diagnostic, not the product
path): loads the timeline build (`python -m plugins_amd.build --timeline`,
lib/libexl3_mi355x_timeline.so, whose K=4 GEMV kernels stamp each wave's
phases with the 100 MHz real-time counter) and prints, per launch type of a
batch-1 Qwen3-8B-shaped pass, the distribution over waves (min, p10, median,
p90, max; microseconds from the launch's first wave) of:

  entry, prepared (rows prepared, after the workgroup barrier), loop done,
  loop duration, reduced (before the split-K hand-off), partial stored (the
  other splits' exit), stores acknowledged (theirs, after a wait the product
  build does not make), first read returned (the last split's first read of
  the slots), hand-off done and finish done (the last split's);

and for gate+up the medians per dispatch round (workgroup id // 256: the
first, second and third workgroup each CU holds).

    python -m plugins_amd.timeline [--lib PATH] [--batch N]

--lib: another timeline build of the library (the default is the one
`python -m plugins_amd.build --timeline` writes); --batch: rows of the
activations (default 1; 16 is config 4's batch).
"""
from __future__ import annotations

import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
WGS = 4096
EVENTS = ("entry", "prepared", "loop done", "reduced", "partial stored", "hand-off done",
          "finish done")


def main() -> int:
    import torch
    sys.path.insert(0, ROOT)
    from plugins_amd import build as B
    from plugins_amd import exl3 as X
    lib = B.TIMELINE_LIB
    if "--lib" in sys.argv:
        lib = sys.argv[sys.argv.index("--lib") + 1]
    if not os.path.exists(lib):
        print("build it first: python -m plugins_amd.build --timeline", file=sys.stderr)
        return 2
    X.LIB_PATH = lib
    L = X.lib()
    L.exl3_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    L.exl3_timeline_clear.argtypes = []
    import bench
    rows = int(sys.argv[sys.argv.index("--batch") + 1]) if "--batch" in sys.argv else 1
    lins = bench.build_model(torch, X, 36, seed=1234, k_bits=4)
    xs = {i: torch.randn(rows, i, device="cuda").to(torch.float16) for i in (4096, 12288)}
    ys = [torch.empty(rows, o, dtype=torch.float16, device="cuda") for _, _, o, _ in lins]
    kinds = {"q+k+v": [0, 1, 2], "o": [3], "gate+up": [4, 5], "down": [6]}

    def launch(g):
        if len(g) == 1:
            lins[g[0]][3](xs[lins[g[0]][1]], out=ys[g[0]])
        else:
            X.matmul_shared([lins[j][3].weight for j in g], xs[lins[g[0]][1]], outs=[ys[j] for j in g])

    for layer in range(36):  # scratch sized, code and weights touched once
        for idx in kinds.values():
            launch([layer * 7 + j for j in idx])
    torch.cuda.synchronize()

    def pct(v):
        v = v[~np.isnan(v)]
        if v.size == 0:
            return "     -"
        return " ".join(f"{float(np.percentile(v, p)):7.2f}" for p in (0, 10, 50, 90, 100))

    print(f"{'':24s} {'min':>7s} {'p10':>7s} {'p50':>7s} {'p90':>7s} {'max':>7s}   (us)")
    for name, idx in kinds.items():
        L.exl3_timeline_clear()
        torch.cuda.synchronize()
        torch.cuda._sleep(int(2.4e7))  # the launch starts on an idle GPU
        launch([20 * 7 + j for j in idx])
        torch.cuda.synchronize()
        buf = np.zeros(WGS * 8 * 8, dtype=np.uint64)
        L.exl3_timeline_read(buf.ctypes.data, buf.nbytes)
        R = buf.reshape(WGS, 8, 8).astype(np.int64)
        live = R[:, 0, 0] > 0
        # the entry stamps carry the workgroup's XCD in bits 56-59
        xcc = (R[live, 0, 0] >> 56) & 15
        wgid = np.nonzero(live)[0]
        R[:, :, 0] &= (1 << 56) - 1
        R = R[live]
        t0 = R[:, :, 0][R[:, :, 0] > 0].min()
        us = np.where(R > 0, (R - t0) * 0.01, np.nan)
        w = us.reshape(-1, 8)
        print(f"== {name}: {len(R)} workgroups, last event at {np.nanmax(us):.2f} us")
        for e, label in enumerate(EVENTS):
            print(f"   {label:21s}{pct(w[:, e])}")
        last = ~np.isnan(w[:, 5])
        print(f"   {'stores acknowledged':21s}{pct(w[~last, 7])}")
        print(f"   {'first read returned':21s}{pct(w[last, 7])}")
        # per column group (workgroup id = split * groups + group): the last
        # split's first read after its own reduce, and its hand-off end after
        # the group's last acknowledged store
        lastwg = ~np.isnan(us[:, 0, 5])
        gx = int(lastwg.sum())
        if gx and len(R) % gx == 0:
            ksplit = len(R) // gx
            g = us.reshape(ksplit, gx, 8, 8)
            fr = g[-1, :, :2, 7] - g[-1, :, :2, 3]
            seen = g[-1, :, 0, 5] - np.nanmax(g[:-1, :, :, 7].reshape(ksplit - 1, gx, -1), axis=(0, 2))
            print(f"   {'first read latency':21s}{pct(fr.ravel())}")
            same = np.mean([len(set(xcc[wgid % gx == c])) == 1 for c in range(gx)])
            rr = max(np.mean(xcc == (wgid + r) % 8) for r in range(8))
            print(f"   XCD: {len(set(xcc.tolist()))} seen; workgroups on XCD (id + r) % 8: {rr:.3f}; "
                  f"column groups with every split on one XCD: {same:.3f}")
            print(f"   {'done after last ack':21s}{pct(seen)}")
        print(f"   {'loop duration':21s}{pct(w[:, 2] - w[:, 1])}")
        print(f"   {'hand-off duration':21s}{pct(w[:, 5] - w[:, 3])}")
        if name == "gate+up":
            for rnd in range(len(R) // 256):
                s = us[rnd * 256:(rnd + 1) * 256]
                print(f"   round {rnd} (wg {rnd * 256}-{rnd * 256 + 255}): entry {np.nanmedian(s[:, :, 0]):6.2f}"
                      f"  prepared {np.nanmedian(s[:, :, 1]):6.2f}  loop done {np.nanmedian(s[:, :, 2]):6.2f}")
        sys.stdout.flush()
    return 0


if __name__ == "__main__":
    sys.exit(main())
