"""Phase timeline of the persistent decode step (profiling tool).

Runs the 28-layer Qwen3-VL-2B persistent step (seeded synthetic weights,
random K/V rows) at a chosen context with the traced library
(``libqwen3vl_decode_trace.so``, built with -DQD_TRACE next to the main
library), reads the per-workgroup timestamps of the last launch and reports,
for every link of a layer's dependency chain, the median over the inner
layers of the time between two consecutive recorded points, where a point's
time is when the LAST workgroup passed it (the chain waits for the slowest
workgroup).  Also the layer period and the launch time (HIP events).

    QD_LIB_PATH=aicasgc-2026_amd/libqwen3vl_decode_trace.so \\
        python -m qwen3vl_hip.phase_trace --ctx 4096 [--ctx 1100] [--reps 4] [--json out.json]

The tracing stores add a few vector stores per layer; the traced launch runs
a little slower than the regular one, so absolute times come from bench.py and
this tool shows where they go.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import sys

import numpy as np

EVENTS = ["layer start", "x gathered", "qkv rows stored", "qkv gathered", "attention loop done",
          "split partials stored", "merged output gathered", "o_proj start", "r rows stored", "r gathered",
          "hidden rows stored", "hidden gathered", "x rows stored"]
# further points of the same poller wave (slots 13..15) and of a streamer wave (slots 16..31)
EXTRA = {13: "poller: W_gate/up rows issued", 14: "poller: W_down rows issued (gate_up phase)",
         15: "poller: q/k RoPE barrier passed",
         16: "streamer: layer start", 17: "streamer: x gathered", 18: "streamer: qkv rows stored",
         19: "streamer: W_gate/up rows issued", 20: "streamer: qkv gathered", 21: "streamer: q/k RoPE barrier passed",
         22: "streamer: attention loop done", 23: "streamer: W_down rows issued", 24: "streamer: slot-merge barrier passed",
         25: "streamer: merged output gathered", 26: "streamer: r rows stored", 27: "streamer: r gathered",
         28: "streamer: hidden rows stored", 29: "streamer: next layer's W_qkv, K/V, W_o issued",
         30: "streamer: hidden gathered", 31: "streamer: x rows stored"}
LINKS = ["x hand-off", "QKV rows", "qkv hand-off", "q/k norm+RoPE, attention", "slot merge + partial store",
         "split merge + merged-output hand-off", "barrier", "o_proj rows", "r hand-off", "gate_up rows",
         "hidden hand-off", "down rows"]
CLOCK_HZ = 100e6   # s_memrealtime


def timeline(ctx: int, reps: int = 4, seed: int = 3) -> dict:
    import torch

    from . import _lib
    from . import synthetic as syn
    from .engine import DecodeEngine

    if _lib.LIB_PATH.resolve() != _lib.TRACE_LIB_PATH.resolve():
        raise RuntimeError(f"load the traced library: set QD_LIB_PATH={_lib.TRACE_LIB_PATH} before starting Python")
    lib = _lib.lib()
    dims = (ctypes.c_int * 3)()
    _lib.check(lib.qd_persistent_trace_read(None, 0, dims), "qd_persistent_trace_read")
    nb, nl, ne = dims[0], dims[1], dims[2]
    dev = torch.device("cuda:0")
    w = syn.model_weights(seed, device=dev)
    eng = DecodeEngine(w, capacity=ctx + 8, step_mode="persistent")
    gen = torch.Generator(device=dev).manual_seed(seed)
    for k, v in zip(eng.k_caches, eng.v_caches):
        k.normal_(generator=gen)
        v.normal_(generator=gen)
    launch_us = []
    for _ in range(reps):
        eng.set_state(1234, ctx - 1, ctx - 1)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        eng.layers_persistent()
        e1.record()
        torch.cuda.synchronize()
        launch_us.append(e0.elapsed_time(e1) * 1000.0)
    if eng.status() != 0:
        raise RuntimeError("a hand-off timed out during the traced launches")
    buf = np.zeros(nb * nl * ne, dtype=np.uint64)
    _lib.check(lib.qd_persistent_trace_read(ctypes.c_void_p(buf.ctypes.data), buf.size, dims),
               "qd_persistent_trace_read")
    n_layers = len(w.layers)
    ev = len(EVENTS)
    t_all = buf.reshape(nb, nl, ne)[:, :n_layers, :].astype(np.int64)
    t = t_all[:, :, :ev]
    us = (t - t[:, 0, 0].min()) / CLOCK_HZ * 1e6
    us_all = (t_all - t[:, 0, 0].min()) / CLOCK_HZ * 1e6
    last = us.max(axis=0)                       # [layer, event]: the last workgroup to pass each point
    inner = slice(1, n_layers - 1)
    links = {}
    for e in range(1, ev):
        links[LINKS[e - 1]] = round(float(np.median(last[inner, e] - last[inner, e - 1])), 2)
    links["next layer start"] = round(float(np.median(last[2:n_layers, 0] - last[1:n_layers - 1, ev - 1])), 2)
    period = float(np.median(np.diff(last[:, ev - 1])))
    # every recorded point as an offset from the layer's start (last workgroup
    # through each), median over the inner layers
    last_all = us_all.max(axis=0)
    med_all = np.median(us_all, axis=0)
    names = {i: f"poller: {n}" for i, n in enumerate(EVENTS)} | (EXTRA if ne > 16 else {})
    timeline_pts = []
    for e, name in names.items():
        if e >= ne:
            continue
        off_last = float(np.median(last_all[inner, e] - last_all[inner, 0]))
        off_med = float(np.median(med_all[inner, e] - med_all[inner, 0]))
        timeline_pts.append((round(off_last, 2), round(off_med, 2), name))
    timeline_pts.sort()
    return {"context_rows": ctx, "launch_us": [round(x, 1) for x in launch_us],
            "traced_span_us": round(float(last[n_layers - 1, ev - 1]), 1), "layer_period_us": round(period, 2),
            "links_us": links,
            "timeline_us": [{"at_last_wg": a, "at_median_wg": b, "point": n} for a, b, n in timeline_pts],
            "method": "median over layers 1..L-2 of the time between consecutive points, each point taken "
                      "when the last workgroup passed it (s_memrealtime, 100 MHz), last of "
                      f"{reps} launches"}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--ctx", type=int, action="append", help="context rows (repeatable; default 1100 and 4096)")
    ap.add_argument("--reps", type=int, default=4)
    ap.add_argument("--json", help="also write the result here")
    args = ap.parse_args(argv)
    out = [timeline(c, args.reps) for c in (args.ctx or [1100, 4096])]
    for r in out:
        print(f"context {r['context_rows']}: layer period {r['layer_period_us']} us, launch "
              f"{r['launch_us'][-1]} us (traced)", file=sys.stderr)
        for k, v in r["links_us"].items():
            print(f"  {k:40s} {v:6.2f} us", file=sys.stderr)
        print("  timeline from layer start (last workgroup / median workgroup):", file=sys.stderr)
        for p in r["timeline_us"]:
            print(f"    {p['at_last_wg']:7.2f} {p['at_median_wg']:7.2f}  {p['point']}", file=sys.stderr)
    print(json.dumps(out), flush=True)
    if args.json:
        with open(args.json, "w") as f:
            json.dump(out, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
