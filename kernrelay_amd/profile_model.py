"""Measure the planner's cost table on this GPU.

* ``profile``          — ``kr_qwen_profile_many`` over the reference's op list
                         at k = 1, 2, 4, 8 row slices (scripts/profile_model.py:
                         13-34): op -> {k: best_us}; plus the relay split's
                         own launches (the o / down GEMM releasing k row
                         tiles to Add+RMSNorm in its workgroups, the fused
                         gate/up GEMM, SwiGLU), which price its flag edges
                         (planner.relay_edges).
* ``measure_constants`` — the cost file's scalars (configs/planner2_costs.json
                         keys): ``launch_us`` (one more kernel in a replayed
                         graph), ``event_us`` (an event record on one stream
                         and a wait on another, over a same-stream
                         dependency),
                         ``traffic_gbps`` (device copy), ``l2_mb`` (the
                         last-level cache a re-read of B can hit: MI355X's
                         256 MB Infinity Cache).
* ``measure_dag_ops``  — unsplit times of the DAG-catalogue shapes the cost
                         file lists (GELU, softmax, cast, add, GEMM at the
                         e3/e9 sizes) on this library's kernels.
* ``build_costs``      — the cost file: ``full`` = the catalogue shapes plus
                         every node of the model's planner DAG (the
                         reference's and the fused program's) at its k=1
                         time, ``curves`` = the (k=1, k=8) slope per shape.

    python -m kernrelay_amd.profile_model --preset qwen2.5-7b --seq 2048 \\
        --out profile.json --costs-out kernrelay_amd/costs_mi355x.json
"""

import argparse
import json
import shutil
import sys
import tempfile
import time
from pathlib import Path

from . import planner

INFINITY_CACHE_MB = 256.0

# catalogue shapes of the reference's cost file that this library runs
# (op, rows, cols) for element-wise / row ops, (M, K, N) for GEMMs
DAG_EW = [("gelu", 32768, 2048), ("softmax", 32768, 2048), ("cast", 32768, 2048),
          ("gelu", 131072, 4096), ("softmax", 131072, 4096), ("cast", 131072, 4096),
          ("add", 131072, 4096)]
DAG_MM = [(8192, 1024, 2048), (24576, 1024, 2048), (32768, 1024, 2048), (65536, 2048, 4096)]


def log(msg):
    print("[profile] " + msg, file=sys.stderr, flush=True)


def profile(model_dir, seq, device=0, ks=(1, 2, 4, 8), ops=planner.PROFILE_OPS):
    from . import libapi
    cases = [{"op": op, "k": k} for op in ops for k in ks]
    raw = libapi.qwen_profile_many(model_dir, cases, seq=seq, device=device)
    if raw.get("_rc") not in (None, 0):
        raise RuntimeError("kr_qwen_profile_many failed: %s" % raw.get("error"))
    return {"table": planner.profile_table(raw), "raw": raw}


def _graph_time_us(body, reps=20):
    """Device time of one replay of a captured graph of ``body``."""
    import torch
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        body()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        body()
    g.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(s):
            e0.record()
            for _ in range(reps):
                g.replay()
            e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / reps)
    return best


def _event_time_us(body, reps=5):
    import torch
    body()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        body()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3)
    return best


def measure_constants(n=256):
    import torch
    x = torch.zeros(64, device="cuda")

    def chain():
        for _ in range(n):
            x.add_(1.0)

    launch_us = _graph_time_us(chain) / n

    # eager: n dependent tiny kernels on one stream vs the same n kernels
    # alternating between two streams with an event handoff between each
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()

    def one_stream():
        with torch.cuda.stream(s1):
            for _ in range(n):
                x.add_(1.0)
        torch.cuda.current_stream().wait_stream(s1)

    def ping_pong():
        cur, other = s1, s2
        cur.wait_stream(torch.cuda.current_stream())
        for _ in range(n):
            with torch.cuda.stream(cur):
                x.add_(1.0)
            other.wait_stream(cur)
            cur, other = other, cur
        torch.cuda.current_stream().wait_stream(cur)

    event_us = max(0.0, (_event_time_us(ping_pong) - _event_time_us(one_stream)) / n)

    a = torch.empty(512 * 1024 * 1024, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    t = _event_time_us(lambda: b.copy_(a))
    traffic_gbps = 2.0 * a.numel() / (t * 1e-6) / 1e9
    del a, b
    torch.cuda.empty_cache()
    return {"launch_us": round(launch_us, 3), "event_us": round(event_us, 3),
            "traffic_gbps": round(traffic_gbps, 1), "l2_mb": INFINITY_CACHE_MB}


def measure_dag_ops():
    import torch
    from . import ops
    full = {}
    g = torch.Generator(device="cuda").manual_seed(1234)
    for op, rows, cols in DAG_EW:
        x = torch.randn(rows, cols, device="cuda", generator=g).to(torch.bfloat16)
        x1 = torch.randn(rows, cols, device="cuda", generator=g).to(torch.bfloat16) if op == "add" else None
        y = torch.empty(rows, cols, device="cuda",
                        dtype=torch.float16 if op == "cast" else torch.bfloat16)
        if op == "softmax":
            body = lambda x=x, y=y: ops.rowop("softmax", x, y)
        else:
            body = lambda op=op, x=x, y=y, x1=x1: ops.elementwise(op, x, y, x1=x1)
        full["%s|%dx%d" % (op, rows, cols)] = round(_event_time_us(body), 3)
        del x, x1, y
    for M, K, N in DAG_MM:
        A = (torch.randn(M, K, device="cuda", generator=g)).to(torch.bfloat16)
        Bt = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        C = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
        full["matmul|%dx%dx%d" % (M, K, N)] = round(
            _event_time_us(lambda A=A, Bt=Bt, C=C: ops.gemm(A, Bt, C)), 3)
        del A, Bt, C
    torch.cuda.empty_cache()
    return full


def _col(v, k):
    return v.get(k, v.get(str(k)))


def build_costs(cfg, seq, table, consts, dag_full, model=""):
    """The cost file (configs/planner2_costs.json layout plus ``curves``)."""
    nodes = planner.layer_dag(cfg, seq)["nodes"] + planner.layer_dag(cfg, seq, fused=True)["nodes"]
    full = dict(dag_full)
    curves = {}
    for n in nodes:
        v = table.get(planner.profile_op(n)) or {}
        t1, t8 = _col(v, 1), _col(v, 8)
        if not t1:
            continue
        key = planner.shape_key(n)
        full[key] = round(float(t1), 3)
        if t8:
            curves[key] = {"op": n["op"], "strategy": "row", "shape": n["shape"],
                           "base_best_us": float(t1),
                           "fit": {"slope_us_per_tile": max(0.0, (float(t8) - float(t1)) / 7.0),
                                   "intercept_us": float(t1)}}
    out = {"description": "planner cost table measured on one MI355X (gfx950): unsplit "
                          "kernel times per shape (full), split curves from the k=1 and "
                          "k=8 row-slice profile (curves), launch / cross-stream event / "
                          "copy-bandwidth constants; written by kernrelay_amd.profile_model",
           "device": "MI355X", "model": model, "seq": seq}
    out.update(consts)
    out["full"] = full
    out["curves"] = curves
    out["profile_table"] = {op: {str(k): v for k, v in sorted(cols.items(), key=lambda x: int(x[0]))}
                            for op, cols in table.items()}
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--preset", default=None, help="write a random-init model dir of this preset")
    ap.add_argument("--model", default=None, help="existing model dir (manifest.json)")
    ap.add_argument("--seq", type=int, default=2048)
    ap.add_argument("--device", type=int, default=0)
    ap.add_argument("--ks", default="1,2,4,8")
    ap.add_argument("--out", required=True, help="profile JSON ({table, raw})")
    ap.add_argument("--costs-out", default=None, help="also write the cost file here")
    args = ap.parse_args(argv)
    import torch
    from . import modeldir
    if not torch.cuda.is_available():
        raise SystemExit("profile_model needs a GPU")
    tmp = None
    try:
        if args.model:
            mdir = Path(args.model)
        else:
            tmp = Path(tempfile.mkdtemp(prefix="kr_profile_"))
            log("writing %s model dir (2 layers: the profile times layer 0) to %s" % (args.preset, tmp))
            mdir = modeldir.write_model_dir(tmp, args.preset, seq=args.seq, layers=2, device="cuda")
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
        cfg = json.loads((mdir / "manifest.json").read_text())["config"]
        ks = [int(k) for k in args.ks.split(",")]
        t0 = time.time()
        ops = planner.PROFILE_OPS + planner.RELAY_PROFILE_OPS
        ops += tuple(o for o in planner.FUSED_PROFILE_OPS if o not in ops)
        log("kr_qwen_profile_many %d ops x k=%s" % (len(ops), ks))
        prof = profile(mdir, args.seq, args.device, ks, ops=ops)
        log("profile done in %.1f s" % (time.time() - t0))
        Path(args.out).write_text(json.dumps(prof, indent=1))
        if args.costs_out:
            log("constants")
            consts = measure_constants()
            log("  %s" % consts)
            log("DAG catalogue shapes")
            dag_full = measure_dag_ops()
            costs = build_costs(cfg, args.seq, prof["table"], consts, dag_full,
                                model=args.preset or str(mdir))
            Path(args.costs_out).write_text(json.dumps(costs, indent=1) + "\n")
            log("wrote %s" % args.costs_out)
        print(json.dumps({"table": prof["table"]}), flush=True)
    finally:
        if tmp:
            shutil.rmtree(tmp, ignore_errors=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
