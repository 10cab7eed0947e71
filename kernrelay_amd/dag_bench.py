"""The mm -> consumer DAG workloads through kr_plan_run on one GPU.

* tiny mm->GELU: X[256,512] . W[512,512] -> GELU-tanh, producer split k=2
  (latency-bound; reported for reference, parity is the point);
* fan-out: X[4096,4096] . W[4096,4096] -> {row softmax, GELU, bf16->fp16
  cast} per row tile, serial (one stream), B0 (two streams, unsplit) and the
  relay split at k = 1, 2, 4, 8 (schedules from kernrelay_amd.schedule, as
  the reference's E3/E4 variants, python/kernrelay/e34.py:16-22);
* the reference's own relay cases (fp16 32768x1024x2048 GEMM -> GELU,
  softmax, cast, {GELU, softmax}; the reverse edge LayerNorm 32768x2048 ->
  GEMM 2048x2048) at its k, next to its published times;
  for an elementwise consumer also the in-register relay (the same split
  schedule with the consumer computed in the GEMM's epilogue,
  KR_PLAN_EPILOGUE=1);
* the reference's two-wave DAGs on one device (two independent mm -> GELU
  chains; mm -> GELU -> mm -> GELU) at k = 4 and 8, next to its published
  times.

Each variant runs as a replayed graph per stream (`graph_per_stream`); the
reported time is the device makespan (HIP events on both streams, best and
median of the timed runs). Every variant's checksum must equal the serial
one (the relay changes when rows are computed, never what they hold).

Also reported: the producer GEMM alone (MFMA fraction of the 2.5 PFLOP/s
bf16 peak) and each consumer alone (GB/s of its algorithmic read + write
bytes against 8 TB/s).

    python -m kernrelay_amd.dag_bench [--iters 20] [--only reference_e9,...]
"""

import argparse
import contextlib
import ctypes
import json
import os
import sys
import tempfile
from pathlib import Path

from . import libapi, schedule, workloads

PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


@contextlib.contextmanager
def _stdout_to_stderr():
    """kr_plan_run prints its result line on stdout (as the reference's
    executor does); keep it off this process's stdout, which carries one
    JSON line."""
    libc = ctypes.CDLL(None)
    sys.stdout.flush()
    libc.fflush(None)
    saved = os.dup(1)
    os.dup2(2, 1)
    try:
        yield
    finally:
        libc.fflush(None)
        os.dup2(saved, 1)
        os.close(saved)


def _plan(sched, tmp, name, iters, warmup, mode="graph_per_stream", env=None):
    path = schedule.dump_schedule(sched, Path(tmp) / (name + ".json"))
    saved = {k: os.environ.get(k) for k in (env or {})}
    os.environ.update(env or {})
    try:
        with _stdout_to_stderr():
            r = libapi.plan_run(path, devices="0", mode=mode, iters=iters, warmup=warmup,
                                out_json=Path(tmp) / (name + "_out.json"))
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    if r.get("_rc") != 0 or not r.get("ok"):
        raise RuntimeError("kr_plan_run %s failed: %s" % (name, r))
    return r


def _times(r):
    return {"device_best_us": round(r["device_best_us"], 2),
            "device_p50_us": round(r["device_p50_us"], 2),
            "wall_p50_us": round(r["p50_us"], 2)}


def fanout(tmp, M=4096, K=4096, N=4096, ks=(1, 2, 4, 8), iters=20, warmup=3):
    dag = workloads.mm_fanout(tmp, M, K, N)
    serial = _plan(schedule.serial_schedule(dag), tmp, "serial", iters, warmup)
    out = {"shape": [M, K, N], "consumers": ["softmax", "gelu", "cast"],
           "serial": _times(serial), "checksum": serial["checksum"]}
    b0 = _plan(workloads.variants(dag, 1)["b0"], tmp, "b0", iters, warmup)
    out["b0"] = _times(b0)
    same = [b0["checksum"] == serial["checksum"]]
    out["split"] = {}
    for k in ks:
        r = _plan(workloads.variants(dag, k)["split"], tmp, "split%d" % k, iters, warmup)
        same.append(r["checksum"] == serial["checksum"])
        t = _times(r)
        t["vs_serial"] = round(serial["device_best_us"] / r["device_best_us"], 4)
        t["vs_b0"] = round(b0["device_best_us"] / r["device_best_us"], 4)
        out["split"][str(k)] = t
    out["checksums_equal"] = all(same)
    return out


def tiny(tmp, iters=50, warmup=5):
    dag = workloads.tiny_mm_gelu(tmp)
    serial = _plan(schedule.serial_schedule(dag), tmp, "tiny_serial", iters, warmup)
    split = _plan(workloads.variants(dag, 2)["split"], tmp, "tiny_split2", iters, warmup)
    # the same split schedule with GELU computed in the GEMM's epilogue
    reg = _plan(workloads.variants(dag, 2)["split"], tmp, "tiny_split2_epi", iters, warmup,
                env={"KR_PLAN_EPILOGUE": "1"})
    return {"shape": [256, 512, 512], "serial": _times(serial), "split2": _times(split),
            "split2_register_relay": dict(_times(reg), epilogue_consumers=reg.get("epilogue_consumers")),
            "checksums_equal": serial["checksum"] == split["checksum"] == reg["checksum"]}


# The reference's relay table (Ascend 910B3, nhp_exec, best of 3 x 5 runs):
# case -> (consumers, k, serial us, B0 us, split us), RESULTS.md:67-76.
E34_REFERENCE = {
    "mm_gelu_k2": (["gelu"], 2, 971.7, 981.1, 890.4),
    "mm_gelu_k4": (["gelu"], 4, 978.8, 974.0, 889.2),
    "mm_gelu_k8": (["gelu"], 8, 1008.4, 1014.9, 911.3),
    "mm_softmax_k4": (["softmax"], 4, 1133.0, 1132.3, 888.4),
    "mm_cast_k4": (["cast"], 4, 1018.6, 966.3, 944.2),
    "mm_fanout_gelu_softmax_k4": (["gelu", "softmax"], 4, 1406.1, 1424.5, 1318.3),
    # the reverse edge: LayerNorm [32768, 2048] releasing row tiles to the
    # GEMM (K = N = 2048) that reads them as A (RESULTS.md:73)
    "e3_ln_mm_k4": (None, 4, 1890.3, 1885.5, 1456.8),
}


def reference_e34(tmp, iters=20, warmup=3):
    """The reference's own relay cases at its shapes and dtype (fp16 GEMM
    32768x1024x2048 -> consumers, and the reverse edge LayerNorm
    32768x2048 -> GEMM K = N = 2048; DetValue inputs, one rank): serial, B0
    and the split at the reference's k, with the reference's published times
    beside ours."""
    out = {}
    for case, (consumers, k, r_serial, r_b0, r_split) in E34_REFERENCE.items():
        dag = workloads.e34_dag(case, consumers)
        v = workloads.variants(dag, k)
        rs = {name: _plan(v[name], tmp, "%s_%s" % (case, name), iters, warmup) for name in ("serial", "b0", "split")}
        if consumers is not None and len(consumers) == 1 and consumers[0] in ("gelu", "silu", "cast"):
            # the same split schedule with the consumer in the GEMM's epilogue
            rs["register_relay"] = _plan(v["split"], tmp, "%s_epi" % case, iters, warmup, env={"KR_PLAN_EPILOGUE": "1"})
        ours = {name: round(rs[name]["device_best_us"], 2) for name in rs}
        out[case] = {
            "k": k,
            "serial_us": ours["serial"], "b0_us": ours["b0"], "split_us": ours["split"],
            "serial_over_split": round(ours["serial"] / ours["split"], 4),
            "flag_edges": rs["split"]["flag_edges"],
            "reference_serial_over_split": round(r_serial / r_split, 4),
            "reference_us": {"serial": r_serial, "b0": r_b0, "split": r_split},
            "checksums_equal": len({rs[n]["checksum"] for n in rs}) == 1,
        }
        if "register_relay" in rs:
            out[case]["register_relay_us"] = ours["register_relay"]
            out[case]["serial_over_register_relay"] = round(ours["serial"] / ours["register_relay"], 4)
    return out


# The reference's two-wave table (Ascend 910B3, nhp_exec, best of 3 x 5 runs):
# case -> (dag, k, serial us, B0 us, split us), RESULTS.md:104-108.
E9_REFERENCE = {
    "e9_two_waves_k4": ("e9_two_waves", 4, 1791.2, 1617.6, 1532.0),
    "e9_two_waves_k8": ("e9_two_waves", 8, 1840.9, 1648.0, 1571.4),
    "e9_chain2_k4": ("e9_chain2", 4, 2270.1, 2276.0, 2063.6),
    "e9_chain2_k8": ("e9_chain2", 8, 2275.8, 2290.0, 2105.0),
}


def reference_e9(tmp, iters=20, warmup=3):
    """The reference's two-wave DAGs on one device at its shapes (fp16,
    DetValue inputs, one rank): two independent mm -> GELU chains, and
    mm -> GELU -> mm -> GELU; serial, B0 and the split at k, with the
    reference's published times beside ours."""
    out = {}
    for case, (name, k, r_serial, r_b0, r_split) in E9_REFERENCE.items():
        v = workloads.variants(workloads.e9_dag(name), k)
        rs = {vn: _plan(v[vn], tmp, "%s_%s" % (case, vn), iters, warmup) for vn in ("serial", "b0", "split")}
        ours = {vn: round(rs[vn]["device_best_us"], 2) for vn in rs}
        out[case] = {
            "k": k,
            "serial_us": ours["serial"], "b0_us": ours["b0"], "split_us": ours["split"],
            "serial_over_split": round(ours["serial"] / ours["split"], 4),
            "b0_over_split": round(ours["b0"] / ours["split"], 4),
            "flag_edges": rs["split"]["flag_edges"],
            "reference_serial_over_split": round(r_serial / r_split, 4),
            "reference_us": {"serial": r_serial, "b0": r_b0, "split": r_split},
            "checksums_equal": len({rs[vn]["checksum"] for vn in rs}) == 1,
        }
    return out


def _event_us(fn, reps=10):
    import torch
    fn()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) * 1e3 / reps)
    return best


def kernels_alone(M=4096, K=4096, N=4096):
    import torch
    from . import ops
    g = torch.Generator(device="cuda").manual_seed(1234)
    A = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    Bt = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    C = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    us = _event_us(lambda: ops.gemm(A, Bt, C))
    tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
    out = {"gemm": {"us": round(us, 2), "tflops": round(tf, 1),
                    "mfma_frac": round(tf / PEAK_BF16_TFLOPS, 4)}}
    y16 = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    yh = torch.empty(M, N, device="cuda", dtype=torch.float16)
    for name, fn, nbytes in (
            ("softmax", lambda: ops.rowop("softmax", C, y16), 4 * M * N),
            ("gelu", lambda: ops.elementwise("gelu", C, y16), 4 * M * N),
            ("cast", lambda: ops.elementwise("cast", C, yh), 4 * M * N)):
        us = _event_us(fn)
        gbs = nbytes / (us * 1e-6) / 1e9
        out[name] = {"us": round(us, 2), "gbs": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)}
    return out


SECTIONS = ("tiny_mm_gelu", "fanout_4096", "alone_4096", "reference_e34", "reference_e9")


def run_all(iters=20, only=SECTIONS):
    with tempfile.TemporaryDirectory(prefix="kr_dag_") as tmp:
        run = {"tiny_mm_gelu": lambda: tiny(tmp), "fanout_4096": lambda: fanout(tmp, iters=iters),
               "alone_4096": kernels_alone, "reference_e34": lambda: reference_e34(tmp, iters=iters),
               "reference_e9": lambda: reference_e9(tmp, iters=iters)}
        return {name: run[name]() for name in SECTIONS if name in only}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--only", default=",".join(SECTIONS),
                    help="comma-separated sections to run (default: all): " + ", ".join(SECTIONS))
    args = ap.parse_args(argv)
    only = [x for x in args.only.split(",") if x]
    unknown = set(only) - set(SECTIONS)
    if unknown:
        raise SystemExit("unknown section(s): %s" % ", ".join(sorted(unknown)))
    print(json.dumps(run_all(args.iters, only)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
