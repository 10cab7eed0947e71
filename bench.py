"""Headline benchmark: Qwen2.5-7B-shaped bf16 prefill at seq 2048 on one
MI355X through kr_qwen_run — serial (graph_whole) vs the relay split at 4
tiles — plus the producer GEMM's roofline and the CPU (oracle) baseline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--tiles 4] [--preset qwen2.5-7b]

Prints ONE JSON line. A step is one full prefill (28 layers + lm_head over all
2048 rows) with weights and inputs resident in HBM; `value` is tokens/s of the
relay-split prefill over exactly K timed steps (each step bracketed by device
synchronisation inside the library). The split's flag edges (o and down
releasing row tiles to Add+RMSNorm) are priced on the card first and only
those that pay are taken (relay_split:<k>:<edges>). Weights are random-init
N(0, 0.02) (`data: synthetic`): no checkpoint can be fetched on this pool.

Beside the headline: the ablations (no flag edge, both flag edges, both
without the SwiGLU fusion); the CPU baseline, the oracle's whole prefill on
the host with its last-row logits compared with the GPU's; the mm ->
consumer DAG workloads (kernrelay_amd.dag_bench); and the Qwen2.5-0.5B (seq
2048) and Qwen3-8B text (seq 4096) prefills, serial and split.
"""

import argparse
import json
import os
import shutil
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA peak (vendor figure, no sparsity)
PEAK_HBM_GBS = 8000.0
REF_BEST_TOK_S = 2048 / 0.1462  # reference graph_whole, Qwen2.5-7B seq 2048, Ascend 910B3 (RESULTS.md:21)
PRESET_NAMES = {"qwen2.5-7b": "Qwen2.5-7B", "qwen2.5-0.5b": "Qwen2.5-0.5B", "qwen3-8b": "Qwen3-8B"}


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


# HBM bytes per launch of the gate/up GEMM with SwiGLU epilogue at
# 2048x37888x3584 (bf16), from two rocprofv3 --pmc passes over single
# launches (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by
# what the same counter reads for a plain 512 MiB device copy; and rocprof's
# MFMA utilisation of the same launches (SQ_VALU_MFMA_BUSY_CYCLES over
# GRBM_GUI_ACTIVE x SIMDs, at the clock the card ran).
GATE_UP_TRAFFIC_BYTES = (423154.0 * 2.0 + 75776.0 * 1.0) * 1024
GATE_UP_MFMA_UTIL = 0.627
GATE_UP_TRAFFIC_SOURCE = "profiles/gemm_gate_up_swiglu_2048x37888x3584.md"


def gemm_roofline(run, serial, S, N, K):
    """The dominant kernel of the measured (relay split) prefill: the gate/up
    GEMM with SwiGLU in its epilogue. With KR_TIME_GATE_UP=1 the library runs
    one more pass of the same program after the timed graph replays,
    launched eagerly with HIP events around each gate/up launch on the
    stream it runs on, and reports their average (28 launches, interleaved
    with the layer's other kernels as in the timed run). Algorithmic work
    2*S*N*K flop per launch; algorithmic bytes A + B + act (the epilogue
    writes act[S, N/2], never the [S, N] product)."""
    avg_us = run["gate_up_avg_us"]
    flops = 2.0 * S * N * K
    achieved = flops / (avg_us * 1e-6) / 1e12
    ser_us = serial["gate_up_avg_us"]
    # the counter passes were run on the 7B layer's shape
    measured = (S, N, K) == (2048, 37888, 3584)
    return {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": round(GATE_UP_TRAFFIC_BYTES) if measured else None,
            "traffic_algorithmic": 2 * (S * K + N * K + S * N // 2),
            "traffic_source": GATE_UP_TRAFFIC_SOURCE if measured else None,
            "kernel": "GemmPipeKernel<bf16,256,256,8 waves> + its 192x256 wave-tail launch, gate/up projection "
                      "%dx%dx%d, SwiGLU epilogue"
                      % (S, N, K),
            "avg_launch_us": round(avg_us, 2), "launches": int(run["gate_up_launches"]),
            "timing": "HIP events around each gate/up GEMM (its launches) in an eager pass of the relay-split prefill",
            "mfma_util_rocprof": GATE_UP_MFMA_UTIL if measured else None,
            "serial_gate_up": {"avg_launch_us": round(ser_us, 2),
                               "achieved": round(flops / (ser_us * 1e-6) / 1e12, 1),
                               "note": "the serial program's plain gate/up GEMM (writes the [S, 2I] product)"}}


def cpu_model():
    """The host CPU's model name: /proc/cpuinfo's "model name", completed
    by lscpu where a hypervisor shortens it (e.g. to "AMD EPYC")."""
    name = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                name = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        info = {k.strip(): v.strip() for k, v in (l.split(":", 1) for l in out.splitlines() if ":" in l)}
        full = info.get("Model name", "")
        if len(full) > len(name):
            name = full
        for key in ("CPU family", "Model", "Stepping"):
            if key in info:
                name += ", %s %s" % (key.lower(), info[key])
    except Exception:
        pass
    if not name:
        import platform
        name = platform.processor() or platform.machine()
    return name


def cpu_share():
    """Threads for the CPU baseline: the CPUs this process may use, i.e. its
    affinity mask, capped by a cgroup CPU quota where one is set (a quota of
    q CPUs under a wider affinity mask would only throttle more threads).
    Returns (threads, how)."""
    aff = len(os.sched_getaffinity(0))
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            quota = int(q) / int(period)
    except (OSError, ValueError):
        try:
            q = int(open("/sys/fs/cgroup/cpu/cpu.cfs_quota_us").read())
            period = int(open("/sys/fs/cgroup/cpu/cpu.cfs_period_us").read())
            if q > 0:
                quota = q / period
        except (OSError, ValueError):
            pass
    if quota is not None and quota < aff:
        return max(1, int(quota)), "cgroup CPU quota %.1f (affinity %d)" % (quota, aff)
    return aff, "affinity mask (%d CPUs, no lower cgroup quota)" % aff


def cpu_baseline(model_dir, gpu_last_logits=None):
    """The oracle (fp32 torch CPU) running the whole prefill on the host: every
    decoder layer and the lm_head over all rows, the work of the GPU step, on
    every CPU the process may use. Its last-row logits are compared with the
    GPU's (bf16 values) in the same run."""
    import numpy as np
    import torch

    from oracle import qwen as oq

    threads, how = cpu_share()
    torch.set_num_threads(threads)
    m = oq.ModelDir(model_dir)
    S = m.ids().numel()
    t0 = time.perf_counter()
    res = oq.prefill(m, lm_all_rows=True)
    total = time.perf_counter() - t0
    out = {"value": round(S / total, 2), "unit": "tok/s", "cores": threads, "threads_from": how,
           "cpu_model": cpu_model(), "kind": "port", "scope": "full",
           "sample": "oracle fp32 torch-CPU, the whole prefill: %d decoder layers + lm_head over all %d rows "
                     "at seq %d, weights converted from the model directory's bf16 as each op runs" % (m.L, S, S),
           "ms_per_prefill": round(total * 1e3, 1), "oracle_argmax": res["argmax"],
           "oracle_top2_margin": round(res["margin"], 5),
           "oracle_argmax_fp32": res["argmax_fp32"], "oracle_top2_margin_fp32": round(res["margin_fp32"], 5)}
    if gpu_last_logits is not None:
        ref = res["last_logits"].float()
        gpu = torch.from_numpy(np.asarray(gpu_last_logits, dtype=np.float32))
        d = (gpu - ref).abs()
        g2 = torch.topk(gpu, 2)
        out["gpu_vs_oracle"] = {"max_abs": round(float(d.max()), 5), "mean_abs": round(float(d.mean()), 6),
                                "argmax_equal": int(gpu.argmax()) == res["argmax"],
                                "argmax_equal_fp32": int(gpu.argmax()) == res["argmax_fp32"],
                                "gpu_argmax": int(gpu.argmax()),
                                "gpu_top2_margin": round(float(g2.values[0] - g2.values[1]), 5)}
    return out


def read_dumped_logits(path):
    """Last-row logits kr_qwen_run wrote under KR_DUMP_DIR (bf16) as fp32."""
    import numpy as np
    raw = np.fromfile(path, dtype=np.uint16)
    return (raw.astype(np.uint32) << 16).view(np.float32)


def profile_gemm(M, N, K, reps, rotate=1):
    """One producer-GEMM launch per repetition on random bf16 inputs: the
    program the rocprofv3 --pmc passes of the roofline's traffic run.
    rotate > 1 cycles the launches through that many weight matrices, so
    that (with rotate x the weight's bytes above the 256 MB Infinity Cache)
    every launch reads its weight cold from HBM, as each layer of a prefill
    does."""
    import torch

    from kernrelay_amd import ops

    g = torch.Generator(device="cuda").manual_seed(7)
    A = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    Bts = [(torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16) for _ in range(rotate)]
    C = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    for i in range(reps):
        ops.gemm(A, Bts[i % rotate], C)
    torch.cuda.synchronize()
    print("gemm %dx%dx%d x%d (%d weights) done" % (M, N, K, reps, rotate), flush=True)


def profile_gemm_swiglu(M, I, K, reps):
    """One gate/up GEMM launch with SwiGLU in its epilogue per repetition
    (the relay split's dominant kernel) on random bf16 inputs: the program
    the rocprofv3 --pmc passes of the roofline's traffic run."""
    import torch

    from kernrelay_amd import ops

    g = torch.Generator(device="cuda").manual_seed(7)
    A = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    Bt = (torch.randn(2 * I, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    act = torch.empty(M, I, device="cuda", dtype=torch.bfloat16)
    for _ in range(reps):
        ops.gemm_swiglu_epilogue(A, Bt, act)
    torch.cuda.synchronize()
    print("gemm+swiglu %dx%dx%d x%d done" % (M, 2 * I, K, reps), flush=True)


def profile_consumers(reps):
    """One launch per repetition of each consumer kernel and of attention at
    the shapes the relay path runs them (the program the rocprofv3 --pmc
    passes of the consumer traffic and the attention counters run):
    row softmax, GELU and bf16->fp16 cast over [4096, 4096] (the fan-out
    DAG's consumers), Add+RMSNorm over
    [2048, 3584] (the 7B residual) and causal attention at 28 query / 4 kv
    heads x 2048 x 128 (the 7B layer)."""
    import torch

    from kernrelay_amd import ops

    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn(4096, 4096, device="cuda", generator=g).to(torch.bfloat16)
    y = torch.empty_like(x)
    yh = torch.empty(4096, 4096, device="cuda", dtype=torch.float16)
    a = torch.randn(2048, 3584, device="cuda", generator=g).to(torch.bfloat16)
    b = torch.randn(2048, 3584, device="cuda", generator=g).to(torch.bfloat16)
    gam = torch.ones(3584, device="cuda", dtype=torch.bfloat16)
    ny, ns = torch.empty_like(a), torch.empty_like(a)
    rstd = torch.empty(2048, device="cuda")
    S, HQ, HKV, D = 2048, 28, 4, 128
    qkv = torch.randn(S, (HQ + 2 * HKV) * D, device="cuda", generator=g).to(torch.bfloat16)
    ld = qkv.stride(0)
    q, k, v = qkv[:, :HQ * D], qkv[:, HQ * D:(HQ + HKV) * D], qkv[:, (HQ + HKV) * D:]
    att = torch.empty(S, HQ * D, device="cuda", dtype=torch.bfloat16)
    for _ in range(reps):
        ops.rowop("softmax", x, y)
        ops.elementwise("gelu", x, y)
        ops.elementwise("cast", x, yh)
        ops.rowop("add_rmsnorm", a, ny, x1=b, gamma=gam, sum_out=ns, rstd_out=rstd)
        ops.attention(q, k, v, att, S, HQ, HKV, D, ldq=ld, ldk=ld, ldv=ld)
    torch.cuda.synchronize()
    print("consumers + attention x%d done" % reps, flush=True)


def profile_prefill(model_dir, preset, S, mode, reps):
    """The prefill alone (kr_qwen_run: 1 warm-up + `reps` timed graph
    replays of `mode`, then its eager timing pass with HIP events around each
    GEMM and attention) on a model directory written first if missing: the
    program the rocprofv3 passes over the prefill's kernels run."""
    import torch

    from kernrelay_amd import libapi, modeldir
    model_dir = Path(model_dir)
    if not (model_dir / "manifest.json").exists():
        modeldir.write_model_dir(model_dir, preset, seq=S, device="cuda")
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        print("model dir %s written" % model_dir, flush=True)
    os.environ["KR_TIME_OPS"] = "1"
    r = libapi.qwen_run(model_dir, mode=mode, seq=S, device=0, warmup=1, iters=reps)
    if r.get("_rc") != 0:
        raise RuntimeError("kr_qwen_run %s failed: %s" % (mode, r.get("error")))
    print(json.dumps({key: r.get(key) for key in ("mode", "best_us", "typical_us", "argmax", "flag_edges",
                                                  "flag_timeouts", "logits_fnv64", "op_avg_us")}), flush=True)


def profile_copy(mib, reps):
    """A plain device copy of known size: what FETCH_SIZE / WRITE_SIZE read
    for it calibrates the counters."""
    import torch

    x = torch.ones(mib * 1024 * 512, dtype=torch.bfloat16, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    print("copy %d MiB x%d done" % (mib, reps), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--tiles", type=int, default=4)
    ap.add_argument("--seq", type=int, default=2048)
    ap.add_argument("--preset", default="qwen2.5-7b")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-dag", action="store_true", help="skip the mm -> consumer DAG workloads")
    ap.add_argument("--no-ablation", action="store_true",
                    help="skip the fusion-only and flag-relay programs")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the Qwen2.5-0.5B (seq 2048) and Qwen3-8B text (seq 4096) configurations")
    ap.add_argument("--keep", default=None, help="keep / reuse the model directory here")
    ap.add_argument("--profile-gemm", nargs=3, type=int, metavar=("M", "N", "K"),
                    help="only launch the producer GEMM --reps times (for rocprofv3 --pmc)")
    ap.add_argument("--profile-gemm-swiglu", nargs=3, type=int, metavar=("M", "I", "K"),
                    help="only launch the gate/up GEMM with SwiGLU epilogue --reps times (for rocprofv3 --pmc)")
    ap.add_argument("--profile-copy", type=int, metavar="MIB", help="only copy MIB MiB --reps times")
    ap.add_argument("--profile-consumers", action="store_true",
                    help="only launch the consumer kernels and attention --reps times (for rocprofv3 --pmc)")
    ap.add_argument("--profile-prefill", metavar="MODE",
                    help="only run the prefill in this kr_qwen_run mode --reps times on the --keep model dir "
                         "(written if missing; for rocprofv3)")
    ap.add_argument("--reps", type=int, default=3)
    ap.add_argument("--rotate", type=int, default=1,
                    help="--profile-gemm: cycle through this many weight matrices (cold weights)")
    args = ap.parse_args()
    if args.profile_gemm:
        profile_gemm(*args.profile_gemm, args.reps, args.rotate)
        return
    if args.profile_gemm_swiglu:
        profile_gemm_swiglu(*args.profile_gemm_swiglu, args.reps)
        return
    if args.profile_copy:
        profile_copy(args.profile_copy, args.reps)
        return
    if args.profile_consumers:
        profile_consumers(args.reps)
        return
    if args.profile_prefill:
        if not args.keep:
            raise SystemExit("--profile-prefill needs --keep <model dir>")
        profile_prefill(args.keep, args.preset, args.seq, args.profile_prefill, args.reps)
        return
    if args.gpus != 1:
        print("bench.py: --gpus %d is not supported: the relay path runs on one GPU (across GPUs it would "
              "shard the sequence's rows, each GPU holding the weights)" % args.gpus, file=sys.stderr)
        sys.exit(2)

    import torch

    from kernrelay_amd import libapi, modeldir

    libapi.lib()
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    cfg = dict(modeldir.PRESETS[args.preset])
    S = args.seq
    k = args.tiles
    tmp = Path(args.keep) if args.keep else model_dir_path()
    try:
        head = prefill_config(tmp, args.preset, S, k, args.steps, args.warmup, ablation=not args.no_ablation,
                              dump_logits=not args.no_cpu)
        serial, split = head["runs"]["serial"], head["runs"]["split"]
        I, H = cfg["intermediate_size"], cfg["hidden_size"]
        roof = gemm_roofline(split, serial, S, 2 * I, H)
        total_split_s = sum(split["samples_us"]) / 1e6
        total_serial_s = sum(serial["samples_us"]) / 1e6
        value = args.steps * S / total_split_s
        flops = modeldir.model_flops(cfg, S)
        cpu = None
        if not args.no_cpu:
            log("cpu baseline: the oracle's whole prefill on the host, last-row logits against the GPU's")
            cpu = cpu_baseline(tmp, read_dumped_logits(head["dump"]))
            log("  %s" % json.dumps(cpu))
    finally:
        if not args.keep:
            shutil.rmtree(tmp, ignore_errors=True)
    dag = None
    if not args.no_dag:
        from kernrelay_amd import dag_bench
        log("DAG workloads: tiny mm->GELU, 4096^3 mm -> {softmax, gelu, cast} at k=1,2,4,8, the reference's "
            "E3/E4 (incl. LayerNorm -> GEMM) and two-wave DAGs")
        dag = dag_bench.run_all()
    extra = {}
    if not args.no_extra and (args.preset, S) == ("qwen2.5-7b", 2048):
        for preset, seq in EXTRA_CONFIGS:
            t2 = model_dir_path()
            try:
                r = prefill_config(t2, preset, seq, k, args.steps, args.warmup, ablation=False,
                                   dump_logits=False)
                extra["%s@%d" % (preset, seq)] = config_summary(r, seq)
            finally:
                shutil.rmtree(t2, ignore_errors=True)
    if head["edges"]:
        workload = ("%s-shaped prefill, batch 1, seq %d: relay split at %d row tiles, flag edges %s -> "
                    "Add+RMSNorm (%d flag blocks per prefill; the fastest edge subset replayed in place), SwiGLU "
                    "fused into the gate/up GEMM epilogue" % (PRESET_NAMES.get(args.preset, args.preset), S, k,
                                                               "+".join(head["edges"]), split["flag_edges"]))
    else:
        workload = ("%s-shaped prefill, batch 1, seq %d: relay split at %d row tiles with SwiGLU fused into the "
                    "gate/up GEMM epilogue; replayed in place, no o/down flag edge subset beat none, so none is "
                    "taken" % (PRESET_NAMES.get(args.preset, args.preset), S, k))
    out = {
        "metric": "Qwen2.5-7B prefill tok/s @seq2048 1 GPU; split-vs-serial speedup; MFMA util",
        "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(total_split_s * 1e3 / args.steps, 3),
        "higher_is_better": True, "scaling": "weak",
        # the published reference number is for the 7B model at seq 2048
        "vs_baseline": round(value / REF_BEST_TOK_S, 3) if (args.preset, S) == ("qwen2.5-7b", 2048) else None,
        "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) bf16 weights, uniform token ids)",
        "config": {"workload": workload, "model": args.preset, "global_batch": 1, "seq_len": S,
                   "parallelism": "none (1 GPU)", "relay_tiles": k, "split_mode": head["split_mode"]},
        "serial_ms_per_step": round(total_serial_s * 1e3 / args.steps, 3),
        "serial_tok_s": round(args.steps * S / total_serial_s, 1),
        "split_vs_serial": round(total_serial_s / total_split_s, 4),
        # flag edges kept by the library after replaying every subset in
        # place (tuned_us: median replay of each; an edge subset is kept
        # only if it beats none by more than 0.5%), and the planner's choice
        # from the per-op profile (priced) for comparison
        "relay_edges": {"chosen": head["edges"], "tuned_us": head["tuned_us"], "planned": head["planned_edges"],
                        "priced": head["edge_costs"]},
        # makespan per program, each against serial
        "relay_breakdown": head["breakdown"],
        "best_ms": {"serial": round(serial["best_us"] / 1e3, 3), "split": round(split["best_us"] / 1e3, 3)},
        "op_avg_us": {"serial": serial.get("op_avg_us"), "split": split.get("op_avg_us")},
        "prefill_tflops": round(flops / 1e12, 3),
        "prefill_mfma_frac": round(flops / (total_split_s / args.steps) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "roofline": roof,
        "cpu_baseline": cpu,
        "configs": extra or None,
        "dag": dag,
        "bit_exact_serial_vs_split": True,
        "argmax": split["argmax"], "flag_edges": split["flag_edges"], "flag_timeouts": split["flag_timeouts"],
    }
    print(json.dumps(out), flush=True)


# the other prefill configurations the reference publishes (RESULTS.md:20,23),
# run serial and split after the headline
EXTRA_CONFIGS = (("qwen2.5-0.5b", 2048), ("qwen3-8b", 4096))


def model_dir_path():
    base = "/dev/shm" if os.path.isdir("/dev/shm") and shutil.disk_usage("/dev/shm").free > 40e9 else None
    return Path(tempfile.mkdtemp(prefix="kr_bench_", dir=base))


def choose_edges(model_dir, S, k):
    """Price the relay split's flag edges on this card (kr_qwen_profile_many:
    each relayed launch at k tiles, and the GEMM, Add+RMSNorm pair it
    replaces) and keep those that pay (planner.relay_edges)."""
    from kernrelay_amd import libapi, planner
    cases = [{"op": "matmul_o", "k": 1}, {"op": "matmul_down", "k": 1}, {"op": "add_rmsnorm", "k": 1},
             {"op": "matmul_o_add_rmsnorm_relay", "k": k}, {"op": "matmul_down_add_rmsnorm_relay", "k": k}]
    raw = libapi.qwen_profile_many(model_dir, cases, seq=S)
    if raw.get("_rc") not in (None, 0):
        raise RuntimeError("kr_qwen_profile_many failed: %s" % raw.get("error"))
    launch_us = json.loads(planner.COSTS_PATH.read_text())["launch_us"]
    return planner.relay_edges(planner.profile_table(raw), k, launch_us)


def run_program(model_dir, name, mode, env, S, steps, warmup):
    log("kr_qwen_run %s %s %s (warmup %d, steps %d)" % (name, mode, env or "", warmup, steps))
    from kernrelay_amd import libapi
    saved = {key: os.environ.get(key) for key in env}
    os.environ.update(env)
    try:
        r = libapi.qwen_run(model_dir, mode=mode, seq=S, device=0, warmup=warmup, iters=steps)
    finally:
        for key, v in saved.items():
            if v is None:
                os.environ.pop(key, None)
            else:
                os.environ[key] = v
    if r.get("_rc") != 0:
        raise RuntimeError("%s failed: %s" % (name, r.get("error")))
    log("  best %.1f us typical %.1f us argmax %s flag edges %s timeouts %s" % (
        r["best_us"], r["typical_us"], r["argmax"], r["flag_edges"], r["flag_timeouts"]))
    if r["flag_timeouts"] != 0:
        raise RuntimeError("%s: %d flag waits timed out" % (name, r["flag_timeouts"]))
    return r


def prefill_config(model_dir, preset, S, k, steps, warmup, ablation, dump_logits):
    """One prefill configuration: write its model directory (unless there),
    run serial (graph_whole) and the relay split (relay_split:<k>: the
    library builds the program with every subset of the o / down flag edges,
    replays each in place and keeps the fastest), plus, with `ablation`, the
    split with no flag edge, with both, and both without the SwiGLU fusion;
    every program's logits must equal serial's bit for bit. The planner's
    pricing of the same edges from the per-op profile is reported beside the
    in-place choice."""
    import torch

    from kernrelay_amd import modeldir
    model_dir = Path(model_dir)
    if not (model_dir / "manifest.json").exists():
        t0 = time.time()
        log("writing %s model dir (seq %d) to %s" % (preset, S, model_dir))
        modeldir.write_model_dir(model_dir, preset, seq=S, device="cuda")
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        log("model dir written in %.1f s" % (time.time() - t0))
    planned, edge_costs = choose_edges(model_dir, S, k)
    log("%s: planner prices the relay edges %s -> %s" % (preset, json.dumps(edge_costs), planned or "none"))
    split_mode = "relay_split:%d" % k
    timing = {"KR_TIME_OPS": "1"}
    dump = None
    split_env = dict(timing)
    if dump_logits:
        split_env["KR_DUMP_DIR"] = str(model_dir)
        dump = model_dir / "last_logits_bf16.bin"
    runs = {name: run_program(model_dir, name, mode, env, S, steps, warmup)
            for name, mode, env in (("serial", "graph_whole", timing), ("split", split_mode, split_env))}
    chosen = runs["split"]["relay_edges"]
    log("%s: edges tuned in place %s -> %s" % (preset, json.dumps(runs["split"].get("relay_edges_tuned_us")), chosen))
    if ablation:
        # the split with no flag edge (the SwiGLU epilogue only), with both
        # flag edges, and both flag edges without the SwiGLU fusion
        plan = []
        if chosen != "none":
            plan.append(("fusion_only", "relay_split:%d:none" % k, timing))
        if chosen != "o+down":
            plan.append(("flag_relay_all", "relay_split:%d:o+down" % k, timing))
        plan.append(("flag_relay_only", "relay_split:%d:o+down" % k, dict(timing, KR_SPLIT_SWIGLU="kernel")))
        for name, mode, env in plan:
            runs[name] = run_program(model_dir, name, mode, env, S, steps, warmup)
        runs.setdefault("fusion_only", runs["split"])
        runs.setdefault("flag_relay_all", runs["split"])
    for name, r in runs.items():
        if r["logits_fnv64"] != runs["serial"]["logits_fnv64"]:
            raise RuntimeError("%s: %s logits differ from serial" % (preset, name))

    def ms(r):
        return round(sum(r["samples_us"]) / len(r["samples_us"]) / 1e3, 3)

    breakdown = {name: {"ms_per_step": ms(r), "vs_serial": round(ms(runs["serial"]) / ms(r), 4),
                        "flag_edges": r["flag_edges"], "relay_edges": r.get("relay_edges")}
                 for name, r in runs.items()}
    edges = [] if chosen == "none" else chosen.split("+")
    return {"runs": runs, "edges": edges, "edge_costs": edge_costs, "planned_edges": planned,
            "tuned_us": runs["split"].get("relay_edges_tuned_us"), "split_mode": split_mode,
            "breakdown": breakdown, "dump": dump}


def config_summary(r, S):
    serial, split = r["runs"]["serial"], r["runs"]["split"]
    ts = sum(serial["samples_us"]) / len(serial["samples_us"])
    tp = sum(split["samples_us"]) / len(split["samples_us"])
    return {"serial_ms": round(ts / 1e3, 3), "split_ms": round(tp / 1e3, 3),
            "serial_tok_s": round(S * 1e6 / ts, 1), "split_tok_s": round(S * 1e6 / tp, 1),
            "split_vs_serial": round(ts / tp, 4), "split_mode": r["split_mode"], "relay_edges": r["edges"],
            "relay_edges_tuned_us": r["tuned_us"], "relay_edges_planned": r["planned_edges"],
            "relay_edges_priced": r["edge_costs"], "flag_edges": split["flag_edges"],
            "flag_timeouts": split["flag_timeouts"], "argmax": split["argmax"], "bit_exact_serial_vs_split": True,
            "op_avg_us": split.get("op_avg_us")}


if __name__ == "__main__":
    main()
