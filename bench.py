"""Headline benchmark: Qwen2.5-7B-shaped bf16 prefill at seq 2048 on one
MI355X through kr_qwen_run — serial (graph_whole) vs relay split at 4 tiles —
plus the producer GEMM's roofline and the CPU (oracle) baseline.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--tiles 4] [--preset qwen2.5-7b]

Prints ONE JSON line. A step is one full prefill (28 layers + lm_head over all
2048 rows) with weights and inputs resident in HBM; `value` is tokens/s of the
relay-split prefill over exactly K timed steps (each step bracketed by device
synchronisation inside the library). Weights are random-init N(0, 0.02)
(`data: synthetic`): no checkpoint can be fetched on this pool.
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
GATE_UP_TRAFFIC_BYTES = (423136.0 * 2.0 + 75776.0 * 1.0) * 1024
GATE_UP_MFMA_UTIL = 0.635
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
    """The host CPU's model name (/proc/cpuinfo), or the platform's."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or platform.machine()


def cpu_baseline(model_dir, seconds_hint=20):
    """Oracle (fp32 torch CPU) on a bounded sample: decoder layer 0 and the
    lm_head over all rows at seq 2048; scaled to the full prefill as
    L * t_layer + t_lm_head."""
    import torch

    from oracle import ops as O
    from oracle import qwen as oq

    # the CPU share this process may use (affinity), at most 16 threads
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    torch.set_num_threads(threads)
    m = oq.ModelDir(model_dir)
    ids = m.ids()
    S = ids.numel()
    cos, sin = m.rope(S)
    with torch.no_grad():
        h = O.embedding(m.tensor("embed.weight"), ids)
        x, _ = O.rmsnorm(h, m.tensor("L00.input_layernorm.weight"), m.eps)
        t0 = time.perf_counter()
        h2, d = oq.layer_forward(m, 0, h, x, cos, sin)
        x, h, _ = O.add_rmsnorm(h2, d, m.tensor("L01.input_layernorm.weight"), m.eps)
        t_layer = time.perf_counter() - t0
        w = m.tensor("lm_head.weight_t")
        t0 = time.perf_counter()
        O.gemm(x, w)
        t_lm = time.perf_counter() - t0
    total = m.L * t_layer + t_lm
    return {"value": round(S / total, 2), "unit": "tok/s", "cores": threads, "cpu_model": cpu_model(), "kind": "port",
            "sample": "oracle fp32 torch-CPU: decoder layer 0 (%.2f s) + lm_head over %d rows (%.2f s) "
                      "at seq %d, scaled to %d layers" % (t_layer, S, t_lm, S, m.L),
            "ms_per_prefill_est": round(total * 1e3, 1)}


def profile_gemm(M, N, K, reps):
    """One producer-GEMM launch per repetition on random bf16 inputs: the
    program the rocprofv3 --pmc passes of the roofline's traffic run."""
    import torch

    from kernrelay_amd import ops

    g = torch.Generator(device="cuda").manual_seed(7)
    A = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    Bt = (torch.randn(N, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    C = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    for _ in range(reps):
        ops.gemm(A, Bt, C)
    torch.cuda.synchronize()
    print("gemm %dx%dx%d x%d done" % (M, N, K, reps), flush=True)


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
                    help="skip the fusion-only and flag-relay-only programs")
    ap.add_argument("--keep", default=None, help="keep / reuse the model directory here")
    ap.add_argument("--profile-gemm", nargs=3, type=int, metavar=("M", "N", "K"),
                    help="only launch the producer GEMM --reps times (for rocprofv3 --pmc)")
    ap.add_argument("--profile-gemm-swiglu", nargs=3, type=int, metavar=("M", "I", "K"),
                    help="only launch the gate/up GEMM with SwiGLU epilogue --reps times (for rocprofv3 --pmc)")
    ap.add_argument("--profile-copy", type=int, metavar="MIB", help="only copy MIB MiB --reps times")
    ap.add_argument("--profile-consumers", action="store_true",
                    help="only launch the consumer kernels and attention --reps times (for rocprofv3 --pmc)")
    ap.add_argument("--reps", type=int, default=3)
    args = ap.parse_args()
    if args.profile_gemm:
        profile_gemm(*args.profile_gemm, args.reps)
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
    base = "/dev/shm" if os.path.isdir("/dev/shm") and shutil.disk_usage("/dev/shm").free > 40e9 else None
    tmp = Path(args.keep) if args.keep else Path(tempfile.mkdtemp(prefix="kr_bench_", dir=base))
    try:
        if not (tmp / "manifest.json").exists():
            t0 = time.time()
            log("writing %s model dir (seq %d) to %s" % (args.preset, S, tmp))
            modeldir.write_model_dir(tmp, args.preset, seq=S, device="cuda")
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
            log("model dir written in %.1f s" % (time.time() - t0))
        runs = {}
        os.environ["KR_TIME_GATE_UP"] = "1"
        split_mode = "relay_split:%d" % args.tiles
        # serial; the relay split as shipped (o and down release k row tiles
        # to Add+RMSNorm through device flags, SwiGLU in the gate/up
        # epilogue); and two ablations separating the flag relays from the
        # epilogue fusion
        plan = [("serial", "graph_whole", {}), ("split", split_mode, {})]
        if not args.no_ablation:
            plan += [("fusion_only", split_mode, {"KR_SPLIT_NORM": "0"}),
                     ("flag_relay_only", split_mode, {"KR_SPLIT_SWIGLU": "kernel"})]
        for name, mode, env in plan:
            log("kr_qwen_run %s %s %s (warmup %d, steps %d)" % (name, mode, env or "", args.warmup, args.steps))
            saved = {k: os.environ.get(k) for k in env}
            os.environ.update(env)
            try:
                r = libapi.qwen_run(tmp, mode=mode, seq=S, device=0, warmup=args.warmup, iters=args.steps)
            finally:
                for k, v in saved.items():
                    if v is None:
                        os.environ.pop(k, None)
                    else:
                        os.environ[k] = v
            if r.get("_rc") != 0:
                raise RuntimeError("%s failed: %s" % (name, r.get("error")))
            log("  best %.1f us typical %.1f us argmax %s flag edges %s timeouts %s" % (
                r["best_us"], r["typical_us"], r["argmax"], r["flag_edges"], r["flag_timeouts"]))
            if r["flag_timeouts"] != 0:
                raise RuntimeError("%s: %d flag waits timed out" % (name, r["flag_timeouts"]))
            runs[name] = r
        serial, split = runs["serial"], runs["split"]
        for name, r in runs.items():
            if r["logits_fnv64"] != serial["logits_fnv64"]:
                raise RuntimeError("%s logits differ from serial" % name)
        I, H = cfg["intermediate_size"], cfg["hidden_size"]
        roof = gemm_roofline(split, serial, S, 2 * I, H)
        total_split_s = sum(split["samples_us"]) / 1e6
        total_serial_s = sum(serial["samples_us"]) / 1e6
        value = args.steps * S / total_split_s
        flops = modeldir.model_flops(cfg, S)
        dag = None
        if not args.no_dag:
            from kernrelay_amd import dag_bench
            log("DAG workloads: tiny mm->GELU, 4096^3 mm -> {softmax, gelu, cast} at k=1,2,4,8, the reference's "
                "E3/E4 and two-wave DAGs")
            dag = dag_bench.run_all()
        cpu = None
        if not args.no_cpu:
            log("cpu baseline (oracle, bounded sample)")
            cpu = cpu_baseline(tmp)
        relay = split["flag_edges"] > 0
        if relay:
            workload = ("%s-shaped prefill, batch 1, seq %d: relay split, o and down projections each releasing %d "
                        "row tiles to their Add+RMSNorm through device flags (%d flag edges per prefill), SwiGLU "
                        "fused into the gate/up GEMM epilogue" % (PRESET_NAMES.get(args.preset, args.preset), S,
                                                                   args.tiles, split["flag_edges"]))
        else:
            workload = ("%s-shaped prefill, batch 1, seq %d: serial program with SwiGLU fused into the gate/up "
                        "GEMM epilogue (no flag relay at this shape)" % (PRESET_NAMES.get(args.preset, args.preset), S))

        def ms(r):
            return round(sum(r["samples_us"]) / len(r["samples_us"]) / 1e3, 3)

        breakdown = {name: {"ms_per_step": ms(r), "vs_serial": round(ms(serial) / ms(r), 4),
                            "flag_edges": r["flag_edges"]} for name, r in runs.items()}
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
                       "parallelism": "none (1 GPU)", "relay_tiles": args.tiles if relay else None},
            "serial_ms_per_step": round(total_serial_s * 1e3 / args.steps, 3),
            "serial_tok_s": round(args.steps * S / total_serial_s, 1),
            "split_vs_serial": round(total_serial_s / total_split_s, 4),
            # makespan per program, each against serial: the flag relays alone
            # (SwiGLU as the serial kernel), the epilogue fusion alone (o and
            # down in stream order), and both (the split as shipped)
            "relay_breakdown": breakdown,
            "best_ms": {"serial": round(serial["best_us"] / 1e3, 3), "split": round(split["best_us"] / 1e3, 3)},
            "prefill_tflops": round(flops / 1e12, 3),
            "prefill_mfma_frac": round(flops / (total_split_s / args.steps) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "roofline": roof,
            "cpu_baseline": cpu,
            "dag": dag,
            "bit_exact_serial_vs_split": True,
            "argmax": split["argmax"], "flag_edges": split["flag_edges"], "flag_timeouts": split["flag_timeouts"],
        }
        print(json.dumps(out), flush=True)
    finally:
        if not args.keep:
            shutil.rmtree(tmp, ignore_errors=True)


if __name__ == "__main__":
    main()
