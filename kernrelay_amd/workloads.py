"""The mm -> consumer DAG workloads of the relay path, as DAG dicts plus
seeded input files for kr_plan_run.

* tiny mm->GELU: X[256,512] ~ N(0,1), W[512,512] ~ N(0,0.02), bf16, the
  producer split into 2 row tiles (the reference's e0-style DAG,
  dags/e0_tiny_mm_gelu.json, at the task's shapes and dtype);
* mm fan-out: X[4096,4096] ~ N(0,1), W[4096,4096] ~ N(0,0.02), bf16; every
  tile feeds row-softmax, GELU and a bf16->fp16 cast (the reference's 1:N
  fan-out, dags/f04_mm_fanout_c2.json, with the cast consumer added);
* the reference's own E3/E4 DAGs at their shapes and dtype (`e34_dag`).

Inputs are written once per (shape, seed) as raw bf16 files: X as [M, K],
W as the weight_t layout [K, N] the executor reads.
"""

from pathlib import Path

import torch

from . import schedule


def write_inputs(out_dir, M, K, N, seed=1234, x_std=1.0, w_std=0.02):
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    g = torch.Generator().manual_seed(seed)
    x = torch.empty(M, K).normal_(0.0, x_std, generator=g).to(torch.bfloat16)
    w = torch.empty(K, N).normal_(0.0, w_std, generator=g).to(torch.bfloat16)
    px, pw = out / ("x_%dx%d_s%d.bin" % (M, K, seed)), out / ("w_%dx%d_s%d.bin" % (K, N, seed))
    x.view(torch.int16).numpy().tofile(px)
    w.view(torch.int16).numpy().tofile(pw)
    return {"in": str(px), "b": str(pw)}


def mm_consumers_dag(name, M, K, N, consumers, dtype="bf16", inputs=None, cast_to="fp16"):
    """DAG dict: one matmul feeding each consumer op in `consumers`."""
    mm = {"name": "mm", "op": "matmul", "engine": "aic", "shape": {"M": M, "K": K, "N": N}, "dtype": dtype}
    if inputs:
        mm["inputs"] = dict(inputs)
    nodes = [mm]
    for op in consumers:
        node = {"name": op, "op": op, "engine": "aiv", "shape": {"rows": M, "cols": N}, "dtype": dtype}
        if op == "cast":
            node["to"] = cast_to
        nodes.append(node)
    edges = [{"src": "mm", "dst": op, "kind": "data"} for op in consumers]
    return {"name": name, "description": "mm -> %s" % ",".join(consumers), "nodes": nodes, "edges": edges}


def tiny_mm_gelu(out_dir, seed=1234):
    inputs = write_inputs(out_dir, 256, 512, 512, seed)
    return schedule.dag_from_dict(mm_consumers_dag("tiny_mm_gelu", 256, 512, 512, ["gelu"], inputs=inputs))


def mm_fanout(out_dir, M=4096, K=4096, N=4096, seed=1234, consumers=("softmax", "gelu", "cast")):
    inputs = write_inputs(out_dir, M, K, N, seed)
    return schedule.dag_from_dict(mm_consumers_dag("mm_fanout", M, K, N, list(consumers), inputs=inputs))


def e34_dag(name, consumers, M=32768, K=1024, N=2048):
    """The reference's E3/E4 relay DAGs (dags/f01_mm_gelu_c2.json,
    e3_mm_softmax.json, e3_mm_cast.json, f04_mm_fanout_c2.json): one fp16
    GEMM X[32768,1024] . W[1024,2048] feeding each consumer, deterministic
    inputs (the executor's DetValue), 4 tiles by default. `consumers` None:
    the reverse edge of dags/e3_ln_mm.json, a LayerNorm [32768, 2048]
    producer feeding a GEMM with K = N = 2048."""
    if consumers is None:
        return schedule.dag_from_dict({"name": name, "nodes": [
            {"name": "ln", "op": "layernorm", "engine": "aiv", "shape": {"rows": M, "cols": 2048},
             "dtype": "fp16", "tiles": 4},
            {"name": "mm", "op": "matmul", "engine": "aic", "shape": {"M": M, "K": 2048, "N": 2048},
             "dtype": "fp16", "tiles": 4}], "edges": [{"src": "ln", "dst": "mm", "kind": "data"}]})
    nodes = [{"name": "mm", "op": "matmul", "engine": "aic", "shape": {"M": M, "K": K, "N": N},
              "dtype": "fp16", "tiles": 4}]
    for c in consumers:
        nodes.append({"name": c, "op": c, "engine": "aiv", "shape": {"rows": M, "cols": N},
                      "dtype": "fp16", "tiles": 4})
    edges = [{"src": "mm", "dst": c, "kind": "data"} for c in consumers]
    return schedule.dag_from_dict({"name": name, "nodes": nodes, "edges": edges})


def e9_dag(name, M=32768):
    """The reference's two-wave DAGs on one device (dags/e9_two_waves.json,
    dags/e9_chain2.json), fp16, DetValue inputs, 4 tiles by default:
    e9_two_waves is two independent mm(32768x1024x2048) -> GELU chains;
    e9_chain2 is mm(K=1024) -> GELU -> mm(K=2048) -> GELU, the second GEMM
    reading the first GELU's output as its A operand."""
    def mm(node, K):
        return {"name": node, "op": "matmul", "engine": "aic", "shape": {"M": M, "K": K, "N": 2048},
                "dtype": "fp16", "tiles": 4}

    def gelu(node):
        return {"name": node, "op": "gelu", "engine": "aiv", "shape": {"rows": M, "cols": 2048},
                "dtype": "fp16", "tiles": 4}

    def edge(src, dst):
        return {"src": src, "dst": dst, "kind": "data"}

    if name == "e9_two_waves":
        nodes = [mm("mm1", 1024), gelu("gelu1"), mm("mm2", 1024), gelu("gelu2")]
        edges = [edge("mm1", "gelu1"), edge("mm2", "gelu2")]
    elif name == "e9_chain2":
        nodes = [mm("mm1", 1024), gelu("gelu1"), mm("mm2", 2048), gelu("gelu2")]
        edges = [edge("mm1", "gelu1"), edge("gelu1", "mm2"), edge("mm2", "gelu2")]
    else:
        raise ValueError("unknown one-device E9 DAG %r (e9_mixed needs an all-reduce)" % name)
    return schedule.dag_from_dict({"name": name, "nodes": nodes, "edges": edges})


def variants(dag, k, nranks=1):
    """serial (one stream), B0 (two streams, unsplit) and split-at-k schedules
    (the reference's E3/E4 variants, python/kernrelay/e34.py:16-22)."""
    chunking = {n.name: k for n in dag.nodes}
    return {
        "serial": schedule.serial_schedule(dag, nranks=nranks),
        "b0": schedule.build_fixed_schedule(dag, {}, nranks=nranks, method="B0-nosplit"),
        "split": schedule.build_fixed_schedule(dag, chunking, nranks=nranks, method="KernRelay-split"),
    }
