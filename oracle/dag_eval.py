"""Node outputs of a schedule.json's DAG on the CPU — test infrastructure only.

Inputs follow the executor convention (oracle/dag_inputs.py; files named in
a node's "inputs" replace them); ops follow oracle/ops.py in the node's
storage dtype. All ops on the path are row-local, so the first `rows` rows of
every node can be computed alone (enough for the reference checksum, which
reads the first 8192 output words of each node, exec/exec_main.cpp:1292-1311).
"""

import math

import numpy as np
import torch

from . import dag_inputs as di
from . import ops

TORCH_DT = {"fp16": torch.float16, "bf16": torch.bfloat16}


def _dtype_name(s):
    s = (s or "fp16").lower()
    return {"float16": "fp16", "f16": "fp16", "fp16": "fp16", "bf16": "bf16", "bfloat16": "bf16",
            "fp32": "fp32", "float32": "fp32", "f32": "fp32"}[s]


def out_dtype(node):
    dt = _dtype_name(node.get("dtype"))
    if node["op"] == "cast":
        to = node.get("to")
        return _dtype_name(to) if to else ("fp32" if dt == "fp16" else "fp16")
    return dt


def _det(seed, n, dt):
    f = di.det_values(seed, n, dtype=None)
    return torch.from_numpy(f).to(TORCH_DT[dt]).to(torch.float32)


def _file(path, n, dt):
    w = np.fromfile(path, dtype=np.uint16)
    if w.size != n:
        raise ValueError("%s: %d elements, expected %d" % (path, w.size, n))
    return torch.from_numpy(w.view(np.int16).copy()).view(TORCH_DT[dt]).to(torch.float32)


def _input(node, role, n, seed, dt):
    files = node.get("inputs") or {}
    return _file(files[role], n, dt) if role in files else _det(seed, n, dt)


def _topo(nodes):
    done, order = set(), []
    pending = list(nodes)
    while pending:
        progressed = False
        for n in list(pending):
            if all(p in done for p in n.get("preds", [])):
                order.append(n)
                done.add(n["id"])
                pending.remove(n)
                progressed = True
        if not progressed:
            raise ValueError("DAG cycle")
    return order


def node_outputs(sched, rank=0, rows=None):
    """{node id: fp32 tensor [r, cols] of the stored output values}, r = rows
    (None = all rows)."""
    outs = {}
    for n in _topo(sched["nodes"]):
        op, dt = n["op"], _dtype_name(n.get("dtype"))
        tdt = TORCH_DT[dt]
        seed = di.node_seed(n["id"], rank)
        R, C = int(n["rows"]), int(n["cols"])
        r = R if rows is None else min(rows, R)
        preds = n.get("preds", [])
        in_cols = int(n["k"]) if op == "matmul" else C
        if preds:
            x = outs[preds[0]][:r]
        else:
            full = _input(n, "in", R * in_cols, (seed + 1) & 0xFFFFFFFF, dt).reshape(R, in_cols)
            x = full[:r]

        def second():
            if len(preds) > 1:
                return outs[preds[1]][:r]
            return _input(n, "x1", R * C, (seed + 3) & 0xFFFFFFFF, dt).reshape(R, C)[:r]

        def gamma():
            return _input(n, "gamma", C, (seed + 2) & 0xFFFFFFFF, dt)

        def beta():
            return _input(n, "beta", C, (seed + 3) & 0xFFFFFFFF, dt)

        eps = float(n.get("eps", 1e-5 if op == "layernorm" else 1e-6))
        if op == "matmul":
            K, N = int(n["k"]), int(n["n"])
            b = _input(n, "b", K * N, (seed + 2) & 0xFFFFFFFF, dt).reshape(K, N)
            y = ops.gemm(x, b, dt=tdt)
        elif op == "gelu":
            y = ops.gelu_tanh(x, tdt)
        elif op == "softmax":
            y = ops.softmax(x, tdt)
        elif op == "cast":
            odt = out_dtype(n)
            y = ops.cast(x, torch.float32 if odt == "fp32" else TORCH_DT[odt]).to(torch.float32)
        elif op == "silu":
            y = ops.silu(x, tdt)
        elif op == "mul":
            y = ops.mul(x, second(), tdt)
        elif op == "add":
            y = ops.add(x, second(), tdt)
        elif op == "swiglu":
            y = ops.swiglu(x, second(), tdt)
        elif op == "rmsnorm":
            y, _ = ops.rmsnorm(x, gamma(), eps, tdt)
        elif op == "add_rmsnorm":
            y, _, _ = ops.add_rmsnorm(x, second(), gamma(), eps, tdt)
        elif op == "layernorm":
            y = ops.layernorm(x, gamma(), beta(), eps, tdt)
        else:
            raise ValueError("op %s has no oracle" % op)
        outs[n["id"]] = y
    return outs


def output_words(node, values):
    """Stored bytes of an output as 16-bit words (fp32 outputs as 2 words each)."""
    odt = out_dtype(node)
    v = values.contiguous()
    if odt == "fp32":
        return v.numpy().astype(np.float32).view(np.uint16).reshape(-1)
    return v.to(TORCH_DT[odt]).view(torch.int16).numpy().view(np.uint16).reshape(-1)


def checksum(sched, nranks=None):
    """The executor checksum restated: sum over ranks and nodes of the first
    8192 16-bit output words (fp32 outputs read as fp16 halves)."""
    nranks = int(sched.get("nranks", 1)) if nranks is None else nranks
    total = 0.0
    need = 1
    for n in sched["nodes"]:
        words_per_row = int(n["cols"]) * (2 if out_dtype(n) == "fp32" else 1)
        need = max(need, math.ceil(8192 / words_per_row))
    for rank in range(nranks):
        outs = node_outputs(sched, rank, rows=need)
        for n in sched["nodes"]:
            w = output_words(n, outs[n["id"]])[:8192]
            odt = out_dtype(n)
            total += di.checksum_words(w, "bf16" if odt == "bf16" else "fp16")
    return total
