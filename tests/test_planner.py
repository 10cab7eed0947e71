"""Split planner: the reference's recorded plans, its TP-layer split search,
its robustness verdicts, and schedule properties fixed by the arithmetic.

Goldens (tests/golden/planner_goldens.json, written by
make_planner_goldens.py from the reference's result files):
* results/final/opt/*/optimize.json — base/planned makespan and splits of
  four models from their measured profile tables;
* results/final/tp_planner/summary.json — accepted splits, per-round gains
  and decisions of the search on the TP layer chain;
* results/final/planner_robustness/summary.json — accept/reject and reason.
"""

import copy
import json
import random
from pathlib import Path

import pytest

from kernrelay_amd import planner as P

GOLD = json.loads((Path(__file__).parent / "golden" / "planner_goldens.json")
                  .read_text(encoding="utf-8"))
MODELS = sorted(GOLD["opt"])


@pytest.mark.parametrize("model", MODELS)
def test_layer_dag_matches_recorded_inventory(model):
    rec = GOLD["opt"][model]
    dag = P.layer_dag(rec["config"], rec["seq"])
    summary = P.project_summary(dag, rec["config"], rec["seq"])
    for key in ("nodes", "edges", "unique_shapes", "inventory", "layers", "hidden"):
        assert summary[key] == rec["summary"][key], key


@pytest.mark.parametrize("model", MODELS)
def test_plan_dag_reproduces_recorded_plan(model):
    rec = GOLD["opt"][model]
    dag = P.layer_dag(rec["config"], rec["seq"])
    plan = P.plan_dag(dag, {"table": rec["profile_table"]}, base=GOLD["base_costs"])
    want = rec["plan"]
    assert plan["splits"] == want["splits"]
    assert plan["base_makespan_us"] == pytest.approx(want["base_makespan_us"], rel=1e-12)
    assert plan["planned_makespan_us"] == pytest.approx(want["planned_makespan_us"], rel=1e-12)


def test_plan_dag_reads_int_and_string_k_columns():
    rec = GOLD["opt"]["qwen2.5-0.5b"]
    dag = P.layer_dag(rec["config"], rec["seq"])
    as_int = {op: {int(k): v for k, v in cols.items()}
              for op, cols in rec["profile_table"].items()}
    a = P.plan_dag(dag, {"table": rec["profile_table"]}, base=GOLD["base_costs"])
    b = P.plan_dag(dag, {"table": as_int}, base=GOLD["base_costs"])
    assert a["base_makespan_us"] == b["base_makespan_us"]


def _tp_case(rec):
    i = rec["inputs"]
    H, K, N = i["H"], i["K"], i["N"]
    full = dict(GOLD["base_costs"]["full"])
    full["matmul|2048x%dx%d" % (K, N)] = i["down_us"]
    full["allreduce|2048x%d" % H] = i["allreduce_us"]
    full["rmsnorm|2048x%d" % H] = i["rmsnorm_us"]
    curve = {"op": "allreduce", "strategy": "row", "shape": {"rows": 2048, "cols": H},
             "base_best_us": i["allreduce_us"],
             "fit": {"slope_us_per_tile": i["allreduce_slope_us"],
                     "intercept_us": i["allreduce_us"]}}
    costs = P.Costs(dict(GOLD["base_costs"], full=full), {"allreduce|2048x%d" % H: curve})
    graph = {"nodes": [
        {"name": "down", "op": "matmul", "engine": "aic", "shape": {"M": 2048, "K": K, "N": N}},
        {"name": "ar", "op": "allreduce", "engine": "hccl", "shape": {"rows": 2048, "cols": H}},
        {"name": "an", "op": "rmsnorm", "engine": "aiv", "shape": {"rows": 2048, "cols": H}},
        {"name": "qkv", "op": "matmul", "engine": "aic", "shape": {"M": 2048, "K": H, "N": H}}],
        "edges": [{"src": "down", "dst": "ar"}, {"src": "ar", "dst": "an"},
                  {"src": "an", "dst": "qkv"}]}
    return graph, costs


@pytest.mark.parametrize("tag", sorted(GOLD["tp"]))
def test_tp_layer_search_reproduces_recorded_splits(tag):
    rec = GOLD["tp"][tag]
    graph, costs = _tp_case(rec)
    splits, cur, hist, base, decisions = P.greedy_plan(graph, costs, max_rounds=10)
    want = rec["expected"]
    assert splits == want["splits"]
    assert base == pytest.approx(want["base_layer_us"], rel=1e-12)
    assert cur["makespan_us"] == pytest.approx(want["planned_layer_us"], rel=1e-12)
    got_hist = [(h["round"], h["k"], h["splits"]) for h in hist]
    assert got_hist == [(h["round"], h["k"], h["splits"]) for h in want["history"]]
    for g, w in zip(hist, want["history"]):
        assert g["gain_us"] == pytest.approx(w["gain_us"], rel=1e-12)
    assert len(decisions) == len(want["decisions"])
    for g, w in zip(decisions, want["decisions"]):
        assert (g["consumer"], g["critical_edge"], g["k"], g["accepted"]) == \
            (w["consumer"], w["critical_edge"], w["k"], w["accepted"])
        assert g["dep_gap_us"] == pytest.approx(w["dep_gap_us"], rel=1e-12)
        assert g["predicted_gain_us"] == pytest.approx(w["predicted_gain_us"], rel=1e-12)


def _node(name, op, engine, shape):
    return {"name": name, "op": op, "engine": engine, "shape": shape}


def _problem_graphs():
    """The reference's problem DAGs (python/kernrelay/planner_bench.py:85-128)."""
    base = {"nodes": [_node("ln", "rmsnorm", "aiv", {"rows": 2048, "cols": 896}),
                      _node("mm", "matmul", "aic", {"M": 2048, "K": 896, "N": 896})],
            "edges": [{"src": "ln", "dst": "mm"}]}
    out = {}
    g = copy.deepcopy(base)
    g["nodes"].append(_node("x", "add", "aiv", {"rows": 2048, "cols": 896}))
    g["edges"].append({"src": "mm", "dst": "ln"})
    out["bad_cycle"] = g
    g = copy.deepcopy(base)
    g["nodes"][1]["op"] = "frobnicate"
    out["bad_unknown_op"] = g
    g = copy.deepcopy(base)
    g["nodes"][1]["shape"]["M"] = 0
    out["bad_shape"] = g
    g = copy.deepcopy(base)
    g["edges"].append({"src": "mm", "dst": "missing"})
    out["bad_edge"] = g
    g = copy.deepcopy(base)
    g["nodes"].append(copy.deepcopy(g["nodes"][0]))
    out["bad_dup_name"] = g
    out["bad_attention"] = {"nodes": [_node("attn", "attention", "aicore",
                                            {"batch": 1, "seq": 2048, "q_heads": 14,
                                             "kv_heads": 3, "head_dim": 64})], "edges": []}
    out["aicpu_producer"] = {"nodes": [
        _node("cpu", "custom_aicpu_scale", "aicpu", {"rows": 2048, "cols": 896}),
        _node("mm", "matmul", "aic", {"M": 2048, "K": 896, "N": 896})],
        "edges": [{"src": "cpu", "dst": "mm"}]}
    out["tiny_matmul"] = {"nodes": [_node("mm", "matmul", "aic",
                                          {"M": 512, "K": 1024, "N": 1024})], "edges": []}
    return out


def test_validate_graph_matches_robustness_rows():
    graphs = dict(GOLD["robustness"]["dags"])
    graphs.update(_problem_graphs())
    for row in GOLD["robustness"]["rows"]:
        errs = P.validate_graph(graphs[row["name"]])
        assert (not errs) == row["accepted"], row["name"]
        assert "; ".join(errs) == row["reason"], row["name"]


@pytest.mark.parametrize("name", ["aicpu_producer", "tiny_matmul"])
def test_valid_graphs_without_profitable_split_plan_zero_splits(name):
    g = _problem_graphs()[name]
    splits, _, hist, _, _ = P.greedy_plan(g, P.Costs(GOLD["base_costs"]))
    assert splits == {} and hist == []


# ---- properties the arithmetic fixes (not taken from the reference) ----

def _free_costs(full):
    """No launch, sync or re-read tax: a split costs nothing extra."""
    return P.Costs({"full": full, "launch_us": 0.0, "event_us": 0.0,
                    "traffic_gbps": 1e12, "l2_mb": 1e9})


def test_one_engine_chain_is_the_sum():
    g = {"nodes": [_node("a", "add", "aiv", {"rows": 64, "cols": 8}),
                   _node("b", "mul", "aiv", {"rows": 64, "cols": 8}),
                   _node("c", "silu", "aiv", {"rows": 64, "cols": 8})],
         "edges": [{"src": "a", "dst": "b"}, {"src": "b", "dst": "c"}]}
    c = _free_costs({"add|64x8": 3.0, "mul|64x8": 5.0, "silu|64x8": 7.0})
    assert P.simulate(g, c)["makespan_us"] == 15.0


@pytest.mark.parametrize("k", [2, 4, 8])
def test_tile_pipeline_closed_form(k):
    """Producer p on one engine, consumer c (c <= p) on another, both split
    into k equal tiles with tile i waiting on tile i: makespan p + c/k."""
    g = {"nodes": [_node("mm", "matmul", "aic", {"M": 4096, "K": 64, "N": 64}),
                   _node("ge", "gelu", "aiv", {"rows": 4096, "cols": 64})],
         "edges": [{"src": "mm", "dst": "ge"}]}
    p, c = 800.0, 240.0
    costs = _free_costs({"matmul|4096x64x64": p, "gelu|4096x64": c})
    sp = {"mm": {"strategy": "row", "k": k}, "ge": {"strategy": "row", "k": k}}
    assert P.simulate(g, costs)["makespan_us"] == p + c
    assert P.simulate(g, costs, sp)["makespan_us"] == pytest.approx(p + c / k, rel=1e-12)


def test_attention_holds_both_engines():
    g = {"nodes": [_node("at", "attention", "aicore", {"batch": 1, "q_heads": 4, "kv_heads": 4,
                                                         "seq": 64, "head_dim": 64}),
                   _node("x", "add", "aiv", {"rows": 8, "cols": 8}),
                   _node("m", "matmul", "aic", {"M": 8, "K": 8, "N": 8})], "edges": []}
    c = _free_costs({"attention|1x4x64x64": 10.0, "add|8x8": 4.0, "matmul|8x8x8": 6.0})
    # add and matmul overlap each other but not the attention: 10 + max(4, 6)
    assert P.simulate(g, c)["makespan_us"] == 16.0


def test_row_ranges_and_uneven_overlap():
    assert P.row_ranges(10, 4) == [(0, 2), (2, 5), (5, 8), (8, 10)]  # round half to even
    src = _node("mm", "matmul", "aic", {"M": 12, "K": 4, "N": 4})
    dst = _node("g", "gelu", "aiv", {"rows": 12, "cols": 4})
    m = P.tile_overlap(src, dst, {"strategy": "row", "k": 2}, {"strategy": "row", "k": 3})
    assert m == {0: [0], 1: [0, 1], 2: [1]}
    part = _node("ar", "allreduce", "hccl", {"rows": 4, "cols": 4})
    m = P.tile_overlap(src, part, {"strategy": "row", "k": 3}, {"strategy": "row", "k": 2})
    assert m == {0: [0], 1: [0]}   # first 4 rows live in producer tile 0


def _scan_schedule(graph, costs, splits):
    """Plain O(n^2) list scheduler: among tasks whose deps are done, start
    the one with the smallest (start, round, tile, node order)."""
    sched = P.simulate(graph, costs, splits)   # for the task set and deps only
    tasks = {t["name"]: t for t in sched["tasks"]}
    order = {n["name"]: i for i, n in enumerate(graph["nodes"])}
    res = {"aicore": ("aic", "aiv")}
    finish, free, out = {}, {}, {}
    while len(finish) < len(tasks):
        best = None
        for name, t in tasks.items():
            if name in finish or any(d not in finish for d in t["deps"]):
                continue
            rs = res.get(t["engine"], (t["engine"],))
            st = max([free.get(r, 0.0) for r in rs] + [finish[d] for d in t["deps"]])
            key = (st, t["round"], t["tile"], order[t["node"]])
            if best is None or key < best[0]:
                best = (key, name, rs)
        key, name, rs = best
        finish[name] = key[0] + tasks[name]["dur"]
        out[name] = key[0]
        for r in rs:
            free[r] = finish[name]
    return out, max(finish.values())


@pytest.mark.parametrize("seed", range(6))
def test_heap_schedule_equals_scan_schedule(seed):
    rnd = random.Random(seed)
    ops = [("matmul", "aic"), ("gelu", "aiv"), ("add", "aiv"), ("allreduce", "hccl"),
           ("attention", "aicore")]
    nodes, edges, full = [], [], {}
    for i in range(40):
        op, eng = rnd.choice(ops)
        if op == "matmul":
            shape = {"M": 4096, "K": 64 * (i + 1), "N": 64}
        elif op == "attention":
            shape = {"batch": 1, "q_heads": 8, "kv_heads": 8, "seq": 64 * (i + 1), "head_dim": 64}
        else:
            shape = {"rows": 4096, "cols": 8 * (i + 1)}
        n = _node("n%d" % i, op, eng, shape)
        nodes.append(n)
        full[P.shape_key(n)] = float(rnd.randint(1, 50))
        for j in rnd.sample(range(i), min(i, rnd.randint(0, 3))):
            edges.append({"src": "n%d" % j, "dst": n["name"]})
    g = {"nodes": nodes, "edges": edges}
    costs = P.Costs({"full": full})
    splits = {n["name"]: {"strategy": "head" if n["op"] == "attention" else "row",
                          "k": rnd.choice([2, 4])}
              for n in nodes if rnd.random() < 0.4}
    sched = P.simulate(g, costs, splits)
    starts, makespan = _scan_schedule(g, costs, splits)
    assert {t["name"]: t["start"] for t in sched["tasks"]} == starts
    assert sched["makespan_us"] == makespan


def test_cycle_rejected():
    g = {"nodes": [_node("a", "add", "aiv", {"rows": 1, "cols": 1}),
                   _node("b", "add", "aiv", {"rows": 1, "cols": 2})],
         "edges": [{"src": "a", "dst": "b"}, {"src": "b", "dst": "a"}]}
    with pytest.raises(ValueError):
        P.simulate(g, P.Costs({"full": {}}))


def test_shipped_mi355x_costs_cover_the_7b_dag():
    """The MI355X cost file prices every node of the Qwen2.5-7B seq-2048 DAG
    from measurement (no roofline fallback), and its own profile table plans
    the same way it was recorded."""
    from kernrelay_amd import modeldir
    costs = P.default_costs()
    table = json.loads(P.COSTS_PATH.read_text())
    assert table["device"] == "MI355X" and table["seq"] == 2048
    cfg = dict(modeldir.PRESETS["qwen2.5-7b"], arch="qwen2.5")
    dag = P.layer_dag(cfg, 2048)
    for n in dag["nodes"]:
        assert P.shape_key(n) in costs.full, P.shape_key(n)
    for key in ("matmul|2048x3584x18944", "matmul|2048x18944x3584", "matmul|2048x3584x152064"):
        assert key in costs.curves
    plan = P.plan_dag(dag, {"table": table["profile_table"]})
    sched = P.simulate(dag, costs)
    # the cost file keeps k=1 times to 1 ns, the profile table unrounded:
    # at most half a nanosecond per node of the DAG (all 28 layers' ops)
    assert abs(plan["base_makespan_us"] - sched["makespan_us"]) <= 0.5e-3 * len(dag["nodes"])
    # serial lower bound: the aic queue alone
    aic = sum(costs.base(n) for n in dag["nodes"] if n["engine"] in ("aic", "aicore"))
    assert plan["base_makespan_us"] >= aic


@pytest.mark.parametrize("preset", ["qwen2.5-7b", "qwen3-8b"])
def test_fused_layer_dag(preset):
    """The DAG of the program the runtime launches: per layer RMSNorm, one
    QKV projection (RoPE in its epilogue; a q/k RMSNorm and RoPE kernel after
    it where the model has q/k norms), attention, o, Add+RMSNorm, one gate/up
    projection (SwiGLU in its epilogue), down, Add+RMSNorm; the same GEMM
    work as the reference's DAG, without its RoPE, SiLU and Mul passes."""
    from kernrelay_amd import modeldir
    cfg = dict(modeldir.PRESETS[preset])
    H, I, L = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"]
    HQ, HKV = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    D = cfg.get("head_dim") or H // HQ
    qk = bool(cfg.get("qk_norm", False))
    ref, dag = P.layer_dag(cfg, 2048), P.layer_dag(cfg, 2048, fused=True)
    assert len(dag["nodes"]) == 3 + L * (8 + 2 * qk)
    ops = [n["op"] for n in dag["nodes"]]
    assert "silu" not in ops and "mul" not in ops and ops.count("rope") == (L if qk else 0)
    names = {n["name"]: n for n in dag["nodes"]}
    assert names["l0.qkv"]["shape"] == {"M": 2048, "K": H, "N": (HQ + 2 * HKV) * D}
    assert names["l0.gate_up"]["shape"] == {"M": 2048, "K": H, "N": 2 * I}
    assert P.profile_op(names["l0.qkv"]) == "matmul_qkv" and P.profile_op(names["l0.gate_up"]) == "matmul_gate_up"
    edges = {(e["src"], e["dst"]) for e in dag["edges"]}
    assert ("l0.gate_up", "l0.down") in edges and ("l0.addnorm1", "l0.gate_up") in edges
    assert (("l0.rope", "l0.attn") if qk else ("l0.qkv", "l0.attn")) in edges
    for e in dag["edges"]:
        assert e["src"] in names and e["dst"] in names

    def flops(d):
        return sum(2 * n["shape"]["M"] * n["shape"]["K"] * n["shape"]["N"] for n in d["nodes"] if n["op"] == "matmul")
    assert flops(dag) == flops(ref)


def test_relay_edges_taken_only_where_they_pay():
    """An o / down flag edge is kept only where its one relayed launch beats
    the GEMM, the Add+RMSNorm kernel and one more launch; the mode string
    names the edges kept."""
    table = {"matmul_o": {1: 55.0}, "matmul_down": {1: 248.0}, "add_rmsnorm": {1: 12.0},
             "matmul_o_add_rmsnorm_relay": {4: 60.0}, "matmul_down_add_rmsnorm_relay": {"4": 265.0}}
    edges, detail = P.relay_edges(table, 4, launch_us=2.0)
    assert edges == ["o"]
    assert detail["o"] == {"relay_us": 60.0, "unrelayed_us": 69.0, "gain_us": 9.0}
    assert detail["down"]["gain_us"] == -3.0
    assert P.relay_mode(table, 4, 2.0) == "relay_split:4:o"
    # at k = 2 nothing is priced: no edge, mode "none"
    assert P.relay_edges(table, 2) == ([], {})
    assert P.relay_mode(table, 2) == "relay_split:2:none"
    table["matmul_down_add_rmsnorm_relay"][4] = 200.0
    assert P.relay_mode(table, 4, 2.0) == "relay_split:4:o+down"
