"""Row-split planner over a measured cost table.

The planner decides which producer -> consumer edges of a prefill DAG to run
as k row tiles (the relay split) by simulating the engines' queues:

* ``layer_dag``      — the per-layer Qwen DAG the planner works on
                       (python/kernrelay/optimize.py:59-142).
* ``Costs``          — unsplit cost per op shape and the tax of k tiles
                       (python/kernrelay/planner2.py:50-166).
* ``simulate``       — list schedule, per-engine FIFO, tile-wise deps
                       (planner2.py:269-382).
* ``bubbles``        — engine idle time caused by a data dependency
                       (planner2.py:385-409).
* ``greedy_plan``    — bubble-driven split search (planner2.py:587-680).
* ``plan_dag``       — feeds a ``kr_qwen_profile_many`` table into the
                       search (optimize.py:179-237).

Tie-breaks, the candidate k sets and the tax formulas follow the reference
exactly, so the same DAG and cost table give the same schedule, makespan and
splits.  The schedule is built with a lazily re-keyed heap instead of a scan
over all pending tasks: a ready task's start key can only grow (engine free
times are monotone), so the first popped entry whose key is current is the
scan's minimum.
"""

import copy
import heapq
import json
import re
from collections import defaultdict
from pathlib import Path

ELEMENTWISE = frozenset({"gelu", "add", "silu", "mul", "cast", "softmax",
                         "layernorm", "rmsnorm", "rope", "custom_aicpu_scale"})
COMM = frozenset({"allreduce", "allgather", "reducescatter"})

# MI355X cost table shipped with the package (measured by
# kernrelay_amd.profile_model on one MI355X); see ``default_costs``.
COSTS_PATH = Path(__file__).resolve().parent / "costs_mi355x.json"


# --------------------------------------------------------------- DAG ----

def shape_key(node):
    """Cost-table key of a node (planner2.py:31-38)."""
    s, op = node["shape"], node["op"]
    if op == "matmul":
        return "matmul|%dx%dx%d" % (s["M"], s["K"], s["N"])
    if op == "attention":
        return "attention|%dx%dx%dx%d" % (s["batch"], s["q_heads"],
                                          s["seq"], s["head_dim"])
    return "%s|%dx%d" % (op, s.get("rows", 0), s.get("cols", 0))


def shape_bytes(node):
    """Bytes the roofline fallback charges for a node (planner2.py:41-47)."""
    s = node["shape"]
    if node["op"] == "matmul":
        return 2 * (s["M"] * s["K"] + s["K"] * s["N"] + s["M"] * s["N"])
    if node["op"] == "attention":
        return 2 * s["batch"] * s["q_heads"] * s["seq"] * s["head_dim"] * 3
    return 4 * s.get("rows", 0) * s.get("cols", 0)


def layer_dag(cfg, seq):
    """Qwen prefill as the planner sees it (optimize.py:59-142).

    ``cfg`` holds the manifest config keys (hidden_size, intermediate_size,
    num_hidden_layers, num_attention_heads, num_key_value_heads, vocab_size,
    head_dim, qk_norm).  GEMMs run on engine ``aic``, vector ops on ``aiv``
    and attention on ``aicore`` (it occupies both).
    """
    H, I = cfg["hidden_size"], cfg["intermediate_size"]
    L, V = cfg["num_hidden_layers"], cfg["vocab_size"]
    HQ, HKV = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    D = cfg.get("head_dim") or H // HQ
    qk = bool(cfg.get("qk_norm", False))
    nodes, edges = [], []

    def node(name, op, engine, **shape):
        nodes.append({"name": name, "op": op, "engine": engine,
                      "shape": shape, "dtype": "bf16"})

    def dep(src, dst):
        edges.append({"src": src, "dst": dst, "kind": "data"})

    def mm(name, M, K, N):
        node(name, "matmul", "aic", M=M, K=K, N=N)

    node("embed", "embedding", "aiv", rows=seq, cols=H)
    prev = "embed"
    for l in range(L):
        p = "l%d." % l
        node(p + "ln1", "rmsnorm", "aiv", rows=seq, cols=H)
        dep(prev, p + "ln1")
        mm(p + "q", seq, H, HQ * D)
        mm(p + "k", seq, H, HKV * D)
        mm(p + "v", seq, H, HKV * D)
        for x in "qkv":
            dep(p + "ln1", p + x)
        qsrc = p + "q"
        if qk:
            node(p + "qk_norm", "rmsnorm", "aiv", rows=seq * HQ, cols=D)
            dep(p + "q", p + "qk_norm")
            dep(p + "k", p + "qk_norm")
            qsrc = p + "qk_norm"
        node(p + "rope", "rope", "aiv", rows=seq, cols=HQ * D)
        dep(qsrc, p + "rope")
        node(p + "attn", "attention", "aicore", batch=1, q_heads=HQ,
             kv_heads=HKV, seq=seq, head_dim=D)
        dep(p + "rope", p + "attn")
        dep(p + "v", p + "attn")
        mm(p + "o", seq, HQ * D, H)
        dep(p + "attn", p + "o")
        node(p + "addnorm1", "add_rmsnorm", "aiv", rows=seq, cols=H)
        dep(prev, p + "addnorm1")
        dep(p + "o", p + "addnorm1")
        mm(p + "gate", seq, H, I)
        mm(p + "up", seq, H, I)
        dep(p + "addnorm1", p + "gate")
        dep(p + "addnorm1", p + "up")
        node(p + "silu", "silu", "aiv", rows=seq, cols=I)
        dep(p + "gate", p + "silu")
        node(p + "mul", "mul", "aiv", rows=seq, cols=I)
        dep(p + "silu", p + "mul")
        dep(p + "up", p + "mul")
        mm(p + "down", seq, I, H)
        dep(p + "mul", p + "down")
        node(p + "addnorm2", "add_rmsnorm", "aiv", rows=seq, cols=H)
        dep(p + "addnorm1", p + "addnorm2")
        dep(p + "down", p + "addnorm2")
        prev = p + "addnorm2"
    node("final_norm", "rmsnorm", "aiv", rows=seq, cols=H)
    dep(prev, "final_norm")
    mm("lm_head", seq, H, V)
    dep("final_norm", "lm_head")
    return {"name": "llm_" + cfg.get("arch", "qwen"), "nodes": nodes,
            "edges": edges}


def unique_ops(dag):
    """Distinct op shapes with counts and engines (optimize.py:145-163)."""
    seen = {}
    for n in dag["nodes"]:
        key = shape_key(n)
        e = seen.setdefault(key, {"key": key, "op": n["op"], "count": 0,
                                  "engines": set()})
        e["count"] += 1
        e["engines"].add(n["engine"])
    out = list(seen.values())
    for e in out:
        e["engines"] = sorted(e["engines"])
    out.sort(key=lambda x: (-x["count"], x["key"]))
    return out


def project_summary(dag, cfg, seq):
    """Inventory block of an optimize result (optimize.py:240-245)."""
    inv = unique_ops(dag)
    return {"arch": cfg.get("arch"), "seq": seq,
            "hidden": cfg.get("hidden_size"),
            "layers": cfg.get("num_hidden_layers"),
            "nodes": len(dag["nodes"]), "edges": len(dag["edges"]),
            "unique_shapes": len(inv), "inventory": inv}


# ------------------------------------------------------------- costs ----

_MM_KEY = re.compile(r"matmul\|(\d+)x(\d+)x(\d+)$")


class Costs:
    """Unsplit cost per shape (``full``) and the tax of splitting into k.

    ``table`` has the layout of a cost file: ``full`` {shape_key: us},
    ``launch_us``, ``traffic_gbps``, ``l2_mb``, ``event_us``.  ``curves``
    maps shape keys to measured split curves
    ``{"base_best_us", "fit": {"slope_us_per_tile", "intercept_us"}}``.
    Shapes missing from ``full`` are scaled from a measured shape with the
    same inner dimensions, else priced by a roofline (planner2.py:86-123).
    """

    def __init__(self, table, curves=None):
        self.data = table
        self.full = dict(table.get("full", {}))
        self.launch = float(table.get("launch_us", 8.0))
        self.bw = float(table.get("traffic_gbps", 600.0)) * 1e9
        self.l2 = float(table.get("l2_mb", 32.0)) * 1024 * 1024
        self.event = float(table.get("event_us", 20.0))
        self.curves = dict(curves or {})
        self._base = {}
        self._tax = {}

    @classmethod
    def from_files(cls, path, curves_path=None):
        """Cost file plus an optional curve file (``{"cases": [...]}``,
        planner2.py:60-73)."""
        table = json.loads(Path(path).read_text(encoding="utf-8"))
        curves = {}
        if curves_path and Path(curves_path).exists():
            raw = json.loads(Path(curves_path).read_text(encoding="utf-8"))
            for case in raw.get("cases", []):
                key = cls.curve_key(case)
                if key:
                    curves[key] = case
        return cls(table, curves)

    @staticmethod
    def curve_key(case):
        op, s = case.get("op"), case.get("shape") or {}
        if op in ("matmul", "attention"):
            return shape_key({"op": op, "shape": s})
        if s.get("rows") and s.get("cols"):
            return "%s|%dx%d" % (op, s["rows"], s["cols"])
        return None

    def base(self, node):
        key = shape_key(node)
        if key in self._base:
            return self._base[key]
        if key in self.full:
            val = self._base[key] = float(self.full[key])
            return val
        s, op = node["shape"], node["op"]
        if op == "custom_aicpu_scale":
            # host-side scalar op: 2.2 ns per element, not cached
            return max(1.0, s.get("rows", 0) * s.get("cols", 0) * 2.2e-3)
        if op == "matmul":
            for k, v in self.full.items():
                m = _MM_KEY.match(k)
                if m and int(m.group(2)) == s["K"] and int(m.group(3)) == s["N"]:
                    val = self._base[key] = float(v) * s["M"] / int(m.group(1))
                    return val
        else:
            pat = re.compile(re.escape(op) + r"\|(\d+)x(\d+)$")
            for k, v in self.full.items():
                if not k.startswith(op + "|"):
                    continue
                m = pat.match(k)
                if m and int(m.group(2)) == s.get("cols", 0):
                    val = float(v) * s.get("rows", 0) / max(int(m.group(1)), 1)
                    self._base[key] = val
                    return val
        hbm_us = shape_bytes(node) / self.bw * 1e6
        if op == "matmul":
            val = max(2.0 * s["M"] * s["K"] * s["N"] / 250e12 * 1e6, hbm_us)
        else:
            val = max(hbm_us, 1.0)
        self._base[key] = val
        return val

    def split_tax(self, node, strategy, k):
        """Extra time of k tiles over the unsplit op, plus one cross-stream
        sync per tile (planner2.py:125-159)."""
        if k <= 1:
            return 0.0
        ck = (shape_key(node), strategy, k)
        if ck in self._tax:
            return self._tax[ck]
        sync = k * self.event
        case = self.curves.get(shape_key(node))
        if case and case.get("fit"):
            fit = case["fit"]
            val = max(0.0, float(fit["slope_us_per_tile"]) * (k - 1)
                      + float(fit["intercept_us"]) - float(case["base_best_us"])
                      ) + sync
        elif strategy == "head":
            val = k * self.launch + sync
        elif strategy in ("col", "m2d"):
            s = node["shape"]
            c_mb = s["M"] * s["N"] * 2 / (1024.0 * 1024.0)
            val = k * self.launch + c_mb * 1.6 + sync
        else:
            reread = 0.0
            if node["op"] == "matmul":
                s = node["shape"]
                b_bytes = s["K"] * s["N"] * 2
                if b_bytes > self.l2:
                    reread = (k - 1) * b_bytes / self.bw * 1e6
            val = k * self.launch + reread + sync
        self._tax[ck] = val
        return val

    def split_total(self, node, strategy, k):
        return self.base(node) + self.split_tax(node, strategy, k)

    def tax_ratio(self, node, strategy, k):
        b = self.base(node)
        return self.split_tax(node, strategy, k) / b if b else 1.0


def default_costs():
    """The MI355X cost table shipped with the package, with the split curves
    derived from its k=1 and k=8 columns."""
    table = json.loads(COSTS_PATH.read_text(encoding="utf-8"))
    return Costs(table, table.get("curves"))


# ---------------------------------------------------------- schedule ----

def topo_rounds(nodes, edges):
    """Kahn levels: round r holds the nodes whose last predecessor is in
    round r-1, in node order (planner2.py:172-193).  Raises on a cycle."""
    names = [n["name"] for n in nodes]
    index = {n: i for i, n in enumerate(names)}
    indeg = {n: 0 for n in names}
    succ = defaultdict(list)
    for e in edges:
        indeg[e["dst"]] += 1
        succ[e["src"]].append(e["dst"])
    frontier = [n for n in names if indeg[n] == 0]
    rounds, node_round, seen = [], {}, 0
    while frontier:
        for n in frontier:
            node_round[n] = len(rounds)
        rounds.append(frontier)
        seen += len(frontier)
        nxt = set()
        for n in frontier:
            for v in succ[n]:
                indeg[v] -= 1
                if indeg[v] == 0:
                    nxt.add(v)
        frontier = sorted(nxt, key=index.__getitem__)
    if seen < len(names):
        raise ValueError("graph cycle")
    return rounds, node_round


def _resources(engine):
    return ("aic", "aiv") if engine == "aicore" else (engine,)


def row_ranges(total, k):
    """k proportional row ranges; boundaries use Python's round (half to
    even), as the reference does (planner2.py:208-210)."""
    b = [round(i * total / k) for i in range(k + 1)]
    return [(b[i], b[i + 1]) for i in range(k)]


def _overlaps(src_ranges, dst_ranges):
    return {j: [i for i, (c, d) in enumerate(src_ranges) if max(a, c) < min(b, d)]
            for j, (a, b) in enumerate(dst_ranges)}


def _split_extent(node, strategy):
    s = node["shape"]
    if strategy == "row" and node["op"] == "matmul":
        return s["M"]
    if strategy == "head":
        return s["q_heads"]
    return s.get("rows") or s.get("M") or 0


def tile_overlap(src, dst, sp_src, sp_dst):
    """Consumer tile -> producer tiles it reads (planner2.py:213-266).

    A consumer reading fewer rows than the producer writes (a partial
    collective) maps onto the head of the producer's range; equal k maps
    one to one; different strategies depend on every tile.
    """
    ks, kd = sp_src["k"], sp_dst["k"]
    dst_rows = dst["shape"].get("rows") or dst["shape"].get("M") or 0
    src_rows = src["shape"].get("M") or src["shape"].get("rows") or 0
    if dst_rows and src_rows and dst_rows < src_rows and sp_dst["strategy"] == "row":
        total = _split_extent(src, sp_src["strategy"]) or src_rows
        return _overlaps(row_ranges(total, ks),
                         row_ranges(min(total, dst_rows), kd))
    if ks == kd:
        return {j: [j] for j in range(kd)}
    if sp_src["strategy"] != sp_dst["strategy"]:
        return {j: list(range(ks)) for j in range(kd)}
    total = _split_extent(src, sp_src["strategy"])
    if not total:
        return {j: list(range(ks)) for j in range(kd)}
    return _overlaps(row_ranges(total, ks), row_ranges(total, kd))


def simulate(graph, costs, splits=None, topo=None):
    """List-schedule the DAG (planner2.py:269-382).

    A split node becomes k consecutive tasks on its engine; tile i of a
    consumer waits for the producer tiles ``tile_overlap`` names.  Of all
    tasks whose deps are done, the one that can start earliest runs next,
    ties broken by (topological round, tile, node order).
    """
    splits = splits or {}
    nodes = graph["nodes"]
    by_name = {n["name"]: n for n in nodes}
    if topo is None:
        rounds, node_round = topo_rounds(nodes, graph["edges"])
        order = {n["name"]: i for i, n in enumerate(nodes)}
    else:
        rounds, node_round, order = topo

    tasks, parts_of = {}, {}
    for n in nodes:
        name = n["name"]
        sp = splits.get(name)
        k = int(sp.get("k", 1)) if sp else 1
        if k <= 1:
            parts = [{"name": name, "tile": 0, "parts": 1,
                      "dur": costs.base(n), "strategy": "none"}]
        else:
            strategy = sp.get("strategy", "row")
            dur = costs.split_total(n, strategy, k) / k
            parts = [{"name": "%s#%d" % (name, i), "tile": i, "parts": k,
                      "dur": dur, "strategy": strategy} for i in range(k)]
        for i, p in enumerate(parts):
            p.update(node=n, engine=n["engine"], round=node_round[name],
                     order=order[name], deps=set(), data_preds=[])
            if i:
                p["deps"].add(parts[i - 1]["name"])
            tasks[p["name"]] = p
        parts_of[name] = parts

    def link(dst_part, src_part):
        dst_part["deps"].add(src_part["name"])
        dst_part["data_preds"].append(src_part["name"])

    for e in graph["edges"]:
        src, dst = e["src"], e["dst"]
        sp_s, sp_d = splits.get(src), splits.get(dst)
        ks = int(sp_s.get("k", 1)) if sp_s else 1
        kd = int(sp_d.get("k", 1)) if sp_d else 1
        s_parts, d_parts = parts_of[src], parts_of[dst]
        if ks <= 1:
            for dp in d_parts:
                link(dp, s_parts[0])
        elif kd <= 1:
            whole = {"strategy": sp_s.get("strategy", "row"), "k": 1}
            need = tile_overlap(by_name[src], by_name[dst], sp_s, whole)
            for i in need.get(0, range(ks)):
                link(d_parts[0], s_parts[i])
        else:
            need = tile_overlap(by_name[src], by_name[dst], sp_s, sp_d)
            for j, dp in enumerate(d_parts):
                for i in need.get(j, range(ks)):
                    link(dp, s_parts[i])

    waiting = {name: len(t["deps"]) for name, t in tasks.items()}
    succ = defaultdict(list)
    for name, t in tasks.items():
        for d in t["deps"]:
            succ[d].append(name)
    finish, engine_free = {}, defaultdict(float)

    def key_of(t, dfin):
        st = max(max(engine_free[r] for r in _resources(t["engine"])), dfin)
        return (st, t["round"], t["tile"], t["order"])

    ready_fin, heap = {}, []
    for name, t in tasks.items():
        if waiting[name] == 0:
            ready_fin[name] = 0.0
            heapq.heappush(heap, (key_of(t, 0.0), name))
    schedule = []
    while heap:
        key, name = heapq.heappop(heap)
        t = tasks[name]
        dfin = ready_fin[name]
        cur = key_of(t, dfin)
        if cur != key:
            heapq.heappush(heap, (cur, name))
            continue
        st = cur[0]
        efree = max(engine_free[r] for r in _resources(t["engine"]))
        en = st + t["dur"]
        finish[name] = en
        for r in _resources(t["engine"]):
            engine_free[r] = en
        critical = None
        if t["data_preds"]:
            critical = max(((d, finish[d]) for d in set(t["data_preds"])),
                           key=lambda x: x[1])
        schedule.append({
            "name": name, "node": t["node"]["name"], "tile": t["tile"],
            "parts": t["parts"], "engine": t["engine"], "round": t["round"],
            "start": st, "end": en, "dur": t["dur"], "ready": dfin,
            "engine_free": efree,
            "critical": critical[0] if critical else None,
            "critical_end": critical[1] if critical else 0.0,
            "deps": sorted(t["deps"]),
            "data_preds": sorted(set(t["data_preds"])),
        })
        for v in succ[name]:
            waiting[v] -= 1
            if waiting[v] == 0:
                ready_fin[v] = max(finish[d] for d in tasks[v]["deps"])
                heapq.heappush(heap, (key_of(tasks[v], ready_fin[v]), v))
    if len(finish) < len(tasks):
        missing = [n for n in tasks if n not in finish]
        raise ValueError("task graph cycle at %s" % missing[:5])
    schedule.sort(key=lambda x: (x["start"], x["engine"], x["name"]))
    makespan = max((s["end"] for s in schedule), default=0.0)
    return {"makespan_us": makespan, "tasks": schedule,
            "splits": copy.deepcopy(splits), "rounds": rounds}


def bubbles(sched):
    """Engine idle gaps caused by a data dependency, largest first
    (planner2.py:385-409)."""
    out = []
    per_engine = defaultdict(list)
    for t in sched["tasks"]:
        per_engine[t["engine"]].append(t)
    for engine, ts in per_engine.items():
        prev_end = 0.0
        for t in sorted(ts, key=lambda x: x["start"]):
            gap = t["ready"] - t["engine_free"]
            if gap > 1e-6 and t["critical"]:
                out.append({"engine": engine, "task": t["name"],
                            "node": t["node"], "tile": t["tile"],
                            "round": t["round"], "dep_gap_us": gap,
                            "engine_gap_us": t["start"] - prev_end,
                            "critical": t["critical"],
                            "critical_end": t["critical_end"],
                            "start": t["start"]})
            prev_end = max(prev_end, t["end"])
    out.sort(key=lambda x: -x["dep_gap_us"])
    return out


SUPPORTED_OPS = frozenset({"matmul", "attention", "embedding",
                           "custom_aicpu_scale"}) | ELEMENTWISE | COMM
ENGINES = ("aic", "aiv", "aicore", "aicpu", "hccl", "compute")
_ROWS_COLS = ("rows", "cols")
_DIMS = {"matmul": ("M", "K", "N"),
         "attention": ("batch", "seq", "q_heads", "kv_heads", "head_dim")}


def validate_graph(graph):
    """Structural checks before planning; a non-empty list of messages means
    the graph is rejected (python/kernrelay/planner_bench.py:16-77).

    The messages are the reference's own text, which its robustness summary
    (results/final/planner_robustness/summary.json) records as the reason.
    """
    nodes, edges = graph.get("nodes"), graph.get("edges")
    if not isinstance(nodes, list) or not nodes:
        return ["nodes 缺失或为空"]
    if not isinstance(edges, list):
        return ["edges 缺失"]
    errs = []
    names = [n.get("name") for n in nodes]
    if any(not n for n in names):
        errs.append("存在空节点名")
    if len(names) != len(set(names)):
        errs.append("节点名重复")
    known = set(names)
    for n in nodes:
        name, op = n.get("name", "?"), n.get("op")
        if op not in SUPPORTED_OPS:
            errs.append("%s: 不支持算子 %r" % (name, op))
            continue
        if n.get("engine") not in ENGINES:
            errs.append("%s: 非法引擎 %r" % (name, n.get("engine")))
        if op == "custom_aicpu_scale":
            continue
        s = n.get("shape") or {}
        try:
            for dim in _DIMS.get(op, _ROWS_COLS):
                if int(s.get(dim, 0)) <= 0:
                    errs.append("%s: %s %s<=0" % (name, op, dim))
            if op == "attention":
                q, kv = int(s.get("q_heads", 0)), int(s.get("kv_heads", 0))
                if q and kv and (q % kv or kv > q):
                    errs.append("%s: attention q_heads=%d 不是 kv_heads=%d 的整数倍"
                                % (name, q, kv))
        except (TypeError, ValueError) as ex:
            errs.append("%s: shape 非法 (%s)" % (name, ex))
    for e in edges:
        src, dst = e.get("src"), e.get("dst")
        if src not in known:
            errs.append("edge src 不存在: %r" % src)
        if dst not in known:
            errs.append("edge dst 不存在: %r" % dst)
        if src == dst:
            errs.append("自环: %s" % src)
    if not errs:
        try:
            topo_rounds(nodes, edges)
        except ValueError as ex:
            errs.append("依赖成环: %s" % ex)
    return errs


# ------------------------------------------------------------ search ----

def _base_name(task_name):
    return task_name.split("#")[0]


class _Graph:
    """Adjacency views of a planner graph."""

    def __init__(self, graph):
        self.graph = graph
        self.node = {n["name"]: n for n in graph["nodes"]}
        self.succ = defaultdict(list)
        self.pred = defaultdict(list)
        for e in graph["edges"]:
            self.succ[e["src"]].append(e["dst"])
            self.pred[e["dst"]].append(e["src"])

    def cross_engine(self, src, dst):
        return self.node[_base_name(src)]["engine"] != self.node[_base_name(dst)]["engine"]

    def chain_after(self, start, limit=3):
        """Same-engine single-successor chain of element-wise ops or GEMMs
        following ``start`` (planner2.py:420-436)."""
        engine = self.node[start]["engine"]
        chain, cur = [], start
        while len(chain) < limit:
            nxt = [v for v in self.succ.get(cur, []) if self.node[v]["engine"] == engine]
            if len(nxt) != 1:
                break
            v = nxt[0]
            if self.node[v]["op"] not in ELEMENTWISE and self.node[v]["op"] != "matmul":
                break
            chain.append(v)
            cur = v
        return chain

    def producers(self, dst, fallback):
        return list(self.pred.get(dst, [])) or [fallback]

    def fanout(self, producers):
        out = []
        for p in producers:
            out.extend(self.succ.get(p, []))
        return out


def candidate_ks(node):
    """Tile counts the search may try for a node (planner2.py:447-459)."""
    s = node["shape"]
    if node["op"] == "attention":
        h = int(s.get("q_heads", 0))
        return [k for k in (2, 4, 7, 8, 14) if h and h % k == 0]
    rows = int(s.get("M") or s.get("rows") or 0)
    if not rows:
        return []
    ks = [k for k in (2, 4, 8, 16) if rows % k == 0]
    if node["op"] == "matmul":
        ks = [k for k in ks if rows // k >= 1024]
    return ks


def _strategy(node):
    if node["op"] == "attention":
        return "head"
    if node["op"] == "matmul" or node["op"] in ELEMENTWISE or node["op"] in COMM:
        return "row"
    return None


def _split_set(g, base_splits, src, dst, kp, kc, chain):
    """Splits for one bubble: every producer of ``dst`` at kp; ``dst``, the
    producers' other consumers and the optional chain at kc
    (planner2.py:462-498).  None when a node cannot take its k."""
    trial = copy.deepcopy(base_splits)
    producers = g.producers(dst, src)
    pset = set(producers)
    names = list(dict.fromkeys(producers + [dst] + g.fanout(producers) + (chain or [])))
    for name in names:
        n = g.node[name]
        if n["op"] == "custom_aicpu_scale":
            if name in pset:
                return None
            continue
        k = kp if name in pset else kc
        strategy = _strategy(n)
        if strategy is None or k not in candidate_ks(n):
            return None
        trial[name] = {"strategy": strategy, "k": k}
    return trial


def _bubble_options(g, costs, cur, b, min_gain_us, topo=None):
    """Split options with positive gain for one bubble, best first
    (planner2.py:501-546)."""
    src, dst = _base_name(b["critical"]), b["node"]
    if g.node[src]["engine"] == g.node[dst]["engine"]:
        return []
    chain = g.chain_after(dst)
    producers = g.producers(dst, src)
    pset = set(producers)
    min_tax = 0.0
    for name in dict.fromkeys(producers + [dst] + g.fanout(producers)):
        n = g.node[name]
        if n["op"] == "custom_aicpu_scale" and name in pset:
            return []
        ks = candidate_ks(n)
        if not ks:
            return []
        min_tax += costs.split_tax(n, "head" if n["op"] == "attention" else "row", min(ks))
    if min_tax >= b["dep_gap_us"]:
        return []
    pairs = {(kp, kc) for kp in candidate_ks(g.node[src])
             for kc in candidate_ks(g.node[dst])}
    pairs = sorted(pairs, key=lambda x: (x[0] > x[1], x[0], x[1]))[:6]
    options = []
    for kp, kc in pairs:
        for with_chain in (False, True):
            trial = _split_set(g, cur["splits"], src, dst, kp, kc,
                               chain if with_chain else None)
            if not trial:
                continue
            try:
                s2 = simulate(g.graph, costs, trial, topo=topo)
            except (ValueError, KeyError):
                continue
            gain = cur["makespan_us"] - s2["makespan_us"]
            if gain >= min_gain_us:
                options.append((gain, (kp, kc), with_chain, trial, s2))
    options.sort(key=lambda x: -x[0])
    return options


def _union(t1, t2):
    """Merge two split sets; None when they disagree on a node."""
    trial = copy.deepcopy(t1)
    for name, spec in t2.items():
        if name in trial and trial[name] != spec:
            return None
        trial[name] = dict(spec)
    return trial


def _decision(rnd, b, options, accepted):
    best = options[0] if options else None
    return {"round": rnd, "consumer": b["node"], "engine": b["engine"],
            "critical_edge": "%s -> %s" % (b["critical"], b["node"]),
            "dep_gap_us": b["dep_gap_us"],
            "k": ("%d/%d" % best[1]) if best else None,
            "split_consumer_chain": best[2] if best else False,
            "predicted_gain_us": best[0] if best else 0.0,
            "alternatives": [{"k": "%d/%d" % o[1], "gain_us": o[0],
                              "split_chain": o[2]} for o in options],
            "accepted": accepted}


def greedy_plan(graph, costs, max_rounds=40, min_gain_us=1.0, top_options=3):
    """Bubble-driven split search (planner2.py:587-680).

    Each round: take the cross-engine dependency bubbles of the current
    schedule (one per distinct (op, shape, gap) signature, at most 8), price
    up to 12 split options per bubble by simulation, then accept the best
    single option or the best union of two options from different bubbles.
    Stops when no option gains ``min_gain_us``.

    Returns (splits, schedule, history, base_makespan_us, decisions).
    """
    g = _Graph(graph)
    nodes = graph["nodes"]
    rounds, node_round = topo_rounds(nodes, graph["edges"])
    topo = (rounds, node_round, {n["name"]: i for i, n in enumerate(nodes)})
    splits = {}
    cur = simulate(graph, costs, splits, topo=topo)
    base = cur["makespan_us"]
    history, decisions, tried = [], [], set()
    for rnd in range(max_rounds):
        cands, sigs = [], set()
        for b in bubbles(cur):
            if not g.cross_engine(b["critical"], b["node"]):
                continue
            if b["dep_gap_us"] < min_gain_us or (b["node"], b["critical"]) in tried:
                continue
            src, dst = g.node[_base_name(b["critical"])], g.node[b["node"]]
            sig = (src["op"], dst["op"],
                   json.dumps(src.get("shape", {}), sort_keys=True),
                   json.dumps(dst.get("shape", {}), sort_keys=True),
                   round(b["dep_gap_us"], 1))
            if sig not in sigs:
                sigs.add(sig)
                cands.append(b)
        if not cands:
            break
        per_bubble = []
        for b in cands[:8]:
            opts = _bubble_options(g, costs, cur, b, min_gain_us, topo=topo)
            if opts:
                per_bubble.append((b, opts))
        if not per_bubble:
            break
        best = None
        for b, opts in per_bubble:
            for o in opts[:top_options]:
                if best is None or o[0] > best[1]:
                    best = ([(b, o)], o[0], o[3], o[4])
        flat = sorted(((b, o) for b, opts in per_bubble for o in opts[:top_options]),
                      key=lambda x: -x[1][0])[:8]
        for i, (b1, o1) in enumerate(flat):
            for b2, o2 in flat[i + 1:]:
                if b1["node"] == b2["node"] and b1["critical"] == b2["critical"]:
                    continue
                trial = _union(o1[3], o2[3])
                if trial is None:
                    continue
                try:
                    s2 = simulate(graph, costs, trial)
                except (ValueError, KeyError):
                    continue
                gain = cur["makespan_us"] - s2["makespan_us"]
                if gain > best[1] + 1e-9:
                    best = ([(b1, o1), (b2, o2)], gain, trial, s2)
        chosen, gain, trial, s2 = best
        chosen_ids = {id(b) for b, _ in chosen}
        for b, opts in per_bubble:
            decisions.append(_decision(rnd, b, opts, id(b) in chosen_ids))
        labels = []
        for b, o in chosen:
            labels.append("k=%d/%d" % o[1] + ("+chain" if o[2] else ""))
            for name in o[3]:
                tried.add((name, b["critical"]))
        history.append({"round": rnd, "gain_us": gain, "k": ", ".join(labels),
                        "split_chain": any(o[2] for _, o in chosen),
                        "splits": copy.deepcopy(trial),
                        "bubble": chosen[0][0],
                        "bubbles": [{"consumer": b["node"], "critical": b["critical"]}
                                    for b, _ in chosen],
                        "makespan_us": s2["makespan_us"]})
        splits, cur = trial, s2
    return splits, cur, history, base, decisions


# ------------------------------------------------- profile -> planner ----

PROFILE_OPS = ("embedding", "rmsnorm", "add", "add_rmsnorm", "rope",
               "matmul_q", "matmul_k", "matmul_v", "attention", "matmul_o",
               "matmul_gate", "matmul_up", "silu", "mul", "matmul_down",
               "matmul_lm")


def profile_op(node):
    """``kr_qwen_profile_many`` op name that times a DAG node
    (optimize.py:193-207)."""
    if node["op"] == "matmul":
        tail = node["name"].rsplit(".", 1)[-1]
        if tail in ("q", "k", "v", "o", "gate", "up", "down"):
            return "matmul_" + tail
        return "matmul_lm" if tail == "lm_head" else "matmul"
    return node["op"]


def profile_table(raw):
    """op -> {k: best_us} from a ``kr_qwen_profile_many`` result
    (scripts/profile_model.py:30-34)."""
    table = {}
    for c in raw.get("cases", []):
        if "best_us" in c and "k" in c:
            table.setdefault(c["op"], {})[int(c["k"])] = float(c["best_us"])
    return table


def plan_dag(dag, profile, layers=None, base=None):
    """Plan a DAG from a profile table (optimize.py:179-237).

    ``profile["table"]`` maps op -> {k: best_us}, k keyed as an int or, after
    a JSON round trip, as a string.  The k=1 column replaces the base cost of
    every node the op times (nodes sharing a shape key take the last such
    op's value, in node order), and the (k=1, k=8) pair gives the op's split
    curve: slope (t8 - t1) / 7 per extra tile.  ``base`` is the cost file the
    table is laid over (default: the MI355X table shipped with the package).
    """
    base = dict(base if base is not None else
                json.loads(COSTS_PATH.read_text(encoding="utf-8")))
    full = dict(base.get("full", {}))
    table = profile["table"]

    def col(v, k):
        return v.get(k, v.get(str(k)))

    keys = {n["name"]: shape_key(n) for n in dag["nodes"]}
    for n in dag["nodes"]:
        v = table.get(profile_op(n)) or {}
        t1 = col(v, 1)
        if t1:
            full[keys[n["name"]]] = t1
    costs = Costs(dict(base, full=full))
    for n in dag["nodes"]:
        v = table.get(profile_op(n)) or {}
        t1, t8 = col(v, 1), col(v, 8)
        if not t1 or not t8:
            continue
        costs.curves[keys[n["name"]]] = {
            "op": n["op"], "strategy": "row", "shape": n["shape"],
            "base_best_us": t1,
            "fit": {"slope_us_per_tile": max(0.0, (t8 - t1) / 7.0),
                    "intercept_us": t1}}
    splits, cur, hist, base_m, decisions = greedy_plan(dag, costs, max_rounds=8)
    return {"base_makespan_us": base_m, "planned_makespan_us": cur["makespan_us"],
            "splits": splits, "history": hist, "decisions": decisions}


def main(argv=None):
    import argparse
    ap = argparse.ArgumentParser(description="plan relay splits for a Qwen "
                                 "model directory from a measured profile")
    ap.add_argument("--model", required=True, help="model dir (manifest.json)")
    ap.add_argument("--profile", required=True, help="profile JSON "
                    "(kernrelay_amd.profile_model --out)")
    ap.add_argument("--seq", type=int, default=None)
    ap.add_argument("--costs", default=None, help="base cost file")
    ap.add_argument("--out", default=None)
    args = ap.parse_args(argv)
    man = json.loads((Path(args.model) / "manifest.json").read_text())
    cfg, seq = man["config"], args.seq or man.get("seq", 2048)
    dag = layer_dag(cfg, seq)
    base = json.loads(Path(args.costs).read_text()) if args.costs else None
    plan = plan_dag(dag, json.loads(Path(args.profile).read_text()), cfg["num_hidden_layers"],
                    base=base)
    out = {"summary": project_summary(dag, cfg, seq),
           "plan": {k: plan[k] for k in ("base_makespan_us",
                                         "planned_makespan_us", "splits")},
           "history": [{k: h[k] for k in ("round", "k", "gain_us", "makespan_us",
                                          "splits")} for h in plan["history"]]}
    text = json.dumps(out, indent=1)
    if args.out:
        Path(args.out).write_text(text)
    print(json.dumps(out["plan"]))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
