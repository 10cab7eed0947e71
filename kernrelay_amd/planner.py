"""Row-split planner over a measured cost table.

The planner decides which producer -> consumer edges of a prefill DAG to run
as k row tiles (the relay split) by simulating the engines' queues:

* ``layer_dag``      — the per-layer Qwen DAG the planner works on (the
                       reference's python/kernrelay/optimize.py:59-142).
* ``Costs``          — unsplit cost per op shape and the tax of k tiles.
* ``simulate``       — event-loop list schedule over a heap, per-engine
                       queues, tile-wise dependencies.
* ``bubbles``        — engine idle time caused by a data dependency.
* ``greedy_plan``    — bubble-driven split search (``_SplitSearch``).
* ``plan_dag``       — feeds a ``kr_qwen_profile_many`` table into the
                       search (optimize.py:179-237).

The code is this package's own; what it shares with the reference's planner
(python/kernrelay/planner2.py) is what a recorded plan depends on: the
cost-file fields and fallback constants, the split-tax rules, the candidate
tile counts, the tile-overlap rules, the order in which ready tasks, bubbles
and options are considered, and validate_graph's messages. With those the
same DAG and cost table give the reference's schedule, makespan, splits and
decisions (tests/test_planner.py against its recorded results).
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


def layer_dag(cfg, seq, fused=False):
    """Qwen prefill as the planner sees it (optimize.py:59-142).

    ``cfg`` holds the manifest config keys (hidden_size, intermediate_size,
    num_hidden_layers, num_attention_heads, num_key_value_heads, vocab_size,
    head_dim, qk_norm).  GEMMs run on engine ``aic``, vector ops on ``aiv``
    and attention on ``aicore`` (it occupies both).

    ``fused=False`` is the reference's program: separate q/k/v projections,
    RoPE, gate and up projections, SiLU and Mul.  ``fused=True`` is the
    program this runtime launches: one QKV projection (its epilogue adds the
    bias and, without q/k norms, applies RoPE), one gate/up projection whose
    epilogue writes SwiGLU, then down.
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
        if fused:
            mm(p + "qkv", seq, H, (HQ + 2 * HKV) * D)
            dep(p + "ln1", p + "qkv")
            asrc = p + "qkv"
            if qk:
                node(p + "qk_norm", "rmsnorm", "aiv", rows=seq * HQ, cols=D)
                dep(p + "qkv", p + "qk_norm")
                node(p + "rope", "rope", "aiv", rows=seq, cols=HQ * D)
                dep(p + "qk_norm", p + "rope")
                asrc = p + "rope"
            node(p + "attn", "attention", "aicore", batch=1, q_heads=HQ,
                 kv_heads=HKV, seq=seq, head_dim=D)
            dep(asrc, p + "attn")
        else:
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
        if fused:
            mm(p + "gate_up", seq, H, 2 * I)
            dep(p + "addnorm1", p + "gate_up")
            mm(p + "down", seq, I, H)
            dep(p + "gate_up", p + "down")
        else:
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
_RC_KEY = re.compile(r"([a-z_0-9]+)\|(\d+)x(\d+)$")

# Fallback constants of a cost file without them, and of the roofline price of
# an unmeasured GEMM (the reference's planner2.py:54-123 uses the same values;
# the recorded plans depend on them).
_TABLE_DEFAULTS = (("launch_us", 8.0), ("traffic_gbps", 600.0), ("l2_mb", 32.0), ("event_us", 20.0))
_ROOFLINE_FLOPS = 250e12           # flop/s of an unmeasured GEMM
_AICPU_US_PER_ELEMENT = 2.2e-3     # host-side scalar op
_COLUMN_SPLIT_US_PER_MB = 1.6      # re-assembly of a column-split output


class Costs:
    """What an op costs unsplit, and what running it as k tiles adds.

    ``table`` has the layout of a cost file: ``full`` {shape_key: us} plus
    the scalars ``launch_us``, ``traffic_gbps``, ``l2_mb``, ``event_us``.
    ``curves`` maps shape keys to measured split curves
    ``{"base_best_us", "fit": {"slope_us_per_tile", "intercept_us"}}``.

    An unsplit cost is resolved in order: the measured entry; for a GEMM, the
    first measured GEMM with the same K and N scaled by M; for a row op, the
    first measured entry of the op with the same columns scaled by rows; else
    a roofline price (the reference's resolution, planner2.py:86-123).
    """

    def __init__(self, table, curves=None):
        self.data = table
        self.full = dict(table.get("full", {}))
        scalars = {name: float(table.get(name, default)) for name, default in _TABLE_DEFAULTS}
        self.launch = scalars["launch_us"]
        self.bw = scalars["traffic_gbps"] * 1e9
        self.l2 = scalars["l2_mb"] * 1024 * 1024
        self.event = scalars["event_us"]
        self.curves = dict(curves or {})
        self._resolved = {}
        self._taxes = {}

    @classmethod
    def from_files(cls, path, curves_path=None):
        """Cost file plus an optional curve file (``{"cases": [...]}``)."""
        table = json.loads(Path(path).read_text(encoding="utf-8"))
        curves = {}
        if curves_path and Path(curves_path).exists():
            for case in json.loads(Path(curves_path).read_text(encoding="utf-8")).get("cases", []):
                key = cls.curve_key(case)
                if key:
                    curves[key] = case
        return cls(table, curves)

    @staticmethod
    def curve_key(case):
        op, shape = case.get("op"), case.get("shape") or {}
        if op in ("matmul", "attention"):
            return shape_key({"op": op, "shape": shape})
        if shape.get("rows") and shape.get("cols"):
            return "%s|%dx%d" % (op, shape["rows"], shape["cols"])
        return None

    # -- unsplit cost --------------------------------------------------------
    def _scaled_neighbour(self, node):
        """A measured entry of the same inner shape, scaled along the rows."""
        shape, op = node["shape"], node["op"]
        for key, us in self.full.items():
            if op == "matmul":
                m = _MM_KEY.match(key)
                if m and (int(m.group(2)), int(m.group(3))) == (shape["K"], shape["N"]):
                    return float(us) * shape["M"] / int(m.group(1))
            else:
                m = _RC_KEY.match(key)
                if m and m.group(1) == op and int(m.group(3)) == shape.get("cols", 0):
                    return float(us) * shape.get("rows", 0) / max(int(m.group(2)), 1)
        return None

    def _roofline(self, node):
        hbm_us = shape_bytes(node) / self.bw * 1e6
        if node["op"] != "matmul":
            return max(hbm_us, 1.0)
        s = node["shape"]
        return max(2.0 * s["M"] * s["K"] * s["N"] / _ROOFLINE_FLOPS * 1e6, hbm_us)

    def base(self, node):
        key = shape_key(node)
        if key not in self._resolved:
            if key in self.full:
                self._resolved[key] = float(self.full[key])
            elif node["op"] == "custom_aicpu_scale":
                s = node["shape"]
                return max(1.0, s.get("rows", 0) * s.get("cols", 0) * _AICPU_US_PER_ELEMENT)
            else:
                scaled = self._scaled_neighbour(node)
                self._resolved[key] = scaled if scaled is not None else self._roofline(node)
        return self._resolved[key]

    # -- the tax of k tiles --------------------------------------------------
    def _weight_reread_us(self, node, k):
        """A row-split GEMM re-reads its weight once per extra tile when the
        weight does not stay in the last-level cache."""
        if node["op"] != "matmul":
            return 0.0
        s = node["shape"]
        weight = s["K"] * s["N"] * 2
        return (k - 1) * weight / self.bw * 1e6 if weight > self.l2 else 0.0

    def split_tax(self, node, strategy, k):
        """Extra time of k tiles over the unsplit op: the measured curve's
        excess over the unsplit time where there is one, else a launch per
        tile (plus the weight re-reads of a row split, or the output
        re-assembly of a column split); always one cross-stream sync per
        tile."""
        if k <= 1:
            return 0.0
        memo = (shape_key(node), strategy, k)
        if memo in self._taxes:
            return self._taxes[memo]
        curve = self.curves.get(shape_key(node))
        if curve and curve.get("fit"):
            fit = curve["fit"]
            work = max(0.0, float(fit["slope_us_per_tile"]) * (k - 1) + float(fit["intercept_us"])
                       - float(curve["base_best_us"]))
        elif strategy == "head":
            work = k * self.launch
        elif strategy in ("col", "m2d"):
            s = node["shape"]
            work = k * self.launch + _COLUMN_SPLIT_US_PER_MB * s["M"] * s["N"] * 2 / (1024.0 * 1024.0)
        else:
            work = k * self.launch + self._weight_reread_us(node, k)
        self._taxes[memo] = work + k * self.event
        return self._taxes[memo]

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
    """Dependency levels: level r holds the nodes whose last producer is on
    level r-1, each level in node order. Raises on a cycle."""
    position = {n["name"]: i for i, n in enumerate(nodes)}
    producers_left = {n["name"]: 0 for n in nodes}
    consumers = defaultdict(list)
    for e in edges:
        producers_left[e["dst"]] += 1
        consumers[e["src"]].append(e["dst"])
    level = [n["name"] for n in nodes if producers_left[n["name"]] == 0]
    rounds, node_round = [], {}
    while level:
        for name in level:
            node_round[name] = len(rounds)
        rounds.append(level)
        unlocked = set()
        for name in level:
            for c in consumers[name]:
                producers_left[c] -= 1
                if producers_left[c] == 0:
                    unlocked.add(c)
        level = sorted(unlocked, key=position.__getitem__)
    if len(node_round) < len(nodes):
        raise ValueError("graph cycle")
    return rounds, node_round


# engines a task occupies: attention ("aicore") holds both the matrix and the
# vector engine
_HOLDS = {"aicore": ("aic", "aiv")}


def _resources(engine):
    return _HOLDS.get(engine, (engine,))


def row_ranges(total, k):
    """k proportional row ranges; the boundaries round half to even (Python's
    round, as the reference's planner2.py:208-210)."""
    cuts = [round(i * total / k) for i in range(k + 1)]
    return list(zip(cuts[:-1], cuts[1:]))


def _meeting(src_ranges, dst_ranges):
    """Consumer range j -> the producer ranges it meets."""
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
    """Consumer tile -> the producer tiles it reads.

    Four cases, in this order (the reference's mapping, planner2.py:213-266):
    a row-split consumer that reads fewer rows than the producer writes (a
    partial collective) meets the head of the producer's range; equal k maps
    tile to tile; splits along different axes need every producer tile;
    otherwise the proportional row ranges decide."""
    ks, kd = sp_src["k"], sp_dst["k"]
    read = dst["shape"].get("rows") or dst["shape"].get("M") or 0
    written = src["shape"].get("M") or src["shape"].get("rows") or 0
    if read and written and read < written and sp_dst["strategy"] == "row":
        extent = _split_extent(src, sp_src["strategy"]) or written
        return _meeting(row_ranges(extent, ks), row_ranges(min(extent, read), kd))
    if ks == kd:
        return {j: [j] for j in range(kd)}
    every = {j: list(range(ks)) for j in range(kd)}
    if sp_src["strategy"] != sp_dst["strategy"]:
        return every
    extent = _split_extent(src, sp_src["strategy"])
    return _meeting(row_ranges(extent, ks), row_ranges(extent, kd)) if extent else every


class _Task:
    """One tile of a node on its engine."""
    __slots__ = ("name", "node", "tile", "parts", "dur", "strategy", "engine", "round", "order", "deps",
                 "data_preds", "ready", "start", "end", "free_at")

    def __init__(self, name, node, tile, parts, dur, strategy, rnd, order):
        self.name, self.node, self.tile, self.parts = name, node, tile, parts
        self.dur, self.strategy, self.engine = dur, strategy, node["engine"]
        self.round, self.order = rnd, order
        self.deps, self.data_preds = set(), []
        self.ready = self.start = self.end = self.free_at = 0.0


def _expand(nodes, costs, splits, node_round, order):
    """Node -> its tile tasks, each tile after the previous one."""
    parts = {}
    for n in nodes:
        name = n["name"]
        sp = splits.get(name)
        k = int(sp.get("k", 1)) if sp else 1
        if k <= 1:
            tiles = [_Task(name, n, 0, 1, costs.base(n), "none", node_round[name], order[name])]
        else:
            strategy = sp.get("strategy", "row")
            each = costs.split_total(n, strategy, k) / k
            tiles = [_Task("%s#%d" % (name, i), n, i, k, each, strategy, node_round[name], order[name])
                     for i in range(k)]
        for prev, t in zip(tiles, tiles[1:]):
            t.deps.add(prev.name)
        parts[name] = tiles
    return parts


def _wire(graph, splits, parts):
    """Data edges between tiles: which producer tiles each consumer tile
    reads (an unsplit side reads or feeds every tile)."""
    by_name = {n["name"]: n for n in graph["nodes"]}
    for e in graph["edges"]:
        sp_s, sp_d = splits.get(e["src"]), splits.get(e["dst"])
        ks = int(sp_s.get("k", 1)) if sp_s else 1
        kd = int(sp_d.get("k", 1)) if sp_d else 1
        src_tiles, dst_tiles = parts[e["src"]], parts[e["dst"]]
        if ks <= 1:
            need = {j: [0] for j in range(len(dst_tiles))}
        else:
            consumer = sp_d if kd > 1 else {"strategy": sp_s.get("strategy", "row"), "k": 1}
            need = tile_overlap(by_name[e["src"]], by_name[e["dst"]], sp_s, consumer)
        for j, t in enumerate(dst_tiles):
            for i in need.get(j, range(ks)):
                t.deps.add(src_tiles[i].name)
                t.data_preds.append(src_tiles[i].name)


def _list_schedule(tasks):
    """Run the tasks on their engines: of the tasks whose dependencies are
    done, the one that can start earliest goes next, ties broken by
    (dependency level, tile, node order). A heap holds the ready tasks keyed
    by their start as of the push; engine free times only grow, so a popped
    key that is out of date is re-keyed and pushed back, and the first key
    found current is the minimum."""
    free = defaultdict(float)
    pending = {t.name: len(t.deps) for t in tasks.values()}
    consumers = defaultdict(list)
    for t in tasks.values():
        for d in t.deps:
            consumers[d].append(t.name)

    def key(t):
        return (max(max(free[r] for r in _resources(t.engine)), t.ready), t.round, t.tile, t.order)

    heap = [(key(t), t.name) for t in tasks.values() if pending[t.name] == 0]
    heapq.heapify(heap)
    done = []
    while heap:
        k, name = heapq.heappop(heap)
        t = tasks[name]
        now = key(t)
        if now != k:
            heapq.heappush(heap, (now, name))
            continue
        t.free_at = max(free[r] for r in _resources(t.engine))
        t.start, t.end = now[0], now[0] + t.dur
        for r in _resources(t.engine):
            free[r] = t.end
        done.append(t)
        for c in consumers[name]:
            pending[c] -= 1
            if pending[c] == 0:
                nxt = tasks[c]
                nxt.ready = max(tasks[d].end for d in nxt.deps)
                heapq.heappush(heap, (key(nxt), c))
    if len(done) < len(tasks):
        raise ValueError("task graph cycle at %s" % [n for n in tasks if pending[n]][:5])
    return done


def _record(t, tasks):
    """The schedule entry of a placed task; `critical` is the data producer
    that finished last (the first listed of equal ones)."""
    critical, critical_end = None, 0.0
    for d in dict.fromkeys(t.data_preds):
        if critical is None or tasks[d].end > critical_end:
            critical, critical_end = d, tasks[d].end
    return {"name": t.name, "node": t.node["name"], "tile": t.tile, "parts": t.parts, "engine": t.engine,
            "round": t.round, "start": t.start, "end": t.end, "dur": t.dur, "ready": t.ready,
            "engine_free": t.free_at, "critical": critical, "critical_end": critical_end,
            "deps": sorted(t.deps), "data_preds": sorted(set(t.data_preds))}


def simulate(graph, costs, splits=None, topo=None):
    """List-schedule the DAG with the given splits (the reference's
    simulator, planner2.py:269-382, as an event loop over a heap).

    A split node becomes k consecutive tile tasks on its engine; a consumer
    tile waits for the producer tiles ``tile_overlap`` names. Returns the
    makespan, every task's placement (sorted by start, engine, name) and the
    dependency levels."""
    splits = splits or {}
    nodes = graph["nodes"]
    if topo is None:
        rounds, node_round = topo_rounds(nodes, graph["edges"])
        order = {n["name"]: i for i, n in enumerate(nodes)}
    else:
        rounds, node_round, order = topo
    parts = _expand(nodes, costs, splits, node_round, order)
    _wire(graph, splits, parts)
    tasks = {t.name: t for tiles in parts.values() for t in tiles}
    placed = _list_schedule(tasks)
    schedule = sorted((_record(t, tasks) for t in placed), key=lambda x: (x["start"], x["engine"], x["name"]))
    return {"makespan_us": max((x["end"] for x in schedule), default=0.0), "tasks": schedule,
            "splits": copy.deepcopy(splits), "rounds": rounds}


def bubbles(sched):
    """Idle time an engine spent waiting for a data producer, one entry per
    task that found its engine free before its inputs were ready; largest
    wait first (engines in order of first appearance, then start time)."""
    lanes = defaultdict(list)
    for t in sched["tasks"]:
        lanes[t["engine"]].append(t)
    found = []
    for engine, lane in lanes.items():
        busy_until = 0.0
        for t in sorted(lane, key=lambda x: x["start"]):
            wait = t["ready"] - t["engine_free"]
            if wait > 1e-6 and t["critical"]:
                found.append({"engine": engine, "task": t["name"], "node": t["node"], "tile": t["tile"],
                              "round": t["round"], "dep_gap_us": wait, "engine_gap_us": t["start"] - busy_until,
                              "critical": t["critical"], "critical_end": t["critical_end"], "start": t["start"]})
            busy_until = max(busy_until, t["end"])
    found.sort(key=lambda b: -b["dep_gap_us"])
    return found


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
        """Up to `limit` nodes that follow `start` one by one on its engine
        (each the only same-engine consumer of the previous), element-wise
        ops or GEMMs only."""
        engine, chain, cur = self.node[start]["engine"], [], start
        while len(chain) < limit:
            same = [v for v in self.succ.get(cur, []) if self.node[v]["engine"] == engine]
            if len(same) != 1 or not (self.node[same[0]]["op"] in ELEMENTWISE or self.node[same[0]]["op"] == "matmul"):
                break
            cur = same[0]
            chain.append(cur)
        return chain

    def producers(self, dst, fallback):
        return list(self.pred.get(dst, [])) or [fallback]

    def fanout(self, producers):
        return [c for p in producers for c in self.succ.get(p, [])]


# tile counts the search tries (the reference's sets, planner2.py:447-459):
# attention by heads, everything else by rows, GEMM tiles of >= 1024 rows
_HEAD_KS = (2, 4, 7, 8, 14)
_ROW_KS = (2, 4, 8, 16)
_MIN_GEMM_TILE_ROWS = 1024


def candidate_ks(node):
    """Tile counts the search may try for a node."""
    s = node["shape"]
    if node["op"] == "attention":
        heads = int(s.get("q_heads", 0))
        return [k for k in _HEAD_KS if heads and heads % k == 0]
    rows = int(s.get("M") or s.get("rows") or 0)
    ks = [k for k in _ROW_KS if rows and rows % k == 0]
    if node["op"] == "matmul":
        ks = [k for k in ks if rows // k >= _MIN_GEMM_TILE_ROWS]
    return ks


def _strategy(node):
    if node["op"] == "attention":
        return "head"
    if node["op"] == "matmul" or node["op"] in ELEMENTWISE or node["op"] in COMM:
        return "row"
    return None


class _Option:
    """One way to remove a bubble: a full split set and its schedule."""
    __slots__ = ("gain", "ks", "chain", "splits", "sched")

    def __init__(self, gain, ks, chain, splits, sched):
        self.gain, self.ks, self.chain, self.splits, self.sched = gain, ks, chain, splits, sched

    @property
    def label(self):
        return "%d/%d" % self.ks


class _SplitSearch:
    """Bubble-driven search for row splits (the reference's greedy planner,
    planner2.py:587-680, whose recorded decisions it reproduces).

    Each round looks at the current schedule's dependency bubbles between
    engines (one per distinct op/shape/gap signature, at most 8), prices up
    to 12 split options per bubble by simulation (producer/consumer tile
    counts, with and without the consumer's chain), and accepts the best
    option, or the best union of two options of different bubbles when that
    gains more. It stops when nothing gains `min_gain_us`."""

    def __init__(self, graph, costs, min_gain_us, top_options):
        self.g = _Graph(graph)
        self.graph, self.costs = graph, costs
        self.min_gain, self.top = min_gain_us, top_options
        rounds, node_round = topo_rounds(graph["nodes"], graph["edges"])
        self.topo = (rounds, node_round, {n["name"]: i for i, n in enumerate(graph["nodes"])})
        self.tried = set()

    def run(self, splits, topo=True):
        return simulate(self.graph, self.costs, splits, topo=self.topo if topo else None)

    def bubbles_to_try(self, sched):
        seen, out = set(), []
        for b in bubbles(sched):
            if not self.g.cross_engine(b["critical"], b["node"]):
                continue
            if b["dep_gap_us"] < self.min_gain or (b["node"], b["critical"]) in self.tried:
                continue
            src, dst = self.g.node[_base_name(b["critical"])], self.g.node[b["node"]]
            sig = (src["op"], dst["op"], json.dumps(src.get("shape", {}), sort_keys=True),
                   json.dumps(dst.get("shape", {}), sort_keys=True), round(b["dep_gap_us"], 1))
            if sig not in seen:
                seen.add(sig)
                out.append(b)
        return out[:8]

    def splits_for(self, base, src, dst, kp, kc, chain):
        """Every producer of dst at kp; dst, the producers' other consumers and
        the optional chain at kc. None when a node cannot take its k."""
        trial = copy.deepcopy(base)
        producers = self.g.producers(dst, src)
        for name in dict.fromkeys(producers + [dst] + self.g.fanout(producers) + (chain or [])):
            n = self.g.node[name]
            if n["op"] == "custom_aicpu_scale":
                if name in producers:
                    return None
                continue
            k = kp if name in producers else kc
            strategy = _strategy(n)
            if strategy is None or k not in candidate_ks(n):
                return None
            trial[name] = {"strategy": strategy, "k": k}
        return trial

    def options(self, cur, b):
        """Options with a positive gain for bubble b, best first."""
        src, dst = _base_name(b["critical"]), b["node"]
        if self.g.node[src]["engine"] == self.g.node[dst]["engine"]:
            return []
        producers = self.g.producers(dst, src)
        # the cheapest split of every node involved must cost less than the gap
        floor = 0.0
        for name in dict.fromkeys(producers + [dst] + self.g.fanout(producers)):
            n = self.g.node[name]
            ks = candidate_ks(n)
            if not ks or (n["op"] == "custom_aicpu_scale" and name in producers):
                return []
            floor += self.costs.split_tax(n, "head" if n["op"] == "attention" else "row", min(ks))
        if floor >= b["dep_gap_us"]:
            return []
        chain = self.g.chain_after(dst)
        pairs = sorted({(kp, kc) for kp in candidate_ks(self.g.node[src]) for kc in candidate_ks(self.g.node[dst])},
                       key=lambda x: (x[0] > x[1], x[0], x[1]))[:6]
        found = []
        for kp, kc in pairs:
            for with_chain in (False, True):
                trial = self.splits_for(cur["splits"], src, dst, kp, kc, chain if with_chain else None)
                if not trial:
                    continue
                try:
                    sched = self.run(trial)
                except (ValueError, KeyError):
                    continue
                gain = cur["makespan_us"] - sched["makespan_us"]
                if gain >= self.min_gain:
                    found.append(_Option(gain, (kp, kc), with_chain, trial, sched))
        found.sort(key=lambda o: -o.gain)
        return found

    def best_move(self, cur, per_bubble):
        """The best single option, or a better union of two options of
        different bubbles. Returns ([(bubble, option)...], gain, splits, sched)."""
        shortlist = [(b, o) for b, opts in per_bubble for o in opts[:self.top]]
        b0, o0 = max(shortlist, key=lambda bo: bo[1].gain)  # first of equal gains
        best = ([(b0, o0)], o0.gain, o0.splits, o0.sched)
        ranked = sorted(shortlist, key=lambda bo: -bo[1].gain)[:8]
        for i, (b1, o1) in enumerate(ranked):
            for b2, o2 in ranked[i + 1:]:
                if (b1["node"], b1["critical"]) == (b2["node"], b2["critical"]):
                    continue
                merged = _merge_splits(o1.splits, o2.splits)
                if merged is None:
                    continue
                try:
                    sched = self.run(merged, topo=False)
                except (ValueError, KeyError):
                    continue
                gain = cur["makespan_us"] - sched["makespan_us"]
                if gain > best[1] + 1e-9:
                    best = ([(b1, o1), (b2, o2)], gain, merged, sched)
        return best


def _merge_splits(a, b):
    """Union of two split sets; None when they give a node different splits."""
    out = copy.deepcopy(a)
    for name, spec in b.items():
        if out.setdefault(name, dict(spec)) != spec:
            return None
    return out


def _decision_record(rnd, b, options, accepted):
    top = options[0] if options else None
    return {"round": rnd, "consumer": b["node"], "engine": b["engine"],
            "critical_edge": "%s -> %s" % (b["critical"], b["node"]), "dep_gap_us": b["dep_gap_us"],
            "k": top.label if top else None, "split_consumer_chain": top.chain if top else False,
            "predicted_gain_us": top.gain if top else 0.0,
            "alternatives": [{"k": o.label, "gain_us": o.gain, "split_chain": o.chain} for o in options],
            "accepted": accepted}


def greedy_plan(graph, costs, max_rounds=40, min_gain_us=1.0, top_options=3):
    """Bubble-driven split search (see _SplitSearch).

    Returns (splits, schedule, history, base_makespan_us, decisions)."""
    search = _SplitSearch(graph, costs, min_gain_us, top_options)
    splits = {}
    cur = search.run(splits)
    base = cur["makespan_us"]
    history, decisions = [], []
    for rnd in range(max_rounds):
        cands = search.bubbles_to_try(cur)
        per_bubble = [(b, opts) for b, opts in ((b, search.options(cur, b)) for b in cands) if opts]
        if not per_bubble:
            break
        chosen, gain, trial, sched = search.best_move(cur, per_bubble)
        picked = {id(b) for b, _ in chosen}
        decisions += [_decision_record(rnd, b, opts, id(b) in picked) for b, opts in per_bubble]
        for b, o in chosen:
            search.tried.update((name, b["critical"]) for name in o.splits)
        history.append({"round": rnd, "gain_us": gain,
                        "k": ", ".join("k=" + o.label + ("+chain" if o.chain else "") for _, o in chosen),
                        "split_chain": any(o.chain for _, o in chosen), "splits": copy.deepcopy(trial),
                        "bubble": chosen[0][0],
                        "bubbles": [{"consumer": b["node"], "critical": b["critical"]} for b, _ in chosen],
                        "makespan_us": sched["makespan_us"]})
        splits, cur = trial, sched
    return splits, cur, history, base, decisions


# ------------------------------------------------- profile -> planner ----

PROFILE_OPS = ("embedding", "rmsnorm", "add", "add_rmsnorm", "rope",
               "matmul_q", "matmul_k", "matmul_v", "attention", "matmul_o",
               "matmul_gate", "matmul_up", "silu", "mul", "matmul_down",
               "matmul_lm")


# the fused projections of ``layer_dag(..., fused=True)`` (QKV with its bias /
# RoPE epilogue, gate/up with its SwiGLU epilogue), timed as plain GEMMs
FUSED_PROFILE_OPS = ("matmul_qkv", "matmul_gate_up")


# the relay split's flag edges, each timed as one relayed launch (the GEMM
# releasing k row tiles, its own workgroups running Add+RMSNorm on each) next
# to the same work unrelayed (the GEMM, then the Add+RMSNorm kernel)
RELAY_EDGES = {"o": ("matmul_o_add_rmsnorm_relay", "matmul_o"),
               "down": ("matmul_down_add_rmsnorm_relay", "matmul_down")}
RELAY_PROFILE_OPS = tuple(v[0] for v in RELAY_EDGES.values()) + ("matmul_gate_up", "swiglu")


def relay_edges(table, k, launch_us=0.0):
    """The relay split's flag edges that pay at k tiles on a measured table.

    An edge is taken only where its relayed launch beats the unrelayed pair
    (the GEMM, the Add+RMSNorm kernel and the extra kernel's launch in a
    replayed graph), as the reference's planner keeps a split only where it
    lowers the makespan (planner2.py:581-671). Returns (edges, detail):
    edges in RELAY_EDGES order, detail = {edge: {relay_us, unrelayed_us,
    gain_us}} for every edge the table prices."""
    def col(v, kk):
        return None if v is None else v.get(kk, v.get(str(kk)))

    edges, detail = [], {}
    norm = col(table.get("add_rmsnorm"), 1)
    for name, (relay_op, gemm_op) in RELAY_EDGES.items():
        r, g = col(table.get(relay_op), k), col(table.get(gemm_op), 1)
        if r is None or g is None or norm is None:
            continue
        unrelayed = float(g) + float(norm) + float(launch_us)
        gain = unrelayed - float(r)
        detail[name] = {"relay_us": round(float(r), 3), "unrelayed_us": round(unrelayed, 3),
                        "gain_us": round(gain, 3)}
        if gain > 0:
            edges.append(name)
    return edges, detail


def relay_mode(table, k, launch_us=0.0):
    """kr_qwen_run mode string of the relay split with the edges that pay
    (relay_split:<k>:<edges>; "none" when no edge does)."""
    edges, _ = relay_edges(table, k, launch_us)
    return "relay_split:%d:%s" % (k, "+".join(edges) if edges else "none")


def profile_op(node):
    """``kr_qwen_profile_many`` op name that times a DAG node
    (optimize.py:193-207)."""
    if node["op"] == "matmul":
        tail = node["name"].rsplit(".", 1)[-1]
        if tail in ("q", "k", "v", "o", "gate", "up", "down", "qkv", "gate_up"):
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
